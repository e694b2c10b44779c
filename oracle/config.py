"""ORACLE (test infrastructure only): model geometry, RoPE tables, weight shapes.

Restates miracle_reasoning/config.py:83-87 (per-layer KV heads / window),
config.py:155-197 (inverse frequencies) and weights.py:211-245 (the canonical
shape table, whose insertion order fixes the synthetic weight stream).  It
reads bundle-format dicts (``backend_format: 1``, config.py:89-99) only.

Pinned by: golden inverse-frequency tables and shape tables written by
tests/golden/make_golden.py from the reference's own config.py, for every
family and every RoPE scaling branch (tests/test_oracle_model.py), plus
closed forms (theta^(-2i/d) for the unscaled table).
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import numpy as np

DEFAULTS = dict(global_layers=(), global_kv_heads=0, rope_theta=1e6, norm_eps=1e-6, tie_embeddings=True,
                qk_norm=True, residual_scale=1.0, latent_dim=0, memory_slots=0, cbr_chunk_size=0,
                cbr_slots=0, cbr_norm_eps=1e-6, inner_loop_steps=1, eos_token_id=2, source={})


class OracleConfig(SimpleNamespace):
    @classmethod
    def from_bundle(cls, data):
        values = dict(DEFAULTS)
        values.update({k: v for k, v in data.items() if k != "backend_format"})
        values["global_layers"] = tuple(values["global_layers"])
        return cls(**values)

    def kv_heads_of(self, layer):
        if layer + 1 in self.global_layers:
            return self.global_kv_heads or self.kv_heads
        return self.kv_heads

    def window_of(self, layer):
        return None if layer + 1 in self.global_layers else self.window

    @property
    def split_half(self):
        return self.family in ("flashnano-1.7", "flashlighting-2.0")


def inverse_frequencies(cfg):
    d, theta, src = cfg.head_dim, cfg.rope_theta, cfg.source
    e = np.arange(0, d, 2, dtype=np.float32) / d          # float32 exponents 2i/d
    base = np.power(np.float32(theta), -e)
    if cfg.family == "heavy-medium-2.0":
        lf = src["long_context"].get("rope_local_fraction", 0.6)
        first_long = int((d // 2) * lf)
        out = base.copy()
        out[first_long:] = np.power(np.float32(theta * 16), -e[first_long:])
        return out
    if cfg.family == "flashlighting-2.0":
        mode = src.get("rope_scaling_type", "yarn")
        s = src.get("rope_scaling_factor", 8.0)
        if not math.isfinite(s) or s < 1:
            raise ValueError("rope_scaling_factor must be finite and >= 1")
        n0 = src.get("max_position_embeddings", cfg.max_positions)
        if mode in ("none", "native"):
            return base
        if mode == "linear":
            return base / s
        if mode == "dynamic_ntk":
            if d <= 2:
                raise ValueError("dynamic_ntk requires head_dim > 2")
            r = s * src.get("extension_max_position_embeddings", n0) / n0 - (s - 1)
            return np.power(np.float32(theta * max(r, 1) ** (d / (d - 2))), -e)
        if mode == "yarn":
            lo_len = n0 / src.get("rope_beta_fast", 32.0)
            hi_len = n0 / src.get("rope_beta_slow", 1.0)
            if hi_len <= lo_len:
                raise ValueError("YaRN requires beta_fast > beta_slow > 0")
            wavelength = 2 * np.pi / base
            t = np.clip((wavelength - lo_len) / (hi_len - lo_len), 0, 1)
            return base * (1 - t) + (base / s) * t
        raise ValueError(f"Unsupported RoPE scaling: {mode}")
    if cfg.family == "flashnano-1.7" and src.get("rope_scaling"):
        y = src["rope_scaling"]
        if y.get("type") != "yarn":
            raise ValueError("FlashNano 1.7 only supports YaRN rope_scaling")
        s = float(y["factor"])
        if not math.isfinite(s) or s < 1:
            raise ValueError("YaRN factor must be finite and >= 1")
        orig = y["orig_max_position"]

        def dim_for(rot):
            return d * math.log(orig / (rot * 2 * math.pi)) / (2 * math.log(theta))

        a = max(math.floor(dim_for(y["beta_fast"])), 0)
        b = min(math.ceil(dim_for(y["beta_slow"])), d - 1)
        if a == b:
            b += 0.001
        t = np.clip((np.arange(d // 2, dtype=np.float32) - a) / max(b - a, 1e-3), 0, 1)
        return (base / s) * (1 - t) + base * t
    return base


def weight_shapes(cfg):
    """Canonical name -> shape, in the reference's insertion order."""
    h, d, f = cfg.hidden_size, cfg.head_dim, cfg.ffn_dim
    out = [("embed", (cfg.vocab_size, h)), ("norm", (h,))]
    if not cfg.tie_embeddings:
        out.append(("output", (cfg.vocab_size, h)))
    fam = cfg.family
    for i in range(cfg.layers):
        p = f"layers.{i}."
        kvw = cfg.kv_heads_of(i) * d
        out += [(p + "a_norm", (h,)), (p + "q", (cfg.query_heads * d, h)), (p + "o", (h, cfg.query_heads * d))]
        if fam != "flashlighting-2.0":
            out.append((p + "f_norm", (h,)))
        if cfg.latent_dim:
            out.append((p + "latent", (cfg.latent_dim, h)))
        if fam == "heavy-medium-2.0":
            E, G = cfg.source["routed_experts"], cfg.source["router_groups"]
            out += [(p + "kv_up", (2 * kvw, cfg.latent_dim)),
                    (p + "router.coarse.weight", (G, h)), (p + "router.coarse.bias", (G,)),
                    (p + "router.fine.weight", (E, h)), (p + "router.fine.bias", (E,)),
                    (p + "router.group_bias", (G,)), (p + "router.expert_bias", (E,))]
        else:
            inner = cfg.latent_dim or h
            out += [(p + "k", (kvw, inner)), (p + "v", (kvw, inner))]
            if cfg.qk_norm:
                out += [(p + "q_norm", (d,)), (p + "k_norm", (d,))]
        if fam == "flashlighting-2.0":
            out += [(p + "latent_norm", (cfg.latent_dim,)), (p + "attention_gate", (1,)), (p + "ffn_gate", (1,))]
        if fam == "flashnano-1.6":
            out.append((p + "cbr", (cfg.cbr_slots, h)))
        if fam == "heavy-medium-2.0":
            mlps = [f"experts.{e}." for e in range(cfg.source["routed_experts"])]
            mlps += [f"shared.{e}." for e in range(cfg.source["shared_experts"])]
        else:
            mlps = ["ffn."]
        for m in mlps:
            out += [(p + m + "gate", (f, h)), (p + m + "up", (f, h)), (p + m + "down", (h, f))]
    return dict(out)
