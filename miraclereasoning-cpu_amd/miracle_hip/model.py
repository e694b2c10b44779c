"""Single-sequence inference on one MI355X with the step-level HIP engine.

Same public API, validation order and error behaviour as the reference engine
(miracle_reasoning/model.py:36-357): ``from_pretrained``, ``prefill``,
``decode``, ``generate``, ``reset``, ``position``.  The whole token step -- all
layers, caches, routing -- runs in the HIP library on device-resident state;
Python only validates inputs and moves token ids and (when asked for) logits.
"""
from __future__ import annotations

import ctypes as C
import json
import math
from pathlib import Path

import numpy as np

from .config import ModelConfig
from . import hip as _hip
from .hip import HIPBackend, HIPError, MR_ERR_NONFINITE, ModelDesc, _check, _DTYPE_TAG
from .weights import BF16Array, SafeTensors, adapt_weights, expected_shapes, storage_of

FAMILY_CODE = {"flashnano-1.5": 0, "flashnano-1.6": 1, "flashnano-1.7": 2, "flashlite-2.0": 3,
               "flashlighting-2.0": 4, "heavy-medium-2.0": 5}

# Canonical weight names -> library weight kinds (miracle_hip.h MR_W_*).
_KIND = {"embed": 0, "output": 1, "norm": 2, "a_norm": 3, "f_norm": 4, "q": 5, "k": 6, "v": 7, "o": 8,
         "q_norm": 9, "k_norm": 10, "gate": 11, "up": 12, "down": 13, "latent": 14, "latent_norm": 15,
         "kv_up": 16, "attention_gate": 17, "ffn_gate": 18, "cbr": 19, "router.coarse.weight": 20,
         "router.coarse.bias": 21, "router.fine.weight": 22, "router.fine.bias": 23, "router.group_bias": 24,
         "router.expert_bias": 25}
_SHARED_KIND = {"gate": 26, "up": 27, "down": 28}

FWD_RETURN_ALL, FWD_BATCHED = 1, 2


def weight_target(name):
    """(kind, layer, expert) of a canonical weight name."""
    if not name.startswith("layers."):
        return _KIND[name], -1, -1
    _, layer, rest = name.split(".", 2)
    layer = int(layer)
    if rest.startswith("ffn."):
        return _KIND[rest[4:]], layer, -1
    if rest.startswith("experts."):
        _, e, part = rest.split(".", 2)
        return _KIND[part], layer, int(e)
    if rest.startswith("shared."):
        _, e, part = rest.split(".", 2)
        return _SHARED_KIND[part], layer, int(e)
    return _KIND[rest], layer, -1


def model_desc(config, context_length):
    c, s = config, config.source
    long = s.get("long_context", {}) if c.family == "heavy-medium-2.0" else {}
    mask = 0
    for i in c.global_layers:
        mask |= 1 << (i - 1)
    return ModelDesc(
        family=FAMILY_CODE[c.family], vocab_size=c.vocab_size, hidden_size=c.hidden_size, layers=c.layers,
        query_heads=c.query_heads, kv_heads=c.kv_heads, global_kv_heads=c.global_kv_heads, head_dim=c.head_dim,
        ffn_dim=c.ffn_dim, context_length=context_length, window=c.window or 0,
        tie_embeddings=int(bool(c.tie_embeddings)), qk_norm=int(bool(c.qk_norm)),
        split_half_rope=int(c.split_half_rope), latent_dim=c.latent_dim, memory_slots=c.memory_slots,
        cbr_chunk_size=c.cbr_chunk_size, cbr_slots=c.cbr_slots, inner_loop_steps=c.inner_loop_steps,
        norm_eps=c.norm_eps, cbr_norm_eps=c.cbr_norm_eps, residual_scale=c.residual_scale,
        routed_experts=s.get("routed_experts", 0), router_groups=s.get("router_groups", 0),
        router_top_k_min=s.get("router_top_k_min", 0), router_top_k_max=s.get("router_top_k_max", 0),
        shared_experts=s.get("shared_experts", 0), global_block_size=long.get("global_block_size", 0),
        global_slots=long.get("global_slots", 0), router_temperature=max(s.get("router_temperature", 1.0), 1e-4),
        alibi_slope_scale=long.get("alibi_slope_scale", 0.015),
        global_layer_mask_lo=mask & ((1 << 64) - 1), global_layer_mask_hi=mask >> 64,
        heavy_step_scale=c.residual_scale / math.sqrt(max(c.inner_loop_steps, 1)),
        heavy_shared_scale=c.residual_scale / max(s.get("shared_experts", 0), 1),
        block_slope=long.get("alibi_slope_scale", 0.015) / math.sqrt(c.head_dim))


class ResidentWeights:
    """The ``weight_cache`` attribute of the reference's engine (WeightCache,
    weights.py:258-297), for code that reads it.  The reference stages FP32
    copies of weights through a cache of at most ``budget`` bytes; here every
    weight is uploaded once, in its stored dtype, into the model's own HBM
    buffers, so the cache holds nothing (``used`` is 0) and ``resident`` counts
    the weight bytes in HBM.  The budget is validated as the reference does."""

    def __init__(self, config, weights, budget_bytes):
        if type(budget_bytes) is not int or budget_bytes < 4096:
            raise ValueError("weight_cache_bytes must be an integer >= 4096")
        self.budget, self.used, self.resident = budget_bytes, 0, 0
        for name, shape in expected_shapes(config).items():
            a = weights[name]
            narrow = len(shape) == 2 and (isinstance(a, BF16Array) or getattr(a, "dtype", None) == np.float16)
            self.resident += math.prod(shape) * (2 if narrow else 4)


class Engine:
    """Owns one mr_model: weights in HBM, caches, step graphs."""

    def __init__(self, backend, config, weights, context_length):
        self.backend, self.lib, self.config = backend, backend.lib, config
        if backend.ctx is None:
            raise HIPError("create model failed: the backend is closed")
        handle = C.c_void_p()
        desc = model_desc(config, context_length)
        _check(self.lib.mr_model_create(backend.ctx, C.byref(desc), C.byref(handle)), "create model")
        self.handle = handle
        backend._engines.add(self)
        for name, shape in expected_shapes(config).items():
            kind, layer, expert = weight_target(name)
            array, tag = storage_of(weights[name])
            if len(shape) == 1:
                array, tag = np.ascontiguousarray(np.asarray(weights[name], dtype=np.float32)), "f32"
            rows, cols = (shape[0], 1) if len(shape) == 1 else shape
            _check(self.lib.mr_model_set_weight(handle, kind, layer, expert, array.ctypes.data, _DTYPE_TAG[tag],
                                                rows, cols), f"upload weight {name}")
        freq = np.ascontiguousarray(config.inverse_frequencies(), dtype=np.float32)
        _check(self.lib.mr_model_set_rope(handle, freq.ctypes.data, freq.size), "upload rope table")
        _check(self.lib.mr_model_finalize(handle), "finalize model")

    def close(self):
        """Free the model's device memory (weights, caches, graphs) now."""
        if getattr(self, "handle", None):
            self.lib.mr_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        if not _hip._shut_down:
            self.close()

    def reset(self):
        _check(self.lib.mr_model_reset(self.handle), "reset")

    def debug_step_timeout(self):
        """Test hook: the next persistent step reports a wait timeout."""
        _check(self.lib.mr_debug_step_timeout(self.handle), "arm step timeout")

    def forward(self, ids, flags, want_logits=True):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        rows = len(ids) if flags & FWD_RETURN_ALL else 1
        out = np.empty((rows, self.config.vocab_size), np.float32) if want_logits else None
        _check(self.lib.mr_model_forward(self.handle, ids.ctypes.data, len(ids), flags,
                                         out.ctypes.data if out is not None else None), "forward")
        return out

    def generate_greedy(self, max_new, eos):
        tokens = np.empty(max(max_new, 1), np.int32)
        produced = C.c_int()
        code = self.lib.mr_model_generate_greedy(self.handle, max_new, eos, tokens.ctypes.data, C.byref(produced))
        if code == MR_ERR_NONFINITE:
            raise FloatingPointError("non-finite output logits")
        _check(code, "generate")
        return [int(t) for t in tokens[:produced.value]]

    KERNELS = {"qkv": 0, "attention": 1, "o": 2, "gate_up": 3, "down": 4, "head": 5}

    def time_kernel(self, which, reps=3):
        """Average device milliseconds of one launch of a step kernel (HIP events)."""
        ms = C.c_float()
        _check(self.lib.mr_model_time_kernel(self.handle, self.KERNELS[which], reps, C.byref(ms)), "time kernel")
        return ms.value

    def position(self):
        pos = C.c_int()
        _check(self.lib.mr_model_position(self.handle, C.byref(pos)), "position")
        return pos.value

    STEP_MODES = {"persistent": 0, "graph": 1, "eager": 2}

    def set_step_mode(self, mode):
        """"persistent" (one kernel per token step), "graph" (per-layer kernels
        replayed from a hipGraph) or "eager" (per-layer kernels, no graph)."""
        _check(self.lib.mr_model_set_step_mode(self.handle, self.STEP_MODES[mode]), "set_step_mode")

    def step_mode(self):
        mode = C.c_int()
        _check(self.lib.mr_model_get_step_mode(self.handle, C.byref(mode)), "get_step_mode")
        return {v: k for k, v in self.STEP_MODES.items()}[mode.value]

    TRACE_FIELDS = 5

    def trace_step(self):
        """Per-phase, per-workgroup record of one persistent greedy decode step:
        array [phases, grid, 5] of (phase entry, input staged, outputs stored
        by the last stream wave, outputs stored by the first stream wave) in µs
        relative to the step start (NaN where not recorded), and a fifth field
        unused there.  In attention phases the fields are (entry, the unit's
        Q/K/V cells staged, the workgroup's end of the phase (after its merge,
        for a merging unit), the unit's partial stored, a merging unit's first
        partial cells seen)."""
        cap = 8 * 1024 * 1024
        buf = np.zeros(cap, np.uint64)
        phases, grid = C.c_int(), C.c_int()
        _check(self.lib.mr_model_trace_step(self.handle, buf.ctypes.data, cap, C.byref(phases), C.byref(grid)),
               "trace step")
        n = self.TRACE_FIELDS
        t = buf[:phases.value * grid.value * n].reshape(phases.value, grid.value, n).astype(np.int64)
        t0 = t[0, :, 0].min()
        return np.where(t > 0, (t - t0) / 100.0, np.nan)   # 100 MHz clock -> µs

    def choices(self):
        """Routing decisions of every position so far (heavy-medium-2.0):
        array [positions, layers, inner_loop_steps, record] of int32; a record
        is (width, experts..., per query head its chosen blocks...), -1 padded."""
        c = self.config
        kmax = c.source["router_top_k_max"]
        rec = 1 + kmax + c.query_heads * c.source["long_context"]["global_slots"]
        pos = self.position()
        buf = np.zeros(max(pos, 1) * c.layers * c.inner_loop_steps * rec, np.int32)
        per = C.c_int()
        _check(self.lib.mr_model_choices(self.handle, buf.ctypes.data, buf.size, C.byref(per)), "read choices")
        return buf[:pos * per.value].reshape(pos, c.layers, c.inner_loop_steps, rec)

    def last_decode_ms(self):
        ms = C.c_float()
        _check(self.lib.mr_model_last_decode_ms(self.handle, C.byref(ms)), "last_decode_ms")
        return ms.value


class MiracleModel:
    """FP32-arithmetic next-token engine for six Miracle architectures on MI355X.

    ``prefill_mode="exact"`` (default) appends a prompt token by token through
    the decode step, so ``decode`` and ``prefill`` agree bit for bit as in the
    reference (tests/test_inference.py:63-64 of the reference);
    ``"batched"`` runs prompts of every family through whole-chunk kernels
    (MFMA projections, windowed attention with the relay rows', the latent
    memory's and the block selection's per-position semantics, grouped expert
    GEMMs), equal to the token loop within FP32 rounding (routing near-ties
    aside); single tokens and geometries outside the kernels' widths keep the
    token loop.
    ``weight_cache_bytes`` is accepted and validated for compatibility: every
    weight stays resident in HBM in its stored dtype, so no cache is needed.
    """

    def __init__(self, config, weights, *, backend=None, context_length=None,
                 weight_cache_bytes=256 * 1024 * 1024, prefill_mode="exact"):
        self.config = config
        if context_length is None:
            context_length = min(2048, config.max_positions)
        if type(context_length) is not int or not 0 < context_length <= config.max_positions:
            raise ValueError(f"context_length must be in [1, {config.max_positions}]")
        if prefill_mode not in ("exact", "batched"):
            raise ValueError("prefill_mode must be 'exact' or 'batched'")
        # Validate the full checkpoint before any device allocation (model.py:50-51).
        self.weights = adapt_weights(config, weights)
        self.backend = backend if backend is not None else HIPBackend()
        self.context_length = context_length
        self.weight_cache = ResidentWeights(config, self.weights, weight_cache_bytes)   # model.py:54
        self.weight_cache_bytes = weight_cache_bytes
        self.prefill_mode = prefill_mode
        self.engine = Engine(self.backend, config, self.weights, context_length)
        self.reset()

    def close(self):
        """Free this model's device memory now (it is also freed at exit)."""
        self.engine.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @classmethod
    def from_pretrained(cls, directory, *, family=None, **kwargs):
        """Load ``config.json`` + ``model.safetensors`` / ``model.npz`` / sharded
        index (reference: model.py:58-72)."""
        directory = Path(directory)
        config = ModelConfig.from_dict(json.loads((directory / "config.json").read_text(encoding="utf-8")), family)
        if (directory / "model.safetensors").is_file():
            weights = SafeTensors(directory / "model.safetensors")
        elif (directory / "model.npz").is_file():
            weights = np.load(directory / "model.npz", allow_pickle=False)
        elif (directory / "model.safetensors.index.json").is_file():
            from .weights import ShardedSafeTensors
            weights = ShardedSafeTensors(directory / "model.safetensors.index.json")
        else:
            raise ValueError("Expected model.safetensors, a safetensors index, or model.npz; "
                             "use the export command for PyTorch checkpoints")
        return cls(config, weights, **kwargs)

    def reset(self):
        """Start a new sequence; weights and compiled step graphs are kept."""
        self.engine.reset()
        self.position, self._failed = 0, False

    def _tokens(self, ids):
        array = np.asarray(ids)
        if array.ndim != 1 or array.size == 0 or array.dtype.kind not in "iu":
            raise ValueError("input_ids must be a non-empty 1D integer sequence")
        if np.any(array < 0) or np.any(array >= self.config.vocab_size):
            raise ValueError("input token is outside the vocabulary")
        return array

    def _forward(self, tokens, return_all, want_logits=True):
        if self._failed:
            raise RuntimeError("A previous device operation failed; call reset() before reusing this model")
        if self.position + len(tokens) > self.context_length:
            raise ValueError("input would exceed context_length; reset or allocate a larger context")
        flags = (FWD_RETURN_ALL if return_all else 0) | (FWD_BATCHED if self.prefill_mode == "batched" else 0)
        try:
            logits = self.engine.forward(tokens, flags, want_logits)
        except Exception:
            self._failed = True
            raise
        self.position += len(tokens)
        if logits is None:
            return None
        return logits if return_all else logits[0]

    def prefill(self, input_ids, *, return_all=False):
        """Append a prompt, returning [vocab] or, if requested, [tokens, vocab]."""
        return self._forward(self._tokens(input_ids), return_all)

    def decode(self, token_id):
        """Append one token and return next-token logits."""
        return self.prefill([token_id])

    def generate(self, input_ids, *, max_new_tokens=32, temperature=0.0, top_k=0, top_p=1.0, seed=17,
                 eos_token_id=None):
        """Return generated token ids, excluding the prompt and including EOS.

        Greedy decoding (temperature 0) runs on device and reads back only token
        ids; sampling reads the logits and uses the reference's numpy stream."""
        tokens = self._tokens(input_ids)
        if type(max_new_tokens) is not int or max_new_tokens < 0:
            raise ValueError("max_new_tokens must be a non-negative integer")
        if not math.isfinite(temperature) or temperature < 0:
            raise ValueError("temperature must be finite and non-negative")
        if type(top_k) is not int or top_k < 0 or not math.isfinite(top_p) or not 0 < top_p <= 1:
            raise ValueError("top_k must be non-negative and top_p must be in (0,1]")
        eos = self.config.eos_token_id if eos_token_id is None else eos_token_id
        if type(eos) is not int or not 0 <= eos < self.config.vocab_size:
            raise ValueError("eos_token_id is outside vocabulary")
        if len(tokens) + max(0, max_new_tokens - 1) > self.context_length:
            raise ValueError("prompt plus requested generation exceeds context_length")
        self.reset()
        if max_new_tokens == 0:
            return []
        if temperature == 0:
            self._forward(tokens, False, want_logits=False)
            try:
                generated = self.engine.generate_greedy(max_new_tokens, eos)
            except HIPError:
                # A failed decode step poisons the instance, as in prefill; a
                # non-finite check (FloatingPointError) does not (model.py:339-340).
                self._failed = True
                raise
            finally:
                self.position = self.engine.position()
            return generated
        rng, generated = np.random.default_rng(seed), []
        logits = self.prefill(tokens)
        for i in range(max_new_tokens):
            if not np.all(np.isfinite(logits)):
                raise FloatingPointError("non-finite output logits")
            order = np.argsort(-logits, kind="stable")
            if top_k:
                order = order[:top_k]
            scores = logits[order].astype(np.float64) / temperature
            probs = np.exp(scores - scores.max())
            probs /= probs.sum()
            cutoff = min(len(order), int(np.searchsorted(np.cumsum(probs), top_p)) + 1)
            order, probs = order[:cutoff], probs[:cutoff]
            token = int(rng.choice(order, p=probs / probs.sum()))
            generated.append(token)
            if token == eos or i + 1 == max_new_tokens:
                break
            logits = self.decode(token)
        return generated
