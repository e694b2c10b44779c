"""Model geometry for the six Miracle families.

Same fields, defaults, validation and bundle format as the reference's
``ModelConfig`` (miracle_reasoning/config.py:13-197), so a ``config.json``
written by either side loads in the other.  The RoPE inverse-frequency table is
computed on the host once per model, in float32 exactly as the reference does,
and uploaded; the kernels never re-derive it.
"""
from __future__ import annotations

import math
from dataclasses import asdict, dataclass, field

import numpy as np

FAMILIES = ("flashnano-1.5", "flashnano-1.6", "flashnano-1.7", "flashlite-2.0",
            "flashlighting-2.0", "heavy-medium-2.0")

# Families whose RoPE pairs (p, p + d/2) instead of (2p, 2p+1) (model.py:91-93).
SPLIT_HALF_FAMILIES = ("flashnano-1.7", "flashlighting-2.0")

_POSITIVE_INT32 = ("vocab_size", "hidden_size", "layers", "query_heads", "kv_heads",
                   "head_dim", "ffn_dim", "max_positions", "inner_loop_steps")
_POSITIVE_FLOAT = ("rope_theta", "norm_eps", "cbr_norm_eps", "residual_scale")
_NON_NEGATIVE_INT = ("latent_dim", "memory_slots", "cbr_chunk_size", "cbr_slots", "global_kv_heads")


def _is_int(value):
    return type(value) is int


@dataclass(frozen=True)
class ModelConfig:
    """Architecture description (reference: config.py:13-39)."""
    family: str
    vocab_size: int
    hidden_size: int
    layers: int
    query_heads: int
    kv_heads: int
    head_dim: int
    ffn_dim: int
    max_positions: int
    window: int | None
    global_layers: tuple[int, ...] = ()
    global_kv_heads: int = 0
    rope_theta: float = 1_000_000.0
    norm_eps: float = 1e-6
    tie_embeddings: bool = True
    qk_norm: bool = True
    residual_scale: float = 1.0
    latent_dim: int = 0
    memory_slots: int = 0
    cbr_chunk_size: int = 0
    cbr_slots: int = 0
    cbr_norm_eps: float = 1e-6
    inner_loop_steps: int = 1
    eos_token_id: int = 2
    source: dict = field(default_factory=dict)

    def __post_init__(self):
        # Same checks and messages as config.py:41-81.
        if self.family not in FAMILIES:
            raise ValueError(f"Unsupported family {self.family!r}; expected one of {FAMILIES}. "
                             "Miracle Neural and architectures without a specification are excluded.")
        for name in _POSITIVE_INT32:
            value = getattr(self, name)
            if not _is_int(value) or not 0 < value < 2**31:
                raise ValueError(f"{name} must be a positive int32")
        if self.head_dim % 2 or self.query_heads % self.kv_heads:
            raise ValueError("head_dim must be even and query_heads must divide into KV groups")
        if self.family != "heavy-medium-2.0" and self.hidden_size != self.query_heads * self.head_dim:
            raise ValueError("hidden_size must equal query_heads * head_dim")
        if self.window is not None and (not _is_int(self.window) or self.window <= 0):
            raise ValueError("window must be positive or null")
        if self.global_kv_heads and (self.global_kv_heads < self.kv_heads
                                     or self.query_heads % self.global_kv_heads):
            raise ValueError("invalid global KV head count")
        layers = self.global_layers
        if len(set(layers)) != len(layers) or any(not _is_int(i) or not 1 <= i <= self.layers for i in layers):
            raise ValueError("global layers must be unique, 1-based layer indices")
        for name in _POSITIVE_FLOAT:
            value = getattr(self, name)
            if not math.isfinite(value) or value <= 0:
                raise ValueError(f"{name} must be finite and positive")
        for name in _NON_NEGATIVE_INT:
            value = getattr(self, name)
            if not _is_int(value) or value < 0:
                raise ValueError(f"{name} must be a non-negative integer")
        if not 0 <= self.eos_token_id < self.vocab_size:
            raise ValueError("eos_token_id is outside vocabulary")
        if self.family == "flashnano-1.6" and not (self.cbr_chunk_size and self.cbr_slots):
            raise ValueError("FlashNano 1.6 requires CBR chunk size and slots")
        if self.family in ("flashnano-1.5", "flashnano-1.6", "flashnano-1.7", "flashlighting-2.0") \
                and not self.qk_norm:
            raise ValueError(f"{self.family} requires Q/K normalization")
        if self.family in ("flashlighting-2.0", "heavy-medium-2.0") and not self.latent_dim:
            raise ValueError("latent attention requires latent_dim")
        if self.family == "heavy-medium-2.0":
            s = self.source
            if not 1 <= s["router_top_k_min"] <= s["router_top_k_max"] <= s["routed_experts"]:
                raise ValueError("invalid router top-k")
            if s["shared_experts"] < 0 or s["router_groups"] < 1:
                raise ValueError("invalid expert/group count")
            long = s["long_context"]
            if long["global_block_size"] <= 0 or long["global_slots"] < 0:
                raise ValueError("invalid sparse attention block geometry")

    # Per-layer geometry (config.py:83-87); ``index`` is 0-based.
    def is_global(self, index):
        return index + 1 in self.global_layers

    def layer_kv_heads(self, index):
        if self.is_global(index):
            return self.global_kv_heads or self.kv_heads
        return self.kv_heads

    def layer_window(self, index):
        return None if self.is_global(index) else self.window

    @property
    def split_half_rope(self):
        return self.family in SPLIT_HALF_FAMILIES

    def to_dict(self):
        """Bundle format 1 (config.py:89-90)."""
        return {"backend_format": 1, **asdict(self)}

    @classmethod
    def from_dict(cls, data, family=None):
        """Bundle-format dicts, or native training configs (config.py:92-153)."""
        if data.get("backend_format") == 1:
            values = dict(data)
            values.pop("backend_format")
            if family is not None and family != values["family"]:
                raise ValueError("family override conflicts with bundle")
            values["global_layers"] = tuple(values.get("global_layers", ()))
            return cls(**values)
        family = family if family is not None else _detect_family(data)
        if family not in FAMILIES:
            raise ValueError(f"Unsupported family: {family}")
        return cls(**_native_fields(data, family))

    def inverse_frequencies(self):
        """float32[head_dim/2] RoPE inverse frequencies (config.py:155-197)."""
        return rope_inverse_frequencies(self)


def _detect_family(data):
    """Architecture auto-detection from native config keys (config.py:100-117)."""
    kind = data.get("model_type", "")
    if "neural" in kind.lower():
        raise ValueError("Miracle Neural is outside this backend's scope")
    rules = (
        ("flashnano-1.7", "flashnano_17" in kind or "global_layer_indices_1based" in data),
        ("flashnano-1.6", "cbr_chunk_size" in data),
        ("flashnano-1.5", "flashnano" in kind),
        ("flashlighting-2.0", kind == "miracle_dense_2_7b" or "kv_latent_dim" in data),
        ("heavy-medium-2.0", "routed_experts" in data),
        ("flashlite-2.0", kind == "miracle_dense"),
    )
    for name, matched in rules:
        if matched:
            return name
    raise ValueError("Cannot identify architecture; specify --family explicitly")


def _native_fields(data, family):
    """Field aliases and family defaults of native configs (config.py:120-153)."""
    def first(*names, default=None):
        for name in names:
            if name in data:
                return data[name]
        if default is None:
            raise ValueError(f"Missing architecture field: {'/'.join(names)}")
        return default

    heavy = family == "heavy-medium-2.0"
    long = data.get("long_context", {})
    hidden = first("hidden_size")
    layers = first("layers", "num_hidden_layers", "num_layers")
    heads = first("query_heads", "num_attention_heads")
    if heavy:
        window = long.get("local_window")
    else:
        window = next((data[k] for k in ("window", "local_window", "local_window_size", "attention_window")
                       if k in data), None)
    residual = data.get("residual_scale")
    if residual is None:
        residual = (2 * layers) ** -0.5 if family in ("flashlite-2.0", "flashlighting-2.0") else 1.0
    return dict(
        family=family, vocab_size=first("vocab_size"), hidden_size=hidden, layers=layers,
        query_heads=heads, kv_heads=first("kv_heads", "num_key_value_heads", "num_kv_heads"),
        head_dim=first("head_dim", default=hidden // heads),
        ffn_dim=first("ffn_dim", "intermediate_size", "expert_intermediate_size"),
        max_positions=long.get("target_context", 1_048_576) if heavy
        else first("max_positions", "max_position_embeddings"),
        window=window,
        global_layers=tuple(data.get("global_layer_indices_1based", data.get("global_attention_layers", ()))),
        global_kv_heads=data.get("global_kv_heads", 0),
        rope_theta=long.get("rope_theta", 1e6) if heavy else data.get("rope_theta", 1e6),
        norm_eps=first("norm_eps", "rms_norm_eps", "norm_epsilon", default=1e-6),
        tie_embeddings=first("tie_embeddings", "tie_word_embeddings", default=True),
        qk_norm=data.get("use_qk_norm", True), residual_scale=residual,
        latent_dim=data.get("kv_latent_dim", data.get("latent_kv_dim", 0)),
        memory_slots=data.get("attention_memory_slots", 0),
        cbr_chunk_size=data.get("cbr_chunk_size", 0), cbr_slots=data.get("cbr_slots", 0),
        cbr_norm_eps=data.get("cbr_norm_eps", 1e-6), inner_loop_steps=data.get("inner_loop_steps", 1),
        eos_token_id=data.get("eos_token_id", 2), source=dict(data))


def rope_inverse_frequencies(config):
    """Base table theta^(-2i/d) in float32, then the family's scaling rule.

    heavy-medium-2.0: the high-index part uses theta*16 (config.py:159-161).
    flashlighting-2.0: linear / dynamic-NTK / YaRN wavelength ramp (config.py:162-182).
    flashnano-1.7: optional YaRN by correction-dimension ramp (config.py:183-196).
    """
    dim, theta, src = config.head_dim, config.rope_theta, config.source
    exponent = np.arange(0, dim, 2, dtype=np.float32) / dim
    inv = np.power(np.float32(theta), -exponent)
    family = config.family
    if family == "heavy-medium-2.0":
        cut = int((dim // 2) * src["long_context"].get("rope_local_fraction", 0.6))
        inv[cut:] = np.power(np.float32(theta * 16), -exponent[cut:])
    elif family == "flashlighting-2.0":
        kind = src.get("rope_scaling_type", "yarn")
        factor = src.get("rope_scaling_factor", 8.0)
        if not math.isfinite(factor) or factor < 1:
            raise ValueError("rope_scaling_factor must be finite and >= 1")
        native = src.get("max_position_embeddings", config.max_positions)
        if kind == "linear":
            inv /= factor
        elif kind == "dynamic_ntk":
            if dim <= 2:
                raise ValueError("dynamic_ntk requires head_dim > 2")
            ratio = factor * src.get("extension_max_position_embeddings", native) / native - (factor - 1)
            inv = np.power(np.float32(theta * max(ratio, 1) ** (dim / (dim - 2))), -exponent)
        elif kind == "yarn":
            low = native / src.get("rope_beta_fast", 32.0)
            high = native / src.get("rope_beta_slow", 1.0)
            if high <= low:
                raise ValueError("YaRN requires beta_fast > beta_slow > 0")
            ramp = np.clip((2 * np.pi / inv - low) / (high - low), 0, 1)
            inv = inv * (1 - ramp) + (inv / factor) * ramp
        elif kind not in ("none", "native"):
            raise ValueError(f"Unsupported RoPE scaling: {kind}")
    elif family == "flashnano-1.7" and src.get("rope_scaling"):
        rs = src["rope_scaling"]
        if rs.get("type") != "yarn":
            raise ValueError("FlashNano 1.7 only supports YaRN rope_scaling")
        factor = float(rs["factor"])
        if not math.isfinite(factor) or factor < 1:
            raise ValueError("YaRN factor must be finite and >= 1")

        def correction_dim(rotations):
            return dim * math.log(rs["orig_max_position"] / (rotations * 2 * math.pi)) / (2 * math.log(theta))

        lo = max(math.floor(correction_dim(rs["beta_fast"])), 0)
        hi = min(math.ceil(correction_dim(rs["beta_slow"])), dim - 1)
        if lo == hi:
            hi += 0.001
        ramp = np.clip((np.arange(dim // 2, dtype=np.float32) - lo) / max(hi - lo, 1e-3), 0, 1)
        inv = (inv / factor) * (1 - ramp) + inv * ramp
    return np.asarray(inv, dtype=np.float32)
