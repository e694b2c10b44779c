"""Checkpoint readers and the canonical weight-name table.

The readers keep BF16 and F16 tensors in their stored bits: the HIP library
uploads those bits to HBM unchanged and widens them to FP32 in registers, which
is exactly the reference's host widening (miracle_reasoning/weights.py:64-74,
``u16 << 16`` for BF16, an IEEE cast for F16).
"""
from __future__ import annotations

import json
import math
import struct
from collections.abc import Mapping
from pathlib import Path

import numpy as np

# safetensors dtype tag -> little-endian storage dtype
_STORAGE = {"F32": "<f4", "F16": "<f2", "BF16": "<u2"}
_HEADER_LIMIT = 100_000_000


class SafeTensors(Mapping):
    """Memory-mapped F32/F16/BF16 safetensors with header validation
    (reference: weights.py:14-61)."""

    def __init__(self, path):
        self.path = Path(path)
        file_size = self.path.stat().st_size
        with self.path.open("rb") as handle:
            head = handle.read(8)
            if len(head) != 8:
                raise ValueError("Truncated safetensors header")
            (header_len,) = struct.unpack("<Q", head)
            if header_len > min(_HEADER_LIMIT, file_size - 8):
                raise ValueError("Invalid safetensors header length")
            header = json.loads(handle.read(header_len))
        self.offset = 8 + header_len
        payload = file_size - self.offset
        self.entries = {}
        spans = []
        for name, entry in header.items():
            if name == "__metadata__":
                continue
            tag = entry["dtype"]
            if tag not in _STORAGE:
                raise ValueError(f"Unsupported weight dtype {tag} in {name}; export to FP32 first")
            shape, offsets = entry["shape"], entry["data_offsets"]
            if not isinstance(shape, list) or any(type(n) is not int or n < 0 for n in shape):
                raise ValueError(f"Invalid shape for {name}")
            if len(offsets) != 2 or any(type(n) is not int for n in offsets):
                raise ValueError(f"Invalid offsets for {name}")
            begin, end = offsets
            nbytes = math.prod(shape) * np.dtype(_STORAGE[tag]).itemsize
            if begin < 0 or end - begin != nbytes or end > payload:
                raise ValueError(f"Invalid safetensors extent for {name}")
            self.entries[name] = (tuple(shape), tag, begin)
            spans.append((begin, end))
        spans.sort()
        for (_, prev_end), (next_begin, _) in zip(spans, spans[1:]):
            if next_begin < prev_end:
                raise ValueError("Overlapping safetensors data")

    def __iter__(self):
        return iter(self.entries)

    def __len__(self):
        return len(self.entries)

    def __getitem__(self, key):
        shape, tag, begin = self.entries[key]
        data = np.memmap(self.path, mode="r", offset=self.offset + begin, dtype=_STORAGE[tag], shape=shape)
        return BF16Array(data) if tag == "BF16" else data


class BF16Array:
    """BF16 storage (raw uint16 bits); slicing widens to FP32 exactly."""

    def __init__(self, bits):
        self.bits = bits
        self.shape = bits.shape

    # The reference's attribute name for the raw bits.
    @property
    def data(self):
        return self.bits

    def __getitem__(self, key):
        return (np.asarray(self.bits[key], dtype=np.uint32) << 16).view(np.float32)

    def __array__(self, dtype=None, copy=None):
        widened = self[:]
        return widened if dtype is None else widened.astype(dtype, copy=False)


def bf16_bits(array):
    """Round FP32 to BF16 (nearest, ties to even) and return the uint16 bits."""
    a = np.ascontiguousarray(array, dtype=np.float32)
    u = a.view(np.uint32)
    # Finite values never carry out of 32 bits here; NaNs are fixed up below.
    out = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        out[nan] = 0x7FC0
    return out.reshape(a.shape)


class ShardedSafeTensors(Mapping):
    """``model.safetensors.index.json`` with shard-path containment
    (reference: weights.py:77-99)."""

    def __init__(self, index):
        index = Path(index)
        self.names = json.loads(index.read_text(encoding="utf-8"))["weight_map"]
        root = index.parent.resolve()
        self.shards = {}
        for filename in sorted(set(self.names.values())):
            path = (root / filename).resolve()
            if not path.is_relative_to(root):
                raise ValueError("Safetensors shard path escapes the model directory")
            self.shards[filename] = SafeTensors(path)
        for key, filename in self.names.items():
            if key not in self.shards[filename]:
                raise ValueError(f"Shard {filename} does not contain {key}")

    def __iter__(self):
        return iter(self.names)

    def __len__(self):
        return len(self.names)

    def __getitem__(self, key):
        return self.shards[self.names[key]][key]


def _stored(value):
    """(safetensors dtype tag, storage view) of one tensor as this package
    keeps it: BF16 bits stay BF16, float16 stays F16, the rest is FP32."""
    if isinstance(value, BF16Array):
        return "BF16", value.bits
    if getattr(value, "dtype", None) == np.float16:
        return "F16", value
    return "F32", value


def write_safetensors(path, tensors, *, widen=False):
    """Write ``tensors`` (name -> array-like with ``.shape``) as one
    safetensors file.

    Each tensor keeps its stored dtype (BF16 bits, F16, else FP32) unless
    ``widen`` asks for FP32 throughout, which is the reference's bundle format
    (weights.py:102-125).  Values are converted and written about 16 MiB at a
    time, so memory-mapped inputs are never materialised whole, and the file
    appears under its name only once complete."""
    plan, header, offset = [], {}, 0
    for name, value in tensors.items():
        tag, view = ("F32", value) if widen else _stored(value)
        shape = tuple(int(n) for n in view.shape)
        dtype = np.dtype(_STORAGE[tag])
        size = math.prod(shape) * dtype.itemsize
        header[name] = {"dtype": tag, "shape": list(shape), "data_offsets": [offset, offset + size]}
        plan.append((view, shape, dtype))
        offset += size
    text = json.dumps(header, separators=(",", ":")).encode("utf-8")
    text += b" " * (-(8 + len(text)) % 8)            # payload starts 8-byte aligned
    path = Path(path)
    partial = path.with_name(path.name + ".partial")
    try:
        with partial.open("wb") as out:
            out.write(struct.pack("<Q", len(text)) + text)
            for view, shape, dtype in plan:
                if not shape:
                    out.write(np.asarray(view, dtype=dtype).tobytes())
                    continue
                rows = max(1, (16 << 20) // max(1, math.prod(shape[1:]) * dtype.itemsize))
                for r in range(0, shape[0], rows):
                    out.write(np.ascontiguousarray(view[r:r + rows], dtype=dtype).tobytes())
        partial.replace(path)
    finally:
        partial.unlink(missing_ok=True)
    return path


class AliasedWeights(Mapping):
    """Canonical names over a native checkpoint (reference: weights.py:128-142)."""

    def __init__(self, original, names):
        self.original, self.names = original, names
        missing = [native for native in names.values() if native not in original]
        if missing:
            raise ValueError(f"Missing checkpoint tensors: {', '.join(missing[:12])}")

    def __iter__(self):
        return iter(self.names)

    def __len__(self):
        return len(self.names)

    def __getitem__(self, key):
        return self.original[self.names[key]]


# Native training-repository layouts, per family (reference: weights.py:145-208).
_LAYER_ROOT = {"flashnano-1.5": "backbone.layers.{i}.", "flashlite-2.0": "backbone.layers.{i}.",
               "flashnano-1.6": "blocks.{i}.", "flashnano-1.7": "blocks.{i}.",
               "flashlighting-2.0": "layers.{i}.", "heavy-medium-2.0": "blocks.{i}."}
# (attention norm, ffn norm, attention module, ffn module)
_LAYER_PARTS = {
    "flashnano-1.5": ("input_norm.weight", "post_attention_norm.weight", "attention.", "feed_forward."),
    "flashlite-2.0": ("input_norm.weight", "post_attention_norm.weight", "attention.", "feed_forward."),
    "flashnano-1.6": ("attn_norm.weight", "ffn_norm.weight", "attn.", "ffn."),
    "flashnano-1.7": ("attn_norm_weight", "ffn_norm_weight", "attn.", "ffn."),
    "flashlighting-2.0": ("input_norm.weight", None, "attention.", "feed_forward."),
    "heavy-medium-2.0": ("attention_norm.weight", "moe_norm.weight", "attention.", None),
}


def native_names(config):
    """Map canonical names (``layers.{i}.q`` ...) to native checkpoint names."""
    c = config
    fam = c.family
    names = {}
    if fam in ("flashnano-1.5", "flashlite-2.0"):
        names["embed"] = "backbone." + ("token_embedding.weight" if fam == "flashnano-1.5"
                                        else "embed_tokens.weight")
        names["norm"] = "backbone.norm.weight"
    else:
        names["embed"] = "embed_tokens.weight" if fam == "flashlighting-2.0" else "embedding.weight"
        names["norm"] = "final_norm_weight" if fam == "flashnano-1.7" else "final_norm.weight"
    if not c.tie_embeddings:
        names["output"] = "lm_head.weight"
    wname = (lambda key: f"w_{key}.weight") if fam == "flashnano-1.6" else (lambda key: f"{key}_proj.weight")
    an, fn, attn, ffn = _LAYER_PARTS[fam]
    for i in range(c.layers):
        p, root = f"layers.{i}.", _LAYER_ROOT[fam].format(i=i)
        names[p + "a_norm"] = root + an
        if fn:
            names[p + "f_norm"] = root + fn
        names[p + "q"] = root + attn + wname("q")
        names[p + "o"] = root + attn + ("out_proj.weight" if fam == "heavy-medium-2.0" else wname("o"))
        if fam == "flashlighting-2.0":
            names[p + "latent"] = root + attn + "kv_down.weight"
            names[p + "latent_norm"] = root + attn + "kv_norm.weight"
            names[p + "k"] = root + attn + "k_up.weight"
            names[p + "v"] = root + attn + "v_up.weight"
            names[p + "attention_gate"] = root + "attention_gate"
            names[p + "ffn_gate"] = root + "ffn_gate"
        elif fam == "heavy-medium-2.0":
            names[p + "latent"] = root + attn + "kv_down.weight"
            names[p + "kv_up"] = root + attn + "kv_up.weight"
        else:
            names[p + "k"] = root + attn + wname("k")
            names[p + "v"] = root + attn + wname("v")
        if c.qk_norm and fam != "heavy-medium-2.0":
            for key in ("q", "k"):
                names[p + key + "_norm"] = root + attn + (f"qk_norm_{key}" if fam == "flashnano-1.7"
                                                          else f"{key}_norm.weight")
        if ffn:
            for key in ("gate", "up", "down"):
                names[p + "ffn." + key] = root + ffn + wname(key)
        if fam == "flashnano-1.6":
            names[p + "cbr"] = root + "cbr.queries"
        if fam == "heavy-medium-2.0":
            for level in ("coarse", "fine"):
                for key in ("weight", "bias"):
                    names[p + f"router.{level}.{key}"] = root + f"moe.router.{level}.{key}"
            for key in ("group_bias", "expert_bias"):
                names[p + "router." + key] = root + "moe.router." + key
            for e in range(c.source["routed_experts"]):
                for key in ("gate", "up", "down"):
                    names[p + f"experts.{e}.{key}"] = root + f"moe.experts.expert_{e}.{key}_weight"
            for e in range(c.source["shared_experts"]):
                for key in ("gate", "up", "down"):
                    names[p + f"shared.{e}.{key}"] = root + f"moe.shared_experts.{e}.{key}_weight"
    return names


def expected_shapes(config):
    """Canonical name -> shape, in a fixed order (reference: weights.py:211-245).

    The insertion order is part of the contract: seeded synthetic weights are
    drawn in this order."""
    c = config
    h, d, f = c.hidden_size, c.head_dim, c.ffn_dim
    qdim = c.query_heads * d
    shapes = {"embed": (c.vocab_size, h), "norm": (h,)}
    if not c.tie_embeddings:
        shapes["output"] = (c.vocab_size, h)
    heavy = c.family == "heavy-medium-2.0"
    for i in range(c.layers):
        p, kv = f"layers.{i}.", c.layer_kv_heads(i) * d
        shapes[p + "a_norm"] = (h,)
        shapes[p + "q"] = (qdim, h)
        shapes[p + "o"] = (h, qdim)
        if c.family != "flashlighting-2.0":
            shapes[p + "f_norm"] = (h,)
        if c.latent_dim:
            shapes[p + "latent"] = (c.latent_dim, h)
        if heavy:
            shapes[p + "kv_up"] = (2 * kv, c.latent_dim)
            experts, groups = c.source["routed_experts"], c.source["router_groups"]
            for level, n in (("coarse", groups), ("fine", experts)):
                shapes[p + f"router.{level}.weight"] = (n, h)
                shapes[p + f"router.{level}.bias"] = (n,)
            shapes[p + "router.group_bias"] = (groups,)
            shapes[p + "router.expert_bias"] = (experts,)
        else:
            inner = c.latent_dim or h
            shapes[p + "k"] = (kv, inner)
            shapes[p + "v"] = (kv, inner)
            if c.qk_norm:
                shapes[p + "q_norm"] = (d,)
                shapes[p + "k_norm"] = (d,)
        if c.family == "flashlighting-2.0":
            shapes[p + "latent_norm"] = (c.latent_dim,)
            shapes[p + "attention_gate"] = (1,)
            shapes[p + "ffn_gate"] = (1,)
        if c.family == "flashnano-1.6":
            shapes[p + "cbr"] = (c.cbr_slots, h)
        if heavy:
            roots = [p + f"experts.{e}." for e in range(c.source["routed_experts"])]
            roots += [p + f"shared.{e}." for e in range(c.source["shared_experts"])]
        else:
            roots = [p + "ffn."]
        for root in roots:
            shapes[root + "gate"] = (f, h)
            shapes[root + "up"] = (f, h)
            shapes[root + "down"] = (h, f)
    return shapes


def adapt_weights(config, original):
    """Resolve native names and check every shape before any device allocation
    (reference: weights.py:248-255)."""
    weights = original if "embed" in original else AliasedWeights(original, native_names(config))
    for key, shape in expected_shapes(config).items():
        if key not in weights:
            raise ValueError(f"Missing tensor {key}")
        if tuple(weights[key].shape) != shape:
            raise ValueError(f"{key}: expected {shape}, got {weights[key].shape}")
    return weights


def storage_of(array):
    """(contiguous numpy array of stored bits, dtype tag) for upload.

    BF16 stays as uint16 bits, F16 as float16, everything else becomes FP32."""
    if isinstance(array, BF16Array):
        return np.ascontiguousarray(array.bits, dtype=np.uint16), "bf16"
    a = np.asarray(array)
    if a.dtype == np.float16:
        return np.ascontiguousarray(a), "f16"
    return np.ascontiguousarray(a, dtype=np.float32), "f32"
