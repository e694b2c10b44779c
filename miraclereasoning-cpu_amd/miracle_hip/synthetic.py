"""Seeded random-init weights and prompts for the named workloads.

The stream is frozen: every fixture and measurement depends on it.
  * tensors are numbered i = 0, 1, ... in ``expected_shapes(config)`` insertion
    order (the order the reference's own tests use,
    tests/test_inference.py:19-21);
  * a 2-D tensor, flattened row-major, is cut into chunks of 2**22 values;
    chunk c draws ``standard_normal(float32)`` from
    ``Generator(PCG64(SeedSequence([seed, i, c])))`` and is scaled by std 0.02,
    except heavy-medium router matrices, std 1/sqrt(hidden) so router logits on
    an RMS-normalised input are about N(0, 1).  Chunks are independent, so they
    are drawn in parallel and the values do not depend on the thread count;
  * 1-D tensors are ones (norm gains, residual gates), except heavy-medium
    router biases, zeros;
  * BF16 workloads round the FP32 draws to BF16 (nearest-even) and store bits;
  * prompt ids are ``default_rng(seed + 1000).integers(0, vocab, length)``.

``micro_weights`` reproduces the reference's unit-test recipe instead
(``default_rng(72)``, 2-D ~ N(0, 0.05) via ``normal``, 1-D ones).
"""
from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from .config import ModelConfig
from .weights import BF16Array, bf16_bits, expected_shapes

_CHUNK = 1 << 22
_ROUTER_BIAS = ("router.coarse.bias", "router.fine.bias", "router.group_bias", "router.expert_bias")


def _as_config(config):
    return config if isinstance(config, ModelConfig) else ModelConfig.from_dict(config)


def synthetic_weights(config, seed, dtype="bf16", std=0.02):
    """Canonical-name dict of FP32 arrays (dtype "f32") or BF16Array (dtype "bf16")."""
    cfg = _as_config(config)
    if dtype not in ("f32", "bf16"):
        raise ValueError("dtype must be f32 or bf16")
    router_std = np.float32(1.0 / math.sqrt(cfg.hidden_size))
    out, jobs = {}, []
    for index, (name, shape) in enumerate(expected_shapes(cfg).items()):
        if len(shape) == 2:
            scale = router_std if ".router." in name else np.float32(std)
            target = np.empty(shape, np.uint16 if dtype == "bf16" else np.float32)
            out[name] = BF16Array(target) if dtype == "bf16" else target
            flat = target.reshape(-1)
            jobs += [(flat, index, c, scale) for c in range(-(-flat.size // _CHUNK))]
        else:
            fill = 0.0 if name.endswith(_ROUTER_BIAS) else 1.0
            out[name] = np.full(shape, fill, np.float32)

    def draw(job):
        flat, index, c, scale = job
        g = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, index, c])))
        begin = c * _CHUNK
        values = g.standard_normal(min(_CHUNK, flat.size - begin), dtype=np.float32)
        values *= scale
        flat[begin:begin + values.size] = bf16_bits(values) if flat.dtype == np.uint16 else values

    with ThreadPoolExecutor(max(1, min(16, len(os.sched_getaffinity(0))))) as pool:
        list(pool.map(draw, jobs))
    return out


def micro_weights(config, seed=72, gates=(0.7, 1.2)):
    """The reference's unit-test weights (tests/test_inference.py:15-22).

    FlashLighting residual gates are set to ``gates`` (attention, ffn), as the
    reference's upstream-parity fixture does (tests/make_reference.py:58-61)."""
    cfg = _as_config(config)
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in expected_shapes(cfg).items():
        if len(shape) == 2:
            out[name] = rng.normal(0, 0.05, shape).astype(np.float32)
        else:
            out[name] = np.ones(shape, np.float32)
    if cfg.family == "flashlighting-2.0" and gates is not None:
        for i in range(cfg.layers):
            out[f"layers.{i}.attention_gate"] = np.full((1,), gates[0], np.float32)
            out[f"layers.{i}.ffn_gate"] = np.full((1,), gates[1], np.float32)
    return out


def prompt_ids(vocab_size, length, seed):
    return np.random.default_rng(seed + 1000).integers(0, vocab_size, length).astype(np.int64)
