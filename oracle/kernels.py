"""ORACLE (test infrastructure only): numpy-facing bindings of oracle/kernels.c.

Every function takes and returns contiguous numpy arrays; shapes follow the
reference backend's op wrappers (miracle_reasoning/opencl.py:241-300).

Pinned by: the closed-form tests restated from tests/test_opencl.py:19-80
(linear, rms, softmax, rope, scores/softmax/mix with GQA, ring wrap and extra
rows), brute-force numpy checks on small shapes for swiglu, axpy, latent_mask,
pool_scores, pool_mix, merge_rows and block_means, and exact lane-order checks
for linear (tests/test_oracle_kernels.py).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
# ORACLE_LIBRARY names another build of kernels.c (the sanitizer build of
# `make -C oracle check-sanitize`); the default is the plain build.
_LIB_PATH = Path(os.environ.get("ORACLE_LIBRARY") or _HERE / "_build" / "liboracle.so")
_lib = None

_F = C.POINTER(C.c_float)
_U16 = C.POINTER(C.c_uint16)
_i, _f = C.c_int, C.c_float

_SIGNATURES = {
    "oc_linear": [_F, _F, _F, _i, _i, _i],
    "oc_linear_bf16": [_F, _U16, _F, _i, _i, _i],
    "oc_rms": [_F, _F, _F, _i, _i, _f, _i],
    "oc_rope": [_F, _F, _F, _F, _i, _i, _i, _i],
    "oc_swiglu": [_F, _F, _F, _i],
    "oc_axpy": [_F, _F, _F, _i, _f],
    "oc_scores": [_F, _F, _F, _F, _i, _i, _i, _i, _i, _i, _i],
    "oc_softmax": [_F, _F, _i, _i],
    "oc_latent_mask": [_F, _F, _i, _i, _i, _i],
    "oc_mix": [_F, _F, _F, _F, _i, _i, _i, _i, _i, _i, _i],
    "oc_pool_scores": [_F, _F, _F, _i, _i, _i],
    "oc_pool_mix": [_F, _F, _F, _F, _i, _i, _i, _i],
    "oc_merge_rows": [_F, _F, _i, _f, _f],
    "oc_block_means": [_F, _F, _i, _i, _i],
}


def build():
    """Compile oracle/kernels.c with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        handle = C.CDLL(str(_LIB_PATH))
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes, fn.restype = args, None
        _lib = handle
    return _lib


def threads():
    """OpenMP threads the oracle uses (OMP_NUM_THREADS, else all affine cores)."""
    env = os.environ.get("OMP_NUM_THREADS")
    return int(env) if env else len(os.sched_getaffinity(0))


def _fp(a):
    return a.ctypes.data_as(_F)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def linear(x, w):
    """y[rows, out] = x[rows, in] . w[out, in]^T; ``w`` is FP32 or BF16 bits (uint16)."""
    x = _f32(x)
    rows, inner = x.shape
    out_dim = w.shape[0]
    if w.shape[1] != inner:
        raise ValueError("linear needs x[rows,in] and weight[out,in]")
    y = np.empty((rows, out_dim), np.float32)
    if w.dtype == np.uint16:
        w = np.ascontiguousarray(w)
        lib().oc_linear_bf16(_fp(x), w.ctypes.data_as(_U16), _fp(y), rows, out_dim, inner)
    else:
        w = _f32(w)
        lib().oc_linear(_fp(x), _fp(w), _fp(y), rows, out_dim, inner)
    return y


def rms(x, weight, width, eps):
    """Row-wise RMSNorm over consecutive ``width`` values; ``weight`` None = non-affine."""
    x = _f32(x)
    if x.size % width or (weight is not None and weight.shape != (width,)):
        raise ValueError("RMSNorm shape mismatch")
    y = np.empty_like(x)
    w = _f32(weight) if weight is not None else x
    lib().oc_rms(_fp(x), _fp(w), _fp(y), x.size // width, width, float(eps), int(weight is not None))
    return y


def rope(x, freq, positions, heads, dim, split_half):
    x, freq, positions = _f32(x), _f32(freq), _f32(positions)
    if x.shape != (positions.size, heads * dim):
        raise ValueError("RoPE shape mismatch")
    y = np.empty_like(x)
    lib().oc_rope(_fp(x), _fp(freq), _fp(positions), _fp(y), positions.size, heads, dim, int(split_half))
    return y


def swiglu(g, u):
    g, u = _f32(g), _f32(u)
    y = np.empty_like(g)
    lib().oc_swiglu(_fp(g), _fp(u), _fp(y), g.size)
    return y


def axpy(x, y, scale):
    """x + float32(scale) * y."""
    x, y = _f32(x), _f32(y)
    if x.shape != y.shape:
        raise ValueError("residual shapes differ")
    z = np.empty_like(x)
    lib().oc_axpy(_fp(x), _fp(y), _fp(z), x.size, float(scale))
    return z


def scores(q, k, extra_k, heads, kv_heads, dim, capacity, start, length, extra_length):
    q, k = _f32(q), _f32(k)
    extra_k = k if extra_k is None else _f32(extra_k)
    total = length + extra_length
    s = np.empty((heads, total), np.float32)
    lib().oc_scores(_fp(q), _fp(k), _fp(extra_k), _fp(s), heads, kv_heads, dim, capacity, start, length,
                    extra_length)
    return s


def softmax(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().oc_softmax(_fp(x), _fp(y), x.shape[0], x.shape[1])
    return y


def latent_mask(s, positions, heads, length, memory, earliest):
    """In place on a contiguous float32 [heads, length] array."""
    positions = _f32(positions)
    lib().oc_latent_mask(_fp(s), _fp(positions), heads, length, memory, earliest)
    return s


def mix(p, v, extra_v, heads, kv_heads, dim, capacity, start, length, extra_length):
    p, v = _f32(p), _f32(v)
    extra_v = v if extra_v is None else _f32(extra_v)
    y = np.empty((1, heads * dim), np.float32)
    lib().oc_mix(_fp(p), _fp(v), _fp(extra_v), _fp(y), heads, kv_heads, dim, capacity, start, length,
                 extra_length)
    return y


def attention(q, k, v, heads, kv_heads, dim, start, length, extra_k=None, extra_v=None, extra_length=0):
    """scores -> softmax -> mix, as the reference backend's ``attention`` op."""
    s = scores(q, k, extra_k, heads, kv_heads, dim, k.shape[0], start, length, extra_length)
    return mix(softmax(s), v, extra_v, heads, kv_heads, dim, v.shape[0], start, length, extra_length)


def pool_scores(u, q, tokens, slots, width):
    u, q = _f32(u), _f32(q)
    s = np.empty((slots, tokens), np.float32)
    lib().oc_pool_scores(_fp(u), _fp(q), _fp(s), tokens, slots, width)
    return s


def pool_mix(u, p, tokens, slots, width, start_position):
    u, p = _f32(u), _f32(p)
    z = np.empty((slots, width), np.float32)
    anchors = np.empty((slots,), np.float32)
    lib().oc_pool_mix(_fp(u), _fp(p), _fp(z), _fp(anchors), tokens, slots, width, start_position)
    return z, anchors


def merge_rows(x, width, a, b):
    x = _f32(x)
    y = np.empty((width,), np.float32)
    lib().oc_merge_rows(_fp(x), _fp(y), width, float(a), float(b))
    return y


def block_means(x, length, width, block):
    x = _f32(x)
    blocks = (length + block - 1) // block
    y = np.empty((blocks, width), np.float32)
    lib().oc_block_means(_fp(x), _fp(y), length, width, block)
    return y
