"""ctypes binding of libmiracle_hip.so and the HIPBackend op surface.

``HIPBackend`` has the method surface of the reference's ``OpenCLBackend``
(miracle_reasoning/opencl.py:129-303): ``empty / upload / read / copy / run /
linear / norm / rotate / add / swiglu / softmax / attention / mix / finish``
plus ``.device``.  The reference's own ``MiracleModel`` therefore runs on it
unchanged, and this package's ``MiracleModel`` uses its step-level engine.

Errors follow the reference: shape misuse raises ``ValueError`` before any
device call; runtime failures raise ``HIPError`` (a ``RuntimeError``) naming the
operation; there is no CPU fallback of any kind.
"""
from __future__ import annotations

import atexit
import ctypes as C
import math
import os
import weakref
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .weights import BF16Array

_LIB_ENV = "MIRACLE_HIP_LIBRARY"
_LIB_DEFAULT = Path(__file__).resolve().parent / "_lib" / "libmiracle_hip.so"

MR_F32, MR_BF16, MR_F16 = 0, 1, 2
_DTYPE_TAG = {"f32": MR_F32, "bf16": MR_BF16, "f16": MR_F16}
MR_ERR_NONFINITE = 5
MR_ERR_TIMEOUT = 7


class HIPError(RuntimeError):
    """A HIP runtime or library failure (the reference's OpenCLError)."""


class _DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("arch", C.c_char * 64), ("memory_bytes", C.c_int64),
                ("max_allocation_bytes", C.c_int64), ("compute_units", C.c_int32), ("pci_bus_id", C.c_int32),
                ("clock_khz", C.c_int32), ("memory_clock_khz", C.c_int32), ("memory_bus_width", C.c_int32),
                ("reserved", C.c_int32)]


class ModelDesc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "family", "vocab_size", "hidden_size", "layers", "query_heads", "kv_heads", "global_kv_heads",
        "head_dim", "ffn_dim", "context_length", "window", "tie_embeddings", "qk_norm", "split_half_rope",
        "latent_dim", "memory_slots", "cbr_chunk_size", "cbr_slots", "inner_loop_steps")] + \
        [(n, C.c_float) for n in ("norm_eps", "cbr_norm_eps", "residual_scale")] + \
        [(n, C.c_int32) for n in ("routed_experts", "router_groups", "router_top_k_min", "router_top_k_max",
                                   "shared_experts", "global_block_size", "global_slots")] + \
        [(n, C.c_float) for n in ("router_temperature", "alibi_slope_scale")] + \
        [("global_layer_mask_lo", C.c_uint64), ("global_layer_mask_hi", C.c_uint64)] + \
        [(n, C.c_float) for n in ("heavy_step_scale", "heavy_shared_scale", "block_slope", "reserved0")]


_P, _i, _f, _sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t
_SIGNATURES = {
    "mr_device_count": [C.POINTER(C.c_int)],
    "mr_device_get_info": [_i, C.POINTER(_DeviceInfo)],
    "mr_ctx_create": [_i, C.POINTER(_P)],
    "mr_ctx_destroy": [_P],
    "mr_sync": [_P],
    "mr_alloc": [_P, _sz, C.POINTER(_P)],
    "mr_free": [_P, _P],
    "mr_h2d": [_P, _P, _P, _sz],
    "mr_d2h": [_P, _P, _P, _sz],
    "mr_d2d": [_P, _P, _P, _sz],
    "mr_linear": [_P, _P, _P, _i, _P, _i, _i, _i],
    "mr_rms": [_P, _P, _P, _P, _i, _i, _f],
    "mr_rope": [_P, _P, _P, _P, _P, _i, _i, _i, _i],
    "mr_swiglu": [_P, _P, _P, _P, _i],
    "mr_axpy": [_P, _P, _P, _P, _i, _f],
    "mr_scores": [_P, _P, _P, _P, _P, _i, _i, _i, _i, _i, _i, _i],
    "mr_softmax": [_P, _P, _P, _i, _i],
    "mr_latent_mask": [_P, _P, _P, _i, _i, _i, _i],
    "mr_mix": [_P, _P, _P, _P, _P, _i, _i, _i, _i, _i, _i, _i],
    "mr_pool_scores": [_P, _P, _P, _P, _i, _i, _i],
    "mr_pool_mix": [_P, _P, _P, _P, _P, _i, _i, _i, _i],
    "mr_merge_rows": [_P, _P, _P, _i, _f, _f],
    "mr_block_means": [_P, _P, _P, _i, _i, _i],
    "mr_attention": [_P, _P, _P, _P, _P, _P, _P, _i, _i, _i, _i, _i, _i, _i],
    "mr_attention_noalloc": [_P, _P, _P, _P, _P, _P, _P, _i, _i, _i, _i, _i, _i, _i],
    "mr_model_create": [_P, C.POINTER(ModelDesc), C.POINTER(_P)],
    "mr_model_destroy": [_P],
    "mr_model_set_weight": [_P, _i, _i, _i, _P, _i, C.c_int64, C.c_int64],
    "mr_model_set_rope": [_P, _P, _i],
    "mr_model_finalize": [_P],
    "mr_model_reset": [_P],
    "mr_model_position": [_P, C.POINTER(C.c_int)],
    "mr_model_forward": [_P, _P, _i, _i, _P],
    "mr_model_generate_greedy": [_P, _i, _i, _P, C.POINTER(C.c_int)],
    "mr_model_set_step_mode": [_P, _i],
    "mr_model_get_step_mode": [_P, C.POINTER(C.c_int)],
    "mr_model_last_decode_ms": [_P, C.POINTER(C.c_float)],
    "mr_model_trace_step": [_P, _P, C.c_int64, C.POINTER(C.c_int), C.POINTER(C.c_int)],
    "mr_model_choices": [_P, _P, C.c_int64, C.POINTER(_i)],
    "mr_model_time_kernel": [_P, _i, _i, C.POINTER(C.c_float)],
    "mr_debug_fail_next": [_P],
    "mr_debug_step_timeout": [_P],
    "mr_debug_gemm": [_P, _P, _P, _P, _P, _i, _i, _i, _i],
    "mr_debug_gemm_grouped": [_P, _P, _P, _P, _P, C.POINTER(C.c_int), _i, _i, _i, _i, _i],
    "mr_debug_prefill_attention": [_P, _P, _P, _P, _P, _i, _i, _i, _i, _i, _i, _i, _i],
    "mr_debug_exp": [_P, _P, _P, _i, _i],
}

_lib = None


def library_path():
    return Path(os.environ.get(_LIB_ENV) or _LIB_DEFAULT)


def _load():
    global _lib
    if _lib is None:
        path = library_path()
        if not path.exists():
            raise HIPError(f"HIP library not found at {path}; build it with `make -C miraclereasoning-cpu_amd/csrc` "
                           "(or __graft_entry__.build()). There is no CPU fallback.")
        try:
            lib = C.CDLL(str(path))
        except OSError as exc:
            raise HIPError(f"Cannot load {path}: {exc}") from exc
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes, fn.restype = args, C.c_int
        lib.mr_last_error.argtypes, lib.mr_last_error.restype = [], C.c_char_p
        _lib = lib
    return _lib


# Teardown order.  Models, then contexts, are released by one atexit hook,
# which Python runs before it tears down modules and before the C runtime's
# exit handlers (the HIP runtime's among them), so no HIP call is left to a
# finalizer running during interpreter shutdown.  After the hook every
# __del__ here does nothing.
_backends = weakref.WeakSet()
_shut_down = False


def close_all():
    """Release every live model and context now.  Backends, models and
    tensors made afterwards work and are released as usual."""
    for backend in list(_backends):
        backend.close()


def _at_exit():
    # The interpreter is ending: release everything, then make the finalizers
    # that still run during module teardown do nothing.
    global _shut_down
    close_all()
    _shut_down = True


atexit.register(_at_exit)


def _check(code, operation):
    if code:
        message = _load().mr_last_error().decode("utf-8", "replace")
        raise HIPError(f"{operation} failed (code {code}): {message}")


@dataclass(frozen=True)
class Device:
    """Same fields as the reference's Device (opencl.py:68-81)."""
    platform_index: int
    device_index: int
    platform: str
    name: str
    vendor: str
    kind: str
    memory_bytes: int
    max_allocation_bytes: int
    handle: int
    arch: str = ""
    compute_units: int = 0

    def to_dict(self):
        return {k: v for k, v in vars(self).items() if k != "handle"}


def list_devices():
    """Visible HIP GPUs (reference: list_devices, opencl.py:113-115)."""
    lib = _load()
    n = C.c_int()
    _check(lib.mr_device_count(C.byref(n)), "enumerate HIP devices")
    out = []
    for i in range(n.value):
        info = _DeviceInfo()
        _check(lib.mr_device_get_info(i, C.byref(info)), "query device")
        out.append(Device(0, i, "HIP", info.name.decode(), "AMD", "gpu", info.memory_bytes,
                          info.max_allocation_bytes, i, info.arch.decode(), info.compute_units))
    return out


class Tensor:
    """A device buffer owned by one backend (reference: opencl.py:118-126).

    ``dtype`` is "f32" for activations; weight tensors made by
    ``upload_weight`` may hold BF16 or F16 bits."""

    def __init__(self, backend, handle, shape, dtype="f32"):
        self.backend, self.handle, self.shape, self.dtype = backend, handle, tuple(shape), dtype
        self.size = math.prod(self.shape)

    @property
    def nbytes(self):
        return self.size * (4 if self.dtype == "f32" else 2)

    def __del__(self):
        if not _shut_down and getattr(self, "handle", None) and getattr(self.backend, "ctx", None):
            _load().mr_free(self.backend.ctx, self.handle)
            self.handle = None


def _shape_ok(shape):
    return bool(shape) and all(isinstance(n, int) and n > 0 for n in shape)


class HIPBackend:
    """FP32 execution on one MI355X.  One instance and its stream must be used
    by a single thread at a time."""

    def __init__(self, *, platform_index=None, device_index=None, device_type="gpu"):
        if device_type not in ("cpu", "gpu"):
            raise ValueError("device_type must be cpu or gpu")
        self.ctx = None
        lib = _load()
        devices = [d for d in list_devices()
                   if (platform_index in (None, 0)) and (device_index is None or d.device_index == device_index)]
        if device_type != "gpu" or not devices:
            raise HIPError(f"No matching HIP {device_type.upper()} device. This backend runs on MI355X (gfx950) "
                           "GPUs only; there is no CPU fallback.")
        self.device = devices[0]
        ctx = C.c_void_p()
        _check(lib.mr_ctx_create(self.device.device_index, C.byref(ctx)), "create context")
        self.ctx = ctx
        self.lib = lib
        self._engines = weakref.WeakSet()   # step-level models created on this context
        _backends.add(self)

    def close(self):
        """Release the models made on this backend, then its stream and buffers.
        Tensors of a closed backend are not freed again."""
        for engine in list(getattr(self, "_engines", ())):
            engine.close()
        if getattr(self, "ctx", None):
            _load().mr_ctx_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        if not _shut_down:
            self.close()

    # ------------------------------------------------------------ memory
    def _owns(self, *tensors):
        if any(t.backend is not self for t in tensors):
            raise ValueError("Tensors belong to different HIP contexts")

    def _alloc(self, shape, dtype="f32"):
        shape = tuple(shape)
        if not _shape_ok(shape):
            raise ValueError(f"invalid tensor shape: {shape}")
        nbytes = math.prod(shape) * (4 if dtype == "f32" else 2)
        if nbytes > self.device.max_allocation_bytes:
            raise HIPError(f"Buffer needs {nbytes:,} bytes, above device allocation limit "
                           f"{self.device.max_allocation_bytes:,}")
        handle = C.c_void_p()
        _check(self.lib.mr_alloc(self.ctx, nbytes, C.byref(handle)), f"allocate {nbytes:,} bytes")
        return Tensor(self, handle.value, shape, dtype)

    def empty(self, shape):
        return self._alloc(shape)

    def upload(self, array):
        array = np.ascontiguousarray(array, dtype=np.float32)
        out = self.empty(array.shape)
        _check(self.lib.mr_h2d(self.ctx, out.handle, array.ctypes.data, array.nbytes), "upload tensor")
        return out

    def upload_weight(self, array):
        """Upload a weight keeping BF16/F16 storage (BF16Array / float16 arrays)."""
        if isinstance(array, BF16Array):
            bits, tag = np.ascontiguousarray(array.bits, dtype=np.uint16), "bf16"
        else:
            a = np.asarray(array)
            if a.dtype == np.float16:
                bits, tag = np.ascontiguousarray(a), "f16"
            else:
                return self.upload(a)
        out = self._alloc(bits.shape, tag)
        _check(self.lib.mr_h2d(self.ctx, out.handle, bits.ctypes.data, bits.nbytes), "upload tensor")
        return out

    def read(self, tensor):
        self._owns(tensor)
        if tensor.dtype != "f32":
            raise ValueError("read() returns float32 tensors only")
        out = np.empty(tensor.shape, dtype=np.float32)
        _check(self.lib.mr_d2h(self.ctx, out.ctypes.data, tensor.handle, out.nbytes), "read tensor")
        return out

    def copy(self, source, target, *, source_offset=0, target_offset=0, count=None):
        self._owns(source, target)
        count = source.size - source_offset if count is None else count
        if min(source_offset, target_offset, count) < 0 or source_offset + count > source.size \
                or target_offset + count > target.size:
            raise ValueError("tensor copy is out of bounds")
        if count:
            _check(self.lib.mr_d2d(self.ctx, target.handle + target_offset * 4, source.handle + source_offset * 4,
                                   count * 4), "copy tensor")

    def finish(self):
        _check(self.lib.mr_sync(self.ctx), "finish queue")

    # ------------------------------------------------------------ kernels by name
    def run(self, name, shape, *args):
        """Enqueue a kernel by its reference name with the reference's argument
        list (opencl.py:219-239).  ``shape`` (the NDRange) is implied by the
        arguments and only checked for rank."""
        if name not in _RUN_TABLE:
            raise HIPError(f"create kernel {name} failed: no such kernel")
        converted = []
        for a in args:
            if isinstance(a, Tensor):
                self._owns(a)
                converted.append(a)
            elif isinstance(a, (float, np.floating)):
                converted.append(float(a))
            elif isinstance(a, (int, np.integer)) and -(2**31) <= a < 2**31:
                converted.append(int(a))
            else:
                raise ValueError(f"unsupported kernel argument: {a}")
        if not isinstance(shape, (tuple, list)) or not 1 <= len(shape) <= 3:
            raise ValueError("run: shape must be a 1-3 dimensional NDRange")
        _RUN_TABLE[name](self, *converted)

    def _call(self, fn, op, *args):
        cargs = [a.handle if isinstance(a, Tensor) else a for a in args]
        _check(fn(self.ctx, *cargs), f"enqueue {op}")

    # ------------------------------------------------------------ op wrappers
    def linear(self, x, weight):
        if len(x.shape) != 2 or len(weight.shape) != 2 or x.shape[1] != weight.shape[1]:
            raise ValueError("linear needs x[rows,in] and weight[out,in]")
        self._owns(x, weight)
        rows, inner = x.shape
        out = self.empty((rows, weight.shape[0]))
        _check(self.lib.mr_linear(self.ctx, x.handle, weight.handle, _DTYPE_TAG[weight.dtype], out.handle, rows,
                                  weight.shape[0], inner), "enqueue linear")
        return out

    def norm(self, x, weight, width, eps):
        if x.size % width or (weight is not None and weight.shape != (width,)):
            raise ValueError("RMSNorm shape mismatch")
        out = self.empty(x.shape)
        _check(self.lib.mr_rms(self.ctx, x.handle, weight.handle if weight is not None else None, out.handle,
                               x.size // width, width, float(eps)), "enqueue rms")
        return out

    def rotate(self, x, frequencies, positions, heads, dim, split_half=False):
        if x.shape != (positions.size, heads * dim):
            raise ValueError("RoPE shape mismatch")
        out = self.empty(x.shape)
        _check(self.lib.mr_rope(self.ctx, x.handle, frequencies.handle, positions.handle, out.handle, positions.size,
                                heads, dim, int(split_half)), "enqueue rope")
        return out

    def add(self, x, y, scale=1.0):
        if x.shape != y.shape:
            raise ValueError("residual shapes differ")
        out = self.empty(x.shape)
        _check(self.lib.mr_axpy(self.ctx, x.handle, y.handle, out.handle, x.size, float(scale)), "enqueue axpy")
        return out

    def swiglu(self, gate, up):
        if gate.shape != up.shape:
            raise ValueError("SwiGLU shapes differ")
        out = self.empty(gate.shape)
        _check(self.lib.mr_swiglu(self.ctx, gate.handle, up.handle, out.handle, gate.size), "enqueue swiglu")
        return out

    def softmax(self, x):
        out = self.empty(x.shape)
        _check(self.lib.mr_softmax(self.ctx, x.handle, out.handle, x.shape[0], math.prod(x.shape[1:])),
               "enqueue softmax")
        return out

    def attention(self, query, keys, values, *, heads, kv_heads, dim, start, length,
                  extra_keys=None, extra_values=None, extra_length=0):
        out = self.empty((1, heads * dim))
        _check(self.lib.mr_attention(self.ctx, query.handle, keys.handle, values.handle,
                                     extra_keys.handle if extra_keys is not None else None,
                                     extra_values.handle if extra_values is not None else None, out.handle,
                                     heads, kv_heads, dim, keys.shape[0], start, length, extra_length),
               "enqueue attention")
        return out

    def mix(self, probs, values, heads, kv_heads, dim, start, length, extra_values=None, extra_length=0):
        out = self.empty((1, heads * dim))
        _check(self.lib.mr_mix(self.ctx, probs.handle, values.handle,
                               extra_values.handle if extra_values is not None else values.handle, out.handle,
                               heads, kv_heads, dim, values.shape[0], start, length, extra_length), "enqueue mix")
        return out

    def debug_gemm(self, a, weight, scheme):
        """a . weight^T through the batched-prefill MFMA GEMM (test hook):
        scheme 0 = BF16 terms, 1 = FP16 terms; ``weight`` a BF16 tensor."""
        self._owns(a, weight)
        if weight.dtype != "bf16" or len(a.shape) != 2 or len(weight.shape) != 2 or a.shape[1] != weight.shape[1]:
            raise ValueError("debug_gemm needs a[m,k] and a BF16 weight[n,k]")
        m, k = a.shape
        n = weight.shape[0]
        out, ws = self.empty((m, n)), self.empty((m,))
        _check(self.lib.mr_debug_gemm(self.ctx, a.handle, weight.handle, out.handle, ws.handle, m, n, k, scheme),
               "debug gemm")
        return out

    def debug_gemm_grouped(self, a, weight, counts, weight2=None, tile_list=True):
        """The batched prefill's grouped (expert) MFMA GEMM in FP16 terms (test
        hook): group z is the next counts[z] rows of ``a`` [rows, k] with
        weight rows z n .. z n + n - 1 of ``weight`` (BF16 [groups n, k]);
        with ``weight2`` (same layout) the SwiGLU of the two products.  Returns
        c [rows, n]."""
        self._owns(a, weight, *([weight2] if weight2 is not None else []))
        groups = len(counts)
        if (weight.dtype != "bf16" or len(a.shape) != 2 or len(weight.shape) != 2 or a.shape[1] != weight.shape[1]
                or groups == 0 or weight.shape[0] % groups or a.shape[0] != sum(counts)
                or (weight2 is not None and (weight2.dtype != "bf16" or weight2.shape != weight.shape))):
            raise ValueError("debug_gemm_grouped needs a[sum(counts), k] and BF16 weights[groups n, k]")
        rows, k = a.shape
        n = weight.shape[0] // groups
        out = self.empty((rows, n))
        c_counts = (C.c_int * groups)(*counts)
        _check(self.lib.mr_debug_gemm_grouped(self.ctx, a.handle, weight.handle,
                                              weight2.handle if weight2 is not None else None, out.handle, c_counts,
                                              groups, n, k, int(weight2 is not None), int(tile_list)),
               "debug grouped gemm")
        return out

    def debug_exp(self, x, which):
        """2^x by the prefill softmax's hardware exp2 (which 0) or e^x by the
        token step's expf (which 1), elementwise (test hook)."""
        self._owns(x)
        out = self.empty(x.shape)
        _check(self.lib.mr_debug_exp(self.ctx, x.handle, out.handle, int(np.prod(x.shape)), which), "debug exp")
        return out

    def debug_prefill_attention(self, qkv, ring_k, ring_v, *, p0, heads, kv_heads, dim, window=0, presplit=False):
        """The batched-prefill attention kernel on device buffers (test hook):
        qkv [rows, (heads + 2 kv_heads) dim], ring_k/ring_v [cap, kv_heads dim]."""
        self._owns(qkv, ring_k, ring_v)
        rows, cap = qkv.shape[0], ring_k.shape[0]
        if qkv.shape[1] != (heads + 2 * kv_heads) * dim or ring_k.shape != (cap, kv_heads * dim) \
                or ring_v.shape != ring_k.shape:
            raise ValueError("debug_prefill_attention: shapes do not match the head geometry")
        out = self.empty((rows, heads * dim))
        _check(self.lib.mr_debug_prefill_attention(self.ctx, qkv.handle, ring_k.handle, ring_v.handle, out.handle,
                                                   rows, p0, heads, kv_heads, dim, cap, window, int(presplit)),
               "debug prefill attention")
        return out

    def fail_next(self):
        """Test hook: the next library call on this context fails."""
        _check(self.lib.mr_debug_fail_next(self.ctx), "arm failure")


def _h(t):
    return t.handle


# Reference kernel name -> call with the reference's argument list (kernels.cl).
_RUN_TABLE = {
    "linear": lambda b, x, w, y, rows, out, inner: b._call(
        b.lib.mr_linear, "linear", x, w, _DTYPE_TAG[w.dtype], y, rows, out, inner),
    "rms": lambda b, x, w, y, rows, width, eps, affine: b._call(
        b.lib.mr_rms, "rms", x, w if affine else None, y, rows, width, eps),
    "rope": lambda b, *a: b._call(b.lib.mr_rope, "rope", *a),
    "swiglu": lambda b, *a: b._call(b.lib.mr_swiglu, "swiglu", *a),
    "axpy": lambda b, *a: b._call(b.lib.mr_axpy, "axpy", *a),
    "scores": lambda b, *a: b._call(b.lib.mr_scores, "scores", *a),
    "softmax": lambda b, *a: b._call(b.lib.mr_softmax, "softmax", *a),
    "latent_mask": lambda b, *a: b._call(b.lib.mr_latent_mask, "latent_mask", *a),
    "mix": lambda b, *a: b._call(b.lib.mr_mix, "mix", *a),
    "pool_scores": lambda b, *a: b._call(b.lib.mr_pool_scores, "pool_scores", *a),
    "pool_mix": lambda b, *a: b._call(b.lib.mr_pool_mix, "pool_mix", *a),
    "merge_rows": lambda b, *a: b._call(b.lib.mr_merge_rows, "merge_rows", *a),
    "block_means": lambda b, *a: b._call(b.lib.mr_block_means, "block_means", *a),
}
