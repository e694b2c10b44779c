"""ORACLE (test infrastructure only): the reference backend's method surface
(miracle_reasoning/opencl.py:178-303) over the oracle's C kernels.

Its one use is tests/golden/make_golden.py, which drives the reference's own
``MiracleModel`` with this object as ``backend`` to write golden fixtures.  Host
numpy arrays stand in for device buffers.  Kernels called by name through
``run`` receive the same argument lists the reference passes
(model.py:129-133, 164-166, 180, 213-216).
"""
from __future__ import annotations

import ctypes as C
import math
from types import SimpleNamespace

import numpy as np

from . import kernels as K


class OracleTensor:
    def __init__(self, device, array):
        self.backend, self.array = device, array
        self.shape = tuple(array.shape)
        self.size = array.size


class OracleDevice:
    def __init__(self, max_allocation_bytes=1 << 40):
        self.device = SimpleNamespace(kind="cpu", name="oracle", max_allocation_bytes=max_allocation_bytes,
                                      to_dict=lambda: {"kind": "cpu", "name": "oracle"})
        self.observe = None   # optional callback receiving every uploaded array

    def _owns(self, *tensors):
        if any(t.backend is not self for t in tensors):
            raise ValueError("Tensors belong to different OpenCL contexts")

    def empty(self, shape):
        shape = tuple(shape)
        if not shape or any(not isinstance(n, int) or n <= 0 for n in shape):
            raise ValueError(f"invalid tensor shape: {shape}")
        if math.prod(shape) * 4 > self.device.max_allocation_bytes:
            raise RuntimeError("allocation above device limit")
        return OracleTensor(self, np.zeros(shape, np.float32))

    def upload(self, array):
        a = np.array(array, dtype=np.float32, order="C", copy=True)
        if self.observe is not None:
            self.observe(a)
        return OracleTensor(self, a)

    def read(self, tensor):
        self._owns(tensor)
        return tensor.array.copy()

    def copy(self, source, target, *, source_offset=0, target_offset=0, count=None):
        self._owns(source, target)
        count = source.size - source_offset if count is None else count
        if min(source_offset, target_offset, count) < 0 or source_offset + count > source.size \
                or target_offset + count > target.size:
            raise ValueError("tensor copy is out of bounds")
        target.array.reshape(-1)[target_offset:target_offset + count] = \
            source.array.reshape(-1)[source_offset:source_offset + count]

    def run(self, name, shape, *args):
        fn = getattr(K.lib(), "oc_" + name)
        converted = []
        for a in args:
            if isinstance(a, OracleTensor):
                self._owns(a)
                converted.append(a.array.ctypes.data_as(C.POINTER(C.c_float)))
            elif isinstance(a, (float, np.floating)):
                converted.append(C.c_float(a))
            elif isinstance(a, (int, np.integer)):
                converted.append(C.c_int(int(a)))
            else:
                raise ValueError(f"unsupported kernel argument: {a}")
        fn(*converted)

    def linear(self, x, weight):
        if len(x.shape) != 2 or len(weight.shape) != 2 or x.shape[1] != weight.shape[1]:
            raise ValueError("linear needs x[rows,in] and weight[out,in]")
        return OracleTensor(self, K.linear(x.array, weight.array))

    def norm(self, x, weight, width, eps):
        if x.size % width or (weight is not None and weight.shape != (width,)):
            raise ValueError("RMSNorm shape mismatch")
        out = K.rms(x.array.reshape(-1, width), None if weight is None else weight.array, width, eps)
        return OracleTensor(self, out.reshape(x.shape))

    def rotate(self, x, frequencies, positions, heads, dim, split_half=False):
        if x.shape != (positions.size, heads * dim):
            raise ValueError("RoPE shape mismatch")
        return OracleTensor(self, K.rope(x.array, frequencies.array, positions.array, heads, dim, split_half))

    def add(self, x, y, scale=1.0):
        if x.shape != y.shape:
            raise ValueError("residual shapes differ")
        return OracleTensor(self, K.axpy(x.array, y.array, float(scale)))

    def swiglu(self, gate, up):
        if gate.shape != up.shape:
            raise ValueError("SwiGLU shapes differ")
        return OracleTensor(self, K.swiglu(gate.array, up.array))

    def softmax(self, x):
        return OracleTensor(self, K.softmax(x.array))

    def attention(self, query, keys, values, *, heads, kv_heads, dim, start, length,
                  extra_keys=None, extra_values=None, extra_length=0):
        s = K.scores(query.array, keys.array, None if extra_keys is None else extra_keys.array, heads, kv_heads,
                     dim, keys.shape[0], start, length, extra_length)
        probs = OracleTensor(self, K.softmax(s))
        return self.mix(probs, values, heads, kv_heads, dim, start, length, extra_values, extra_length)

    def mix(self, probs, values, heads, kv_heads, dim, start, length, extra_values=None, extra_length=0):
        y = K.mix(probs.array, values.array, None if extra_values is None else extra_values.array, heads,
                  kv_heads, dim, values.shape[0], start, length, extra_length)
        return OracleTensor(self, y)

    def finish(self):
        pass
