"""mr_attention_noalloc, the allocation-free variant of mr_attention, called
through the C ABI: bit-identical to mr_attention (same plan and kernels) on
two calls in a row, the second smaller (its counters land where the first
call's partials were, so a missed clear would show), and a call whose scratch
need exceeds the static array is refused before any launch."""
import ctypes as C

import numpy as np
import pytest

from miracle_hip import hip

pytestmark = pytest.mark.gpu

MR_ERR_INVALID = 1


def _case(backend, rng, heads, kv_heads, dim, capacity, start, length, extra):
    q = backend.upload(rng.normal(size=(1, heads * dim)).astype(np.float32))
    k = backend.upload(rng.normal(size=(capacity, kv_heads * dim)).astype(np.float32))
    v = backend.upload(rng.normal(size=(capacity, kv_heads * dim)).astype(np.float32))
    ek = backend.upload(rng.normal(size=(max(extra, 1), kv_heads * dim)).astype(np.float32))
    ev = backend.upload(rng.normal(size=(max(extra, 1), kv_heads * dim)).astype(np.float32))
    return q, k, v, ek, ev


def _noalloc(backend, q, k, v, ek, ev, heads, kv_heads, dim, capacity, start, length, extra):
    out = backend.empty((1, heads * dim))
    rc = hip._load().mr_attention_noalloc(backend.ctx, q.handle, k.handle, v.handle, ek.handle if extra else None,
                                          ev.handle if extra else None, out.handle, heads, kv_heads, dim, capacity,
                                          start, length, extra)
    return rc, out


@pytest.mark.parametrize("order", ["large-then-small", "generic-then-tiled"])
def test_noalloc_attention_equals_mr_attention(backend, order):
    rng = np.random.default_rng(11)
    shapes = {"large-then-small": [(16, 4, 128, 1024, 700, 1000, 10), (8, 2, 64, 256, 0, 100, 0)],
              "generic-then-tiled": [(4, 2, 6, 40, 30, 40, 3), (16, 8, 128, 512, 100, 300, 0)]}[order]
    for heads, kv_heads, dim, capacity, start, length, extra in shapes:
        print("case", heads, kv_heads, dim, capacity, start, length, extra, flush=True)
        q, k, v, ek, ev = _case(backend, rng, heads, kv_heads, dim, capacity, start, length, extra)
        want = backend.read(backend.attention(q, k, v, heads=heads, kv_heads=kv_heads, dim=dim, start=start,
                                              length=length, extra_keys=ek if extra else None,
                                              extra_values=ev if extra else None, extra_length=extra))
        rc, out = _noalloc(backend, q, k, v, ek, ev, heads, kv_heads, dim, capacity, start, length, extra)
        assert rc == 0, hip._load().mr_last_error()
        np.testing.assert_array_equal(backend.read(out), want)


def test_noalloc_attention_refuses_more_scratch_than_it_has(backend):
    # 128 query heads on one KV head over 65536 keys: 512 splits x 128 heads x
    # 130 floats = 34 MB of partials, above the 8 MiB array.  The buffers are
    # full size, though the call returns before any launch.
    rng = np.random.default_rng(12)
    heads, kv_heads, dim, capacity = 128, 1, 128, 65536
    q, k, v, ek, ev = _case(backend, rng, heads, kv_heads, dim, capacity, 0, capacity, 0)
    rc, _ = _noalloc(backend, q, k, v, ek, ev, heads, kv_heads, dim, capacity, 0, capacity, 0)
    assert rc == MR_ERR_INVALID
    assert b"scratch" in hip._load().mr_last_error()
    # the entry point still works after the refusal
    q, k, v, ek, ev = _case(backend, rng, 8, 2, 64, 128, 0, 128, 0)
    want = backend.read(backend.attention(q, k, v, heads=8, kv_heads=2, dim=64, start=0, length=128))
    rc, out = _noalloc(backend, q, k, v, ek, ev, 8, 2, 64, 128, 0, 128, 0)
    assert rc == 0
    np.testing.assert_array_equal(backend.read(out), want)
