"""HIPBackend op surface on the GPU: the reference's closed-form kernel tests
(tests/test_opencl.py:19-80 of the reference) and every op against the oracle's
C restatement on seeded inputs.

Tolerances: elementwise ops with the same formula agree to 1-2 ulp (rtol 1e-6);
dot products (linear, scores, mix, pool) sum in a different order on the GPU
(lanes + shuffles + FMA) and agree to rtol 1e-5 / atol 1e-6 at these sizes.
"""
import numpy as np
import pytest

from oracle import kernels as K

pytestmark = pytest.mark.gpu


def test_primitives_with_non_aligned_shapes(backend):
    b = backend
    rng = np.random.default_rng(9)
    x = rng.normal(size=(3, 19)).astype(np.float32)
    w = rng.normal(size=(7, 19)).astype(np.float32)
    np.testing.assert_allclose(b.read(b.linear(b.upload(x), b.upload(w))), x @ w.T, atol=4e-6)
    scales = rng.normal(size=19).astype(np.float32)
    expected = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-6) * scales
    np.testing.assert_allclose(b.read(b.norm(b.upload(x), b.upload(scales), 19, 1e-6)), expected, atol=1e-6)
    logits = np.array([[1000, 1001, -1000], [-1000, -1001, -1002]], np.float32)
    e = np.exp(logits - logits.max(axis=1, keepdims=True))
    np.testing.assert_allclose(b.read(b.softmax(b.upload(logits))), e / e.sum(axis=1, keepdims=True), atol=1e-7)


@pytest.mark.parametrize("split", [False, True])
def test_rope_layouts(backend, split):
    rng = np.random.default_rng(3)
    x = rng.normal(size=(2, 3, 6)).astype(np.float32)
    pos = np.array([7, 29], np.float32)
    freq = np.array([1, .1, .01], np.float32)
    ang = pos[:, None, None] * freq[None, None, :]
    a, c = (x[..., :3], x[..., 3:]) if split else (x[..., ::2], x[..., 1::2])
    u, v = a * np.cos(ang) - c * np.sin(ang), a * np.sin(ang) + c * np.cos(ang)
    want = np.concatenate([u, v], axis=-1) if split else np.stack([u, v], axis=-1).reshape(2, 3, 6)
    got = backend.rotate(backend.upload(x.reshape(2, 18)), backend.upload(freq), backend.upload(pos), 3, 6, split)
    np.testing.assert_allclose(backend.read(got).reshape(x.shape), want, atol=3e-6)


def test_attention_group_mapping_ring_and_relays(backend):
    b, rng = backend, np.random.default_rng(6)
    q = rng.normal(size=(4, 6)).astype(np.float32)
    k, v = [rng.normal(size=(5, 2, 6)).astype(np.float32) for _ in range(2)]
    rk, rv = [rng.normal(size=(3, 2, 6)).astype(np.float32) for _ in range(2)]
    keys, values = np.concatenate([k[[3, 4, 0, 1]], rk]), np.concatenate([v[[3, 4, 0, 1]], rv])
    want = []
    for h in range(4):
        logits = keys[:, h // 2] @ q[h] / np.sqrt(6)
        p = np.exp(logits - logits.max())
        want.append((p / p.sum()) @ values[:, h // 2])
    got = b.attention(b.upload(q.reshape(1, -1)), b.upload(k.reshape(5, -1)), b.upload(v.reshape(5, -1)),
                      heads=4, kv_heads=2, dim=6, start=3, length=4,
                      extra_keys=b.upload(rk.reshape(3, -1)), extra_values=b.upload(rv.reshape(3, -1)),
                      extra_length=3)
    np.testing.assert_allclose(b.read(got).reshape(4, 6), want, atol=1e-6)


@pytest.mark.parametrize("rows,out,inner,dtype", [
    (1, 2048, 2048, "bf16"), (1, 5632, 2048, "bf16"), (1, 2048, 5632, "bf16"), (1, 32000, 2048, "bf16"),
    (1, 1000, 256, "bf16"), (1, 37, 19, "f32"), (1, 300, 64, "f32"), (1, 24, 12, "bf16"), (4, 70, 33, "f32"),
    (3, 129, 256, "bf16"), (1, 64, 1024, "f16")])
def test_linear_matches_oracle(backend, rows, out, inner, dtype):
    from miracle_hip.weights import BF16Array, bf16_bits
    rng = np.random.default_rng(rows * 7 + out)
    x = rng.normal(size=(rows, inner)).astype(np.float32)
    w32 = (rng.normal(size=(out, inner)) * 0.02).astype(np.float32)
    if dtype == "bf16":
        bits = bf16_bits(w32)
        wt = backend.upload_weight(BF16Array(bits))
        want = K.linear(x, bits)
    elif dtype == "f16":
        w16 = w32.astype(np.float16)
        wt = backend.upload_weight(w16)
        want = K.linear(x, w16.astype(np.float32))
    else:
        wt = backend.upload(w32)
        want = K.linear(x, w32)
    got = backend.read(backend.linear(backend.upload(x), wt))
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_elementwise_ops_match_oracle(backend):
    b, rng = backend, np.random.default_rng(11)
    x = rng.normal(size=(5, 64)).astype(np.float32)
    g = rng.normal(size=64).astype(np.float32)
    np.testing.assert_allclose(b.read(b.norm(b.upload(x), b.upload(g), 64, 1e-5)), K.rms(x, g, 64, 1e-5),
                               rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(b.read(b.norm(b.upload(x), None, 16, 1e-6)), K.rms(x, None, 16, 1e-6),
                               rtol=2e-6, atol=1e-7)
    u = rng.normal(size=(5, 64)).astype(np.float32)
    np.testing.assert_allclose(b.read(b.swiglu(b.upload(x), b.upload(u))), K.swiglu(x, u), rtol=2e-6, atol=1e-7)
    np.testing.assert_array_equal(b.read(b.add(b.upload(x), b.upload(u), 0.37)), K.axpy(x, u, 0.37))
    big = (rng.normal(size=(3, 4099)) * 30).astype(np.float32)
    np.testing.assert_allclose(b.read(b.softmax(b.upload(big))), K.softmax(big), rtol=1e-5, atol=1e-9)


def test_rope_large_positions_match_oracle(backend):
    rng = np.random.default_rng(12)
    x = rng.normal(size=(3, 4 * 128)).astype(np.float32)
    pos = np.array([0, 4095, 8191], np.float32)
    from miracle_hip import ModelConfig, presets
    freq = ModelConfig.from_dict(presets.workload("flashnano-1.7")["config"]).inverse_frequencies()
    for split in (0, 1):
        got = backend.read(backend.rotate(backend.upload(x), backend.upload(freq), backend.upload(pos), 4, 128, split))
        np.testing.assert_allclose(got, K.rope(x, freq, pos, 4, 128, split), rtol=1e-6, atol=1e-6)


def test_scores_softmax_mix_latent_mask_match_oracle(backend):
    b, rng = backend, np.random.default_rng(13)
    heads, kvh, d, cap, start, length, extra = 8, 2, 32, 40, 33, 37, 5
    q = rng.normal(size=(1, heads * d)).astype(np.float32)
    k = rng.normal(size=(cap, kvh * d)).astype(np.float32)
    v = rng.normal(size=(cap, kvh * d)).astype(np.float32)
    ek = rng.normal(size=(extra, kvh * d)).astype(np.float32)
    ev = rng.normal(size=(extra, kvh * d)).astype(np.float32)
    total = length + extra
    s = b.empty((heads, total))
    b.run("scores", (total, heads), b.upload(q), b.upload(k), b.upload(ek), s, heads, kvh, d, cap, start, length,
          extra)
    want_s = K.scores(q, k, ek, heads, kvh, d, cap, start, length, extra)
    np.testing.assert_allclose(b.read(s), want_s, rtol=1e-5, atol=1e-5)
    p = b.softmax(s)
    got = b.read(b.mix(p, b.upload(v), heads, kvh, d, start, length, b.upload(ev), extra))
    want = K.mix(K.softmax(want_s), v, ev, heads, kvh, d, cap, start, length, extra)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    fused = b.read(b.attention(b.upload(q), b.upload(k), b.upload(v), heads=heads, kv_heads=kvh, dim=d, start=start,
                               length=length, extra_keys=b.upload(ek), extra_values=b.upload(ev), extra_length=extra))
    np.testing.assert_allclose(fused, want, rtol=1e-5, atol=1e-5)
    positions = np.arange(total, dtype=np.float32)
    sm = b.upload(want_s)
    b.run("latent_mask", (total, heads), sm, b.upload(positions), heads, total, 3, 20)
    np.testing.assert_array_equal(b.read(sm), K.latent_mask(want_s.copy(), positions, heads, total, 3, 20))


@pytest.mark.parametrize("length", [1, 100, 1023, 1024, 4097, 8192])
def test_fused_attention_long_windows(backend, length):
    """Split-key attention at decode shapes of the 1.7 workload (d 128, 16/4 and
    16/8 heads), including a wrapped ring and the full 8192 global window."""
    b, rng = backend, np.random.default_rng(length)
    heads, d = 16, 128
    kvh = 8 if length > 1024 else 4
    cap = max(length, 1024)
    start = (cap - 7) % cap if length < cap else 0
    q = rng.normal(size=(1, heads * d)).astype(np.float32)
    k = rng.normal(size=(cap, kvh * d)).astype(np.float32)
    v = rng.normal(size=(cap, kvh * d)).astype(np.float32)
    got = b.read(b.attention(b.upload(q), b.upload(k), b.upload(v), heads=heads, kv_heads=kvh, dim=d, start=start,
                             length=length))
    want = K.attention(q, k, v, heads, kvh, d, start, length)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_pool_merge_block_means_match_oracle(backend):
    b, rng = backend, np.random.default_rng(14)
    u = rng.normal(size=(6, 48)).astype(np.float32)
    q = rng.normal(size=(3, 48)).astype(np.float32)
    s = b.empty((3, 6))
    b.run("pool_scores", (6, 3), b.upload(u), b.upload(q), s, 6, 3, 48)
    want_s = K.pool_scores(u, q, 6, 3, 48)
    np.testing.assert_allclose(b.read(s), want_s, rtol=1e-5, atol=1e-6)
    p = K.softmax(want_s)
    z, anchors = b.empty((3, 48)), b.empty((3,))
    b.run("pool_mix", (48, 3), b.upload(u), b.upload(p), z, anchors, 6, 3, 48, 100)
    want_z, want_a = K.pool_mix(u, p, 6, 3, 48, 100)
    np.testing.assert_allclose(b.read(z), want_z, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(b.read(anchors), want_a)
    y = b.empty((48,))
    b.run("merge_rows", (48,), b.upload(u[:2]), y, 48, 3.0, 5.0)
    np.testing.assert_allclose(b.read(y), K.merge_rows(u[:2], 48, 3.0, 5.0), rtol=1e-6)
    rows = rng.normal(size=(131, 24)).astype(np.float32)
    bm = b.empty((3, 24))
    b.run("block_means", (24, 3), b.upload(rows), bm, 131, 24, 64)
    np.testing.assert_allclose(b.read(bm), K.block_means(rows, 131, 24, 64), rtol=1e-6, atol=1e-7)


def test_copy_bounds_and_ownership(backend):
    b = backend
    src = b.upload(np.arange(10, dtype=np.float32))
    dst = b.empty((6,))
    b.copy(src, dst, source_offset=4, count=6)
    np.testing.assert_array_equal(b.read(dst), np.arange(4, 10, dtype=np.float32))
    with pytest.raises(ValueError, match="out of bounds"):
        b.copy(src, dst, source_offset=3, count=7, target_offset=1)
    with pytest.raises(ValueError):
        b.empty((0, 3))


# (rows, columns, K) and the FP16-term tile each selects on a 256-CU MI355X:
# K not a multiple of 64 takes the tile that stages its operands through
# registers; otherwise the buffer unit copies them into LDS, in 128 x 256
# tiles of eight waves where those still give a tile per CU (else 128 x 128
# of four), with two LDS stages where the grid has no more tiles than CUs.
GEMM_TILE_CASES = {
    "registers": (200, 300, 1000),
    "lds-128x128-two-stages": (200, 300, 1024),   # 6 tiles
    "lds-128x128-one-stage": (12700, 300, 512),   # 300 tiles of 128 x 128, 200 of 128 x 256
    "lds-128x256-two-stages": (4096, 2000, 512),  # 256 tiles
    "lds-128x256-one-stage": (4100, 3072, 512),   # 396 tiles
}


@pytest.mark.parametrize("case", list(GEMM_TILE_CASES))
def test_prefill_gemm_term_schemes(backend, case):
    """The batched-prefill MFMA GEMM in both term schemes against a float64
    product, on rows that stress FP16's range: ordinary values, a row far above
    FP16's maximum (6.5e4), a row of tiny values (1e-20), a zero row and a row
    mixing magnitudes 1e4 .. 1e-4; BF16 weights of magnitudes 2^-20 .. 8 with
    a few zeros.  Bound per element: 2^-20 * sum_k |a| |w| (FP32 accumulation
    of up to about 1000 products of operands carried to 2^-22 or better); the
    FP16 scheme's row and matrix scales are powers of two, so they add no
    error.  The shapes take each form of the FP16-term tile (GEMM_TILE_CASES),
    with partial tiles in rows or columns."""
    from miracle_hip.weights import BF16Array, bf16_bits
    b, rng = backend, np.random.default_rng(21)
    m, n, k = GEMM_TILE_CASES[case]
    a = rng.normal(size=(m, k)).astype(np.float32)
    a[1] *= 3.0e6
    a[2] *= 1.0e-20
    a[3] = 0.0
    a[4] *= np.exp(rng.uniform(np.log(1e-4), np.log(1e4), size=k)).astype(np.float32)
    w = rng.normal(size=(n, k)) * np.exp2(rng.integers(-20, 4, size=(n, k)))
    w[rng.random(size=(n, k)) < 0.01] = 0.0
    bits = bf16_bits(w.astype(np.float32))
    wf = BF16Array(bits)[:].astype(np.float64)
    want = a.astype(np.float64) @ wf.T
    bound = 2.0 ** -20 * (np.abs(a).astype(np.float64) @ np.abs(wf).T) + 1e-38
    dev_a, dev_w = b.upload(a), b.upload_weight(BF16Array(bits))
    for scheme in (0, 1):
        got = b.read(b.debug_gemm(dev_a, dev_w, scheme)).astype(np.float64)
        assert np.all(np.isfinite(got)), scheme
        assert np.all(got[3] == 0.0), scheme
        worst = np.max(np.abs(got - want) / bound)
        print("scheme", scheme, "worst error / bound", worst, flush=True)
        assert worst <= 1.0, scheme


@pytest.mark.parametrize("swiglu", [False, True])
def test_grouped_gemm_groups_against_float64(backend, swiglu):
    """The batched prefill's grouped (expert) GEMM in FP16 terms against float64
    per group: groups of 130, 0, 1, 257, 0 and 64 rows (empty groups, a single
    row, partial 128-row tiles), each with its own BF16 weights of its own
    magnitude (so its own power-of-two FP16 scale), K = 1024; 384 output
    columns (a partial 256-column tile), or 192 SwiGLU columns.  Bound per
    element as in the plain GEMM's test: 2^-20 sum_k |a| |w| for each product
    (the SwiGLU of the two products checked against their float64 SwiGLU
    with the bound carried through its derivative).  The kernel over the
    groups' own row tiles and the one over max(counts) rows in every group
    give the same bits."""
    from miracle_hip.weights import BF16Array, bf16_bits
    b, rng = backend, np.random.default_rng(33)
    counts = [130, 0, 1, 257, 0, 64]
    k, n = 1024, (192 if swiglu else 384)
    rows = sum(counts)
    a = rng.normal(size=(rows, k)).astype(np.float32)
    a[5] *= 3.0e4
    a[140] = 0.0

    def weights():
        w = np.concatenate([rng.normal(size=(n, k)) * 2.0 ** rng.integers(-12, 6) for _ in counts])
        bits = bf16_bits(w.astype(np.float32))
        return bits, BF16Array(bits)[:].astype(np.float64)

    bits, wf = weights()
    bits2, wf2 = weights() if swiglu else (None, None)
    want = np.zeros((rows, n))
    bound = np.zeros((rows, n))
    r0 = 0
    for z, cnt in enumerate(counts):
        sl = slice(r0, r0 + cnt)
        wz = wf[z * n:(z + 1) * n]
        g = a[sl].astype(np.float64) @ wz.T
        eg = 2.0 ** -20 * (np.abs(a[sl]).astype(np.float64) @ np.abs(wz).T)
        if swiglu:
            uz = wf2[z * n:(z + 1) * n]
            u = a[sl].astype(np.float64) @ uz.T
            eu = 2.0 ** -20 * (np.abs(a[sl]).astype(np.float64) @ np.abs(uz).T)
            e = np.exp(-np.abs(g))   # the logistic function without overflow, accurate in both tails
            sig = np.where(g >= 0.0, 1.0 / (1.0 + e), e / (1.0 + e))
            silu = g * sig
            dsilu = np.abs(sig * (1.0 + g * (1.0 - sig)))
            want[sl] = silu * u
            # first-order error of silu(g) u, plus FP32 rounding of the epilogue
            bound[sl] = dsilu * eg * np.abs(u) + np.abs(silu) * eu + 1e-6 * np.abs(silu * u)
        else:
            want[sl] = g
            bound[sl] = eg
        r0 += cnt
    bound += 1e-30
    dev_a = b.upload(a)
    dev_w = b.upload_weight(BF16Array(bits))
    dev_w2 = b.upload_weight(BF16Array(bits2)) if swiglu else None
    got = b.read(b.debug_gemm_grouped(dev_a, dev_w, counts, weight2=dev_w2, tile_list=True))
    ref = b.read(b.debug_gemm_grouped(dev_a, dev_w, counts, weight2=dev_w2, tile_list=False))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.all(got[140] == 0.0)
    worst = np.max(np.abs(got.astype(np.float64) - want) / bound)
    print("grouped", "swiglu" if swiglu else "store", "worst error / bound", worst, flush=True)
    assert worst <= 1.0


@pytest.mark.parametrize("presplit", [False, True])
@pytest.mark.parametrize("dim", [32, 64, 128])
def test_prefill_attention_term_scaling(backend, dim, presplit):
    """The batched-prefill attention (FP16-term matrix-core form for head dims
    32/64/128) against float64 on inputs outside FP16's range: values of
    kv head 0 up to ~1e6, keys of kv head 1 times 1e6 with their queries times
    1e-6 (moderate scores), and queries of head 0 times 1e-20 (uniform
    weights).  70 rows from position 50, the earlier keys from the ring, a
    64-key window, 4 query heads over 2 kv heads; the keys and values split
    per tile by the workgroups or once beforehand (per-head scales).  Bound
    per element: 2e-5 max |v| of the kv head over the rows attended (the terms
    carry 22 significant bits of the scale's range)."""
    b, rng = backend, np.random.default_rng(dim)
    heads, kvh, rows, p0, win = 4, 2, 70, 50, 64
    cap = win

    def fill(n):
        x = rng.normal(size=(n, heads + 2 * kvh, dim))
        x[:, heads + kvh + 0] *= np.where(rng.random(size=dim) < 0.5, 3e5, 1.0)   # values, kv head 0
        x[:, heads + 1] *= 1e6                                                     # keys, kv head 1
        x[:, 2:4] *= 1e-6                                                          # its queries
        x[:, 0] *= 1e-20                                                           # queries of head 0
        return x.astype(np.float32)

    chunk, old = fill(rows), fill(cap)
    ring_k = old[:, heads:heads + kvh].reshape(cap, kvh * dim)
    ring_v = old[:, heads + kvh:].reshape(cap, kvh * dim)
    got = b.read(b.debug_prefill_attention(b.upload(chunk.reshape(rows, -1)), b.upload(ring_k), b.upload(ring_v),
                                           p0=p0, heads=heads, kv_heads=kvh, dim=dim, window=win,
                                           presplit=presplit))
    got = got.reshape(rows, heads, dim).astype(np.float64)
    for t in range(rows):
        p = p0 + t
        pos = np.arange(max(0, p - win + 1), p + 1)
        src = [old[q % cap] if q < p0 else chunk[q - p0] for q in pos]
        keys = np.stack([s[heads:heads + kvh] for s in src]).astype(np.float64)
        vals = np.stack([s[heads + kvh:] for s in src]).astype(np.float64)
        for h in range(heads):
            kv = h // (heads // kvh)
            s = keys[:, kv] @ chunk[t, h].astype(np.float64) / np.sqrt(dim)
            w = np.exp(s - s.max())
            want = (w / w.sum()) @ vals[:, kv]
            bound = 2e-5 * np.abs(vals[:, kv]).max()
            assert np.all(np.abs(got[t, h] - want) <= bound), (t, h, np.abs(got[t, h] - want).max() / bound)


@pytest.mark.parametrize("dim", [32, 64, 128])
def test_prefill_attention_wide_chunk(backend, dim):
    """The presplit attention on a chunk wide enough for its two-row-set form
    (each wave two sets of 16 query rows; taken at 512 workgroups or more):
    2048 rows from position 300, 32 query heads over 8 kv heads, a 256-key
    window reaching into the ring, against float64.  Bound per element: 2e-5
    max |v| of the kv head."""
    b, rng = backend, np.random.default_rng(100 + dim)
    heads, kvh, rows, p0, win = 32, 8, 2048, 300, 256
    cap = win
    chunk = rng.normal(size=(rows, heads + 2 * kvh, dim)).astype(np.float32)
    old = rng.normal(size=(cap, heads + 2 * kvh, dim)).astype(np.float32)
    ring_k = old[:, heads:heads + kvh].reshape(cap, kvh * dim)
    ring_v = old[:, heads + kvh:].reshape(cap, kvh * dim)
    got = b.read(b.debug_prefill_attention(b.upload(chunk.reshape(rows, -1)), b.upload(ring_k), b.upload(ring_v),
                                           p0=p0, heads=heads, kv_heads=kvh, dim=dim, window=win, presplit=True))
    got = got.reshape(rows, heads, dim).astype(np.float64)
    first = p0 - win + 1
    pos = np.arange(first, p0 + rows)
    src = np.stack([old[q % cap] if q < p0 else chunk[q - p0] for q in pos]).astype(np.float64)
    qpos = p0 + np.arange(rows)
    seen = (pos[None, :] <= qpos[:, None]) & (pos[None, :] > qpos[:, None] - win)
    for h in range(heads):
        kv = h // (heads // kvh)
        s = chunk[:, h].astype(np.float64) @ src[:, heads + kv].T / np.sqrt(dim)
        s = np.where(seen, s, -np.inf)
        w = np.exp(s - s.max(axis=1, keepdims=True))
        want = (w / w.sum(axis=1, keepdims=True)) @ src[:, heads + kvh + kv]
        bound = 2e-5 * np.abs(src[:, heads + kvh + kv]).max()
        err = np.abs(got[:, h] - want)
        assert np.all(err <= bound), (h, err.max() / bound)


def test_softmax_exponentials_error_bound(backend, record_property):
    """The batched prefill's softmax weights come from the hardware exp2 (log2 e
    folded into the score scale), the token step's from expf.  Over the
    arguments a softmax produces after its maximum is subtracted (x <= 0,
    down to where the result leaves FP32's normal range: 2^x for x in
    [-125, 0], e^x for x in [-87, 0]), both against float64: the largest
    relative error is recorded and bounded by 2 ulp of FP32 (2^-22)."""
    b = backend
    errs = {}
    for which, name, ref, lo in ((0, "exp2_hw", np.exp2, 125.0), (1, "expf", np.exp, 87.0)):
        x = np.concatenate([-np.linspace(0.0, lo, 1 << 20), -np.abs(np.random.default_rng(5).normal(size=1 << 16)),
                            np.float32([0.0, -1e-30, -0.5, -1.0])]).astype(np.float32)
        got = b.read(b.debug_exp(b.upload(x), which)).astype(np.float64)
        want = ref(x.astype(np.float64))
        rel = np.abs(got - want) / want
        errs[name] = float(rel.max())
        print(f"{name}: max relative error {errs[name]:.3e} ({errs[name] / 2.0 ** -23:.2f} ulp)", flush=True)
        record_property(f"{name}_max_rel_error", errs[name])
        assert errs[name] <= 2.0 ** -22, name
