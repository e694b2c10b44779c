"""Pins the oracle's kernel restatement (oracle/kernels.c).

Closed forms restated from the reference's kernel tests
(tests/test_opencl.py:19-80 of the reference), brute force on small shapes for
the kernels those tests leave open, and checks that would fail on the plausible
mistakes (lane order of ``linear``, dropped tail, wrong ring index, wrong
half-pairing, wrong group mapping, anchors rounding).
"""
import numpy as np
import pytest

from oracle import kernels as K


def test_linear_rms_softmax_closed_forms_non_aligned():
    # reference tests/test_opencl.py:19-30
    rng = np.random.default_rng(9)
    x = rng.normal(size=(3, 19)).astype(np.float32)
    w = rng.normal(size=(7, 19)).astype(np.float32)
    np.testing.assert_allclose(K.linear(x, w), x @ w.T, atol=4e-6)
    g = rng.normal(size=19).astype(np.float32)
    expected = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-6) * g
    np.testing.assert_allclose(K.rms(x, g, 19, 1e-6), expected, atol=1e-6)
    logits = np.array([[1000, 1001, -1000], [-1000, -1001, -1002]], np.float32)
    e = np.exp(logits - logits.max(axis=1, keepdims=True))
    np.testing.assert_allclose(K.softmax(logits), e / e.sum(axis=1, keepdims=True), atol=1e-7)


def test_linear_lane_order_is_exact():
    """Four stride-4 lane sums folded ((l0+l1)+l2)+l3, then the tail; each
    product rounded before the add (no FMA). Checked bit for bit."""
    rng = np.random.default_rng(1)
    for n in (1, 3, 4, 7, 19, 64, 130):
        x = rng.normal(size=(2, n)).astype(np.float32)
        w = rng.normal(size=(5, n)).astype(np.float32)
        want = np.empty((2, 5), np.float32)
        for r in range(2):
            for o in range(5):
                lanes = [np.float32(0)] * 4
                full = n - n % 4
                for j in range(0, full, 4):
                    for l in range(4):
                        lanes[l] = np.float32(lanes[l] + np.float32(x[r, j + l] * w[o, j + l]))
                v = np.float32(np.float32(np.float32(lanes[0] + lanes[1]) + lanes[2]) + lanes[3])
                for j in range(full, n):
                    v = np.float32(v + np.float32(x[r, j] * w[o, j]))
                want[r, o] = v
        np.testing.assert_array_equal(K.linear(x, w), want)


def test_linear_bf16_equals_widened():
    rng = np.random.default_rng(2)
    w = rng.normal(size=(9, 37)).astype(np.float32)
    bits = (w.view(np.uint32) >> 16).astype(np.uint16)
    widened = (bits.astype(np.uint32) << 16).view(np.float32)
    x = rng.normal(size=(3, 37)).astype(np.float32)
    np.testing.assert_array_equal(K.linear(x, bits), K.linear(x, widened))


def test_rms_non_affine_and_order():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(4, 8)).astype(np.float32)
    y = K.rms(x, None, 8, 1e-5)
    for r in range(4):
        v = np.float32(0)
        for a in x[r]:
            v = np.float32(v + np.float32(a * a))
        scale = np.float32(1) / np.sqrt(np.float32(v / np.float32(8) + np.float32(1e-5)))
        np.testing.assert_array_equal(y[r], (x[r] * scale).astype(np.float32))


@pytest.mark.parametrize("split", [False, True])
def test_rope_layouts(split):
    # reference tests/test_opencl.py:33-44
    rng = np.random.default_rng(3)
    x = rng.normal(size=(2, 3, 6)).astype(np.float32)
    pos = np.array([7, 29], np.float32)
    freq = np.array([1, .1, .01], np.float32)
    ang = pos[:, None, None] * freq[None, None, :]
    a, b = (x[..., :3], x[..., 3:]) if split else (x[..., ::2], x[..., 1::2])
    u, v = a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)
    want = np.concatenate([u, v], axis=-1) if split else np.stack([u, v], axis=-1).reshape(2, 3, 6)
    got = K.rope(x.reshape(2, 18), freq, pos, 3, 6, split)
    np.testing.assert_allclose(got.reshape(x.shape), want, atol=3e-6)


def test_rope_large_angles_accurate():
    """Angles up to ~1e4 rad (position x frequency); cos/sin must be accurate
    there, not just near zero."""
    pos = np.array([8191], np.float32)
    freq = np.array([1.0, 0.731, 0.05], np.float32)
    x = np.ones((1, 6), np.float32)
    got = K.rope(x, freq, pos, 1, 6, True)
    ang = (pos[0] * freq).astype(np.float32).astype(np.float64)
    want = np.concatenate([np.cos(ang) - np.sin(ang), np.sin(ang) + np.cos(ang)]).astype(np.float32)
    np.testing.assert_allclose(got[0], want, atol=2e-7)


def test_attention_group_mapping_ring_and_extra_rows():
    # reference tests/test_opencl.py:47-63
    rng = np.random.default_rng(6)
    q = rng.normal(size=(4, 6)).astype(np.float32)
    k, v = [rng.normal(size=(5, 2, 6)).astype(np.float32) for _ in range(2)]
    rk, rv = [rng.normal(size=(3, 2, 6)).astype(np.float32) for _ in range(2)]
    keys, values = np.concatenate([k[[3, 4, 0, 1]], rk]), np.concatenate([v[[3, 4, 0, 1]], rv])
    want = []
    for h in range(4):
        logits = keys[:, h // 2] @ q[h] / np.sqrt(6)
        p = np.exp(logits - logits.max())
        want.append((p / p.sum()) @ values[:, h // 2])
    got = K.attention(q.reshape(1, -1), k.reshape(5, -1), v.reshape(5, -1), 4, 2, 6, 3, 4,
                      rk.reshape(3, -1), rv.reshape(3, -1), 3)
    np.testing.assert_allclose(got.reshape(4, 6), want, atol=1e-6)


def test_swiglu_axpy_brute_force():
    g = np.array([-3.0, -0.5, 0.0, 0.25, 4.0], np.float32)
    u = np.array([1.0, 2.0, 3.0, -1.0, 0.5], np.float32)
    want = (g / (1 + np.exp(-g.astype(np.float64)))) * u
    np.testing.assert_allclose(K.swiglu(g, u), want, rtol=1e-6)
    x = np.arange(5, dtype=np.float32)
    np.testing.assert_array_equal(K.axpy(x, u, 0.5), (x + np.float32(0.5) * u).astype(np.float32))


def test_latent_mask_only_non_memory_old_rows():
    s = np.zeros((2, 5), np.float32)
    pos = np.array([0, 1, 2, 6, 7], np.float32)
    K.latent_mask(s, pos, 2, 5, 1, 3)   # rows >= 1 with position < 3 are masked
    want = np.zeros((2, 5), np.float32)
    want[:, 1:3] = -np.inf
    np.testing.assert_array_equal(s, want)


def test_pool_scores_mix_brute_force():
    rng = np.random.default_rng(5)
    u = rng.normal(size=(3, 8)).astype(np.float32)
    q = rng.normal(size=(2, 8)).astype(np.float32)
    s = K.pool_scores(u, q, 3, 2, 8)
    np.testing.assert_allclose(s, (q @ u.T) / np.sqrt(8), atol=1e-6)
    p = K.softmax(s)
    z, anchors = K.pool_mix(u, p, 3, 2, 8, 10)
    np.testing.assert_allclose(z, p @ u, atol=1e-6)
    np.testing.assert_array_equal(anchors, np.rint(p @ np.array([10, 11, 12], np.float32)))
    # ties round to even: weight 0.5/0.5 over positions 10 and 11 -> 10.5 -> 10
    z, anchors = K.pool_mix(u[:2], np.array([[0.5, 0.5]], np.float32), 2, 1, 8, 10)
    assert anchors[0] == 10.0


def test_merge_rows_and_block_means():
    x = np.array([[1, 2, 3], [5, 6, 7]], np.float32)
    np.testing.assert_allclose(K.merge_rows(x, 3, 3.0, 1.0), (3 * x[0] + x[1]) / 4)
    rows = np.arange(14, dtype=np.float32).reshape(7, 2)
    got = K.block_means(rows, 7, 2, 3)     # blocks [0,3), [3,6), [6,7) (partial)
    want = np.stack([rows[0:3].mean(0), rows[3:6].mean(0), rows[6:7].mean(0)])
    np.testing.assert_allclose(got, want)
