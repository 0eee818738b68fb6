"""Pins the oracle's int8 W8A8 functions (the reference's own fused numerics).

Checks are independent of the C formulas: numpy int64 matmuls for the exact
integer sums, float64 closed forms for the SwiGLU, invariants of the per-token
quantiser (|q| reaches 127 at the row maximum, dequantisation error within half
a step), and the closed form of the reference test's shared-expert weights
(all entries +-4, the sign alternating by column, test_fused_deep_moe.py:321-326).
"""
import numpy as np

from oracle import oracle as orc


def _rng(seed):
    return np.random.default_rng(seed)


def _w_int8(rng, shape):
    # the reference test's weight recipe: randint(-16, 16) int8 (test_fused_deep_moe.py:303-308)
    return rng.integers(-16, 16, shape).astype(np.int8)


def _ch_scale(rng, shape):
    return (rng.random(shape) * 0.003 + 0.0015).astype(np.float32)   # test_fused_deep_moe.py:309-312


def test_gmm1_int8_matches_int64_matmul_and_float64_swiglu():
    rng = _rng(1)
    counts = np.array([3, 0, 5, 1], np.int64)
    L, H, I = 4, 256, 128
    M = int(counts.sum())
    A = rng.integers(-127, 128, (M, H)).astype(np.int8)
    As = (rng.random(M) * 0.05).astype(np.float32)
    W1 = _w_int8(rng, (L, 2 * I, H))
    W1s = _ch_scale(rng, (L, 2 * I))
    h = orc.gmm1_swiglu_int8(A, As, counts, W1, W1s)
    off = np.concatenate([[0], np.cumsum(counts)])
    for e in range(L):
        rows = slice(off[e], off[e + 1])
        acc = A[rows].astype(np.int64) @ W1[e].T.astype(np.int64)          # exact
        v = acc.astype(np.float64) * W1s[e].astype(np.float64) * As[rows, None].astype(np.float64)
        g, u = v[:, :I], v[:, I:]
        ref = g / (1 + np.exp(-g)) * u                                       # left half is the gate
        if ref.size:
            np.testing.assert_allclose(h[rows], ref, rtol=2e-5, atol=1e-6 * np.abs(ref).max())


def test_gmm1_int8_gate_is_left_half():
    # up rows zero -> h == 0 whatever the gate; gate rows zero -> silu(0) = 0 -> h == 0
    rng = _rng(2)
    A = rng.integers(-127, 128, (4, 128)).astype(np.int8)
    As = np.ones(4, np.float32)
    W1 = _w_int8(rng, (1, 256, 128))
    W1s = np.full((1, 256), 1e-3, np.float32)
    up0 = W1.copy()
    up0[0, 128:] = 0
    assert np.all(orc.gmm1_swiglu_int8(A, As, np.array([4]), up0, W1s) == 0)
    g0 = W1.copy()
    g0[0, :128] = 0
    assert np.all(orc.gmm1_swiglu_int8(A, As, np.array([4]), g0, W1s) == 0)
    # swapping the halves changes the result (silu is not symmetric)
    sw = np.concatenate([W1[:, 128:], W1[:, :128]], axis=1)
    assert not np.allclose(orc.gmm1_swiglu_int8(A, As, np.array([4]), W1, W1s),
                           orc.gmm1_swiglu_int8(A, As, np.array([4]), sw, W1s))


def test_quant_rows_int8_invariants():
    rng = _rng(3)
    h = (rng.standard_normal((6, 384)) * np.exp2(rng.integers(-20, 10, (6, 1)))).astype(np.float32)
    h[4] = 0.0
    q, s = orc.quant_rows_int8(h)
    for m in range(6):
        amax = np.abs(h[m]).max()
        if amax == 0:
            assert np.all(q[m] == 0) and s[m] == 0
            continue
        assert np.abs(q[m].astype(int)).max() == 127
        assert q[m][np.abs(h[m]).argmax()] == np.sign(h[m][np.abs(h[m]).argmax()]) * 127
        assert abs(s[m] - amax / 127) <= 1e-6 * amax / 127
        # dequantisation error within half a step (plus the fp32 rounding of the scale)
        assert np.all(np.abs(q[m] * np.float64(s[m]) - h[m]) <= 0.5 * s[m] * (1 + 1e-5))


def test_gmm2_int8_bit_exact_vs_numpy_fp32_sequence():
    rng = _rng(4)
    counts = np.array([2, 7, 0], np.int64)
    L, I, H = 3, 256, 256
    M = int(counts.sum())
    Hq = rng.integers(-127, 128, (M, I)).astype(np.int8)
    Hs = (rng.random(M) * 0.01).astype(np.float32)
    W2 = _w_int8(rng, (L, H, I))
    W2s = _ch_scale(rng, (L, H))
    out = orc.gmm2_int8(Hq, Hs, counts, W2, W2s)
    off = np.concatenate([[0], np.cumsum(counts)])
    for e in range(L):
        rows = slice(off[e], off[e + 1])
        acc = Hq[rows].astype(np.int64) @ W2[e].T.astype(np.int64)
        v = (acc.astype(np.float32) * W2s[e]) * Hs[rows, None]              # fp32, in this order
        assert np.array_equal(out[rows], orc.f32_to_bf16(v))


def test_shared_expert_closed_form():
    # reference shared weights: every entry 4, negated at even output columns; scales 0.0015
    rng = _rng(5)
    T, H, Ish = 5, 256, 128
    A = rng.integers(-127, 128, (T, H)).astype(np.int8)
    As = (rng.random(T) * 0.02).astype(np.float32)
    w1 = np.full((2 * Ish, H), 4, np.int8)
    w1[::2] *= -1                      # [n, k] storage: even output columns are negative
    s1 = np.full((1, 2 * Ish), 0.0015, np.float32)
    h = orc.gmm1_swiglu_int8(A, As, np.array([T]), w1[None], s1)
    S = A.astype(np.int64).sum(1).astype(np.float64)
    base = 4 * S * 0.0015 * As.astype(np.float64)          # value of a positive column
    sign = np.where(np.arange(2 * Ish) % 2 == 0, -1.0, 1.0)
    v = base[:, None] * sign[None, :]
    g, u = v[:, :Ish], v[:, Ish:]
    np.testing.assert_allclose(h, g / (1 + np.exp(-g)) * u, rtol=2e-5, atol=1e-9)


def test_dispatch_int8_fused_recipe():
    rng = _rng(6)
    T, H, K, E = 7, 512, 3, 8
    x = orc.f32_to_bf16((rng.random((T, H)) * 10 - 5).astype(np.float32))
    x[5] = 0                                                # zero row: q = 0, scale 0
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    ids[2, 1] = -1
    _, nte, _, sti = orc.dispatch_layout(ids.astype(np.int64), E, 1)
    so, _, _, _ = orc.notify_dispatch(nte)
    smooth = (rng.random((E, H)) + 0.5).astype(np.float32)
    for sm in (None, smooth):
        q, sc, eidx = orc.dispatch_int8_fused(x, ids, so, sti, E, smooth=sm)
        xf = orc.bf16_to_f32(x)
        for r in range(q.shape[0]):
            t, k = eidx[r, 1], eidx[r, 2]
            f = xf[t] if sm is None else xf[t] * sm[ids[t, k]]          # fp32 products
            amax = np.abs(f).max()
            if amax == 0:
                assert np.all(q[r] == 0) and sc[r] == 0
                continue
            s = np.float32(127.0) / amax
            assert np.array_equal(q[r], np.rint(f * s).astype(np.int8))
            assert sc[r] == np.float32(1.0) / s
            assert np.abs(q[r].astype(int)).max() == 127
    # without smooth scales the K rows of a token are identical
    q, sc, eidx = orc.dispatch_int8_fused(x, ids, so, sti, E)
    for t in range(T):
        rows = np.where(eidx[:, 1] == t)[0]
        assert all(np.array_equal(q[rows[0]], q[r]) for r in rows)
