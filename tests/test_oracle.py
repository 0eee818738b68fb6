"""Pins the CPU oracle (oracle/cam_oracle.c) before it is trusted as the checker.

Each function is checked against something independent of its own formula:
the committed golden vectors (library routines, tests/golden/make_golden.py),
brute force on tiny inputs, torch's float8_e4m3fn / bfloat16 casts, numpy's
stable sort, IEEE fp32 arithmetic in numpy, and the reference's closed forms
(identity experts: out = x * sum(w), test_moe_dispatch_combine_prefill.py:163-168;
round-robin expert ids, test_fused_deep_moe.py:298-302).
"""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def gold(name):
    return dict(np.load(os.path.join(GOLD, name), allow_pickle=False))


# ------------------------------------------------------------------ numerics

def _fp8_probe_values():
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    codes = codes[torch.isfinite(codes)]
    s = torch.sort(codes).values
    mids = (s[1:] + s[:-1]) / 2
    up = torch.nextafter(mids, torch.full_like(mids, 1e9))
    dn = torch.nextafter(mids, torch.full_like(mids, -1e9))
    g = torch.Generator().manual_seed(0)
    rnd = torch.randn(4000, generator=g) * torch.exp2(torch.randint(-14, 9, (4000,), generator=g).float())
    return torch.cat([codes, mids, up, dn, rnd.clamp(-448, 448), torch.tensor([0.0, -0.0, 1e-30, 448.0])])


def test_e4m3_encode_matches_torch_cast():
    vals = _fp8_probe_values()
    ref = vals.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([orc.f32_to_e4m3(v) for v in vals.tolist()], np.uint8)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, [(vals[i].item(), got[i], ref[i]) for i in bad[:10]]


def test_e4m3_saturates_above_max():
    # OCP e4m3fn has no infinity; the quantiser saturates to +-448 (0x7e / 0xfe)
    assert orc.f32_to_e4m3(448.0) == 0x7E
    assert orc.f32_to_e4m3(1e6) == 0x7E
    assert orc.f32_to_e4m3(-1e6) == 0xFE
    assert orc.f32_to_e4m3(-0.0) == 0x80


def test_e4m3_decode_matches_torch():
    tab = orc.e4m3_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(tab), np.isnan(ref))
    assert np.array_equal(tab[fin].view(np.uint32), ref[fin].view(np.uint32))


def test_bf16_rne_matches_torch():
    g = torch.Generator().manual_seed(1)
    f = torch.randn(20000, generator=g) * torch.exp2(torch.randint(-30, 30, (20000,), generator=g).float())
    ref = f.bfloat16().view(torch.int16).numpy().view(np.uint16)
    got = np.array([orc.lib().orc_f32_to_bf16(v) for v in f.tolist()], np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(orc.f32_to_bf16(f.numpy()), ref)


# ------------------------------------------------------------------ R0

@pytest.mark.parametrize("name", ["cfg1_tiny.npz", "skew_bias.npz"])
def test_route_matches_golden(name):
    d = gold(name)
    K = d["idx"].shape[1]
    idx, w = orc.route(d["logits"], d.get("bias"), K)
    assert np.array_equal(idx, d["idx"])
    np.testing.assert_allclose(w, d["w"], rtol=2e-6, atol=1e-7)


def test_route_ties_and_bruteforce():
    rng = np.random.default_rng(5)
    # heavy ties: logits from a tiny integer grid
    logits = rng.integers(-2, 3, size=(40, 12)).astype(np.float32)
    bias = rng.integers(0, 2, size=12).astype(np.float32)
    K = 4
    idx, w = orc.route(logits, bias, K)
    for t in range(40):
        s = logits[t] + bias
        # brute force: ordered by descending score, then ascending index
        exp_order = sorted(range(12), key=lambda e: (-s[e], e))[:K]
        assert list(idx[t]) == exp_order
        ex = np.exp(logits[t] - logits[t].max())
        ref = ex[exp_order] / ex[exp_order].sum()
        np.testing.assert_allclose(w[t], ref, rtol=2e-6)
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)


# ------------------------------------------------------------------ D1 / D2

@pytest.mark.parametrize("name", ["cfg1_tiny.npz", "skew_bias.npz"])
def test_layout_matches_golden(name):
    d = gold(name)
    E = d["logits"].shape[1]
    ntr, nte, itr, sti = orc.dispatch_layout(d["idx"].astype(np.int64), E, 1)
    assert np.array_equal(nte, d["counts"])
    assert np.array_equal(sti, d["send_token_idx"])
    assert ntr[0] == d["idx"].shape[0] and itr.all()


def test_layout_round_robin_closed_form():
    d = gold("round_robin.npz")
    _, nte, _, sti = orc.dispatch_layout(d["idx"], 16, 1)
    assert np.array_equal(nte, d["counts"])
    # round robin: flat entry i goes to expert i % E with rank i // E
    flat = np.arange(d["idx"].size)
    assert np.array_equal(sti.reshape(-1), flat // 16)


def test_layout_multi_rank_and_invalid_ids():
    rng = np.random.default_rng(3)
    T, K, E, R = 50, 6, 32, 4
    ids = rng.integers(-1, E, size=(T, K)).astype(np.int64)  # -1: not routed
    ntr, nte, itr, sti = orc.dispatch_layout(ids, E, R)
    assert (sti[ids < 0] == -1).all()
    for e in range(E):
        pos = np.argwhere(ids.reshape(-1) == e).reshape(-1)
        assert nte[e] == pos.size
        assert np.array_equal(sti.reshape(-1)[pos], np.arange(pos.size))
    for t in range(T):
        ranks = {int(e) // (E // R) for e in ids[t] if e >= 0}
        assert set(np.nonzero(itr[t])[0].tolist()) == ranks
    assert np.array_equal(ntr, itr.sum(0))


def test_notify_prefix():
    c = np.array([3, 0, 5, 1, 0, 7], np.int32)
    so, rc, rtpe, tot = orc.notify_dispatch(c)
    assert list(so) == [0, 3, 3, 8, 9, 9]
    assert list(rc) == [3, 3, 8, 9, 9, 16]
    assert list(rtpe) == list(c) and rtpe.dtype == np.int64 and tot == 16


# ------------------------------------------------------------------ D3 / Q

def _dispatch_from_gold(d, mode):
    E = d["logits"].shape[1]
    so, _, _, _ = orc.notify_dispatch(d["counts"])
    return orc.dispatch(d["x"], d["idx"], so, d["send_token_idx"], E, mode)


@pytest.mark.parametrize("name", ["cfg1_tiny.npz", "skew_bias.npz"])
def test_dispatch_fp8_matches_golden(name):
    d = gold(name)
    ex, sc, eidx = _dispatch_from_gold(d, orc.QUANT_FP8)
    T, K = d["idx"].shape
    rows = d["row_of"].reshape(-1)
    t_of = np.repeat(np.arange(T), K)
    k_of = np.tile(np.arange(K), T)
    assert np.array_equal(ex[rows], d["fp8_codes"][t_of])
    assert np.array_equal(sc[rows].view(np.uint32), d["fp8_scales"][t_of].view(np.uint32))
    assert np.array_equal(eidx[rows], np.stack([np.zeros_like(t_of), t_of, k_of], 1))


def test_dispatch_int8_and_bf16_match_golden():
    d = gold("cfg1_tiny.npz")
    T, K = d["idx"].shape
    rows = d["row_of"].reshape(-1)
    t_of = np.repeat(np.arange(T), K)
    ex, sc, _ = _dispatch_from_gold(d, orc.QUANT_INT8)
    assert np.array_equal(ex[rows], d["int8_codes"][t_of])
    np.testing.assert_array_equal(sc[rows], d["int8_scales"][t_of])
    ex, _, _ = _dispatch_from_gold(d, orc.QUANT_NONE)
    assert np.array_equal(ex[rows], d["x"][t_of])


def test_dispatch_rows_sorted_stable_bijection():
    d = gold("skew_bias.npz")
    _, _, eidx = _dispatch_from_gold(d, orc.QUANT_NONE)
    T, K = d["idx"].shape
    experts = d["idx"][eidx[:, 1], eidx[:, 2]]
    assert (np.diff(experts) >= 0).all()                       # sorted by expert
    flat = eidx[:, 1] * K + eidx[:, 2]
    same = np.diff(experts) == 0
    assert (np.diff(flat)[same] > 0).all()                     # stable within expert
    assert np.array_equal(np.sort(flat), np.arange(T * K))     # bijection


def test_fp8_zero_block_and_saturation():
    H = 256
    x = np.zeros((2, H), np.float32)
    x[1, :128] = np.linspace(-3, 3, 128)
    x[1, 128:] = 1e-6                       # amax below the 1e-4 clamp
    xb = orc.f32_to_bf16(x)
    ids = np.zeros((2, 1), np.int32)
    ex, sc, _ = orc.dispatch(xb, ids, np.zeros(1, np.int32), np.array([[0], [1]], np.int32), 1, orc.QUANT_FP8)
    assert (ex[0] == 0).all() and np.allclose(sc[0], 1e-4 / 448)
    assert ex[1, 0] == 0xFE and ex[1, 127] == 0x7E           # +-amax -> +-448
    assert sc[1, 0] == np.float32(np.float32(orc.bf16_to_f32(xb[1, 0:1]))[0] * -1) / np.float32(448.0)


# ------------------------------------------------------------------ C1

def test_combine_identity_closed_form():
    d = gold("cfg1_tiny.npz")
    E = d["logits"].shape[1]
    ex, _, eidx = _dispatch_from_gold(d, orc.QUANT_NONE)
    out = orc.combine(ex, eidx, d["idx"], d["w"], E)
    got = orc.bf16_to_f32(out)
    ref = orc.bf16_to_f32(d["ident_out"])
    # one bf16 ulp from rounding the fp32 sum twice at most
    np.testing.assert_allclose(got, ref, rtol=2 ** -7, atol=1e-6)


def test_combine_fp32_sequence_bit_exact():
    # numpy float32 ops are IEEE single: mul then add in k order, then RNE to bf16
    rng = np.random.default_rng(9)
    T, K, H, E = 12, 4, 64, 8
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    ids[3, 1] = -1                                     # placeholder slot: skipped
    w = rng.random((T, K)).astype(np.float32)
    _, nte, _, sti = orc.dispatch_layout(ids.astype(np.int64), E, 1)
    so, _, _, _ = orc.notify_dispatch(nte)
    y = orc.f32_to_bf16(rng.standard_normal((int(nte.sum()), H)).astype(np.float32))
    eidx = np.zeros((int(nte.sum()), 3), np.int32)
    for t in range(T):
        for k in range(K):
            if ids[t, k] >= 0:
                eidx[so[ids[t, k]] + sti[t, k]] = (0, t, k)
    out = orc.combine(y, eidx, ids, w, E)
    yf = orc.bf16_to_f32(y)
    ref = np.zeros((T, H), np.float32)
    for t in range(T):
        acc = np.zeros(H, np.float32)
        for k in range(K):
            if ids[t, k] < 0:
                continue
            acc = acc + yf[so[ids[t, k]] + sti[t, k]] * w[t, k]
        ref[t] = acc
    assert np.array_equal(out, orc.f32_to_bf16(ref))


# ------------------------------------------------------------------ G1..G3

def test_gemm_bf16_matches_golden():
    d = gold("gemm_bf16_small.npz")
    h = orc.gmm1_swiglu_bf16(d["A"], d["counts"], d["W1"])
    hf, hr = orc.bf16_to_f32(h), orc.bf16_to_f32(d["h"])
    # both round the same double-accumulated value; differences come only
    # from silu's exp in float vs double (a bf16 ulp at most)
    np.testing.assert_allclose(hf, hr, rtol=2 ** -7, atol=1e-6)
    out = orc.gmm2_bf16(d["h"], d["counts"], d["W2"])
    np.testing.assert_allclose(orc.bf16_to_f32(out), orc.bf16_to_f32(d["out"]), rtol=2 ** -7, atol=1e-6)


def test_gemm_fp8_matches_float64_dequant():
    rng = np.random.default_rng(4)
    Ms, H, I = [3, 0, 7], 256, 128
    L, M = len(Ms), sum(Ms)
    tab = orc.e4m3_table()
    finite = np.nonzero(np.isfinite(tab))[0].astype(np.uint8)
    A = rng.choice(finite, size=(M, H))
    As = rng.uniform(0.01, 0.1, size=(M, H // 128)).astype(np.float32)
    W1 = rng.choice(finite, size=(L, 2 * I, H))
    W1s = rng.uniform(1e-4, 1e-3, size=(L, 2 * I // 128, H // 128)).astype(np.float32)
    W2 = rng.choice(finite, size=(L, H, I))
    W2s = rng.uniform(1e-4, 1e-3, size=(L, H // 128, I // 128)).astype(np.float32)
    hq, hs = orc.gmm1_swiglu_fp8(A, As, np.array(Ms), W1, W1s)
    out = orc.gmm2_fp8(hq, hs, np.array(Ms), W2, W2s)
    off = 0
    for e, m in enumerate(Ms):
        if m == 0:
            continue
        a = tab[A[off:off + m]].astype(np.float64) * np.repeat(As[off:off + m], 128, axis=1)
        w1 = tab[W1[e]].astype(np.float64) * np.kron(W1s[e], np.ones((128, 128)))
        gu = a @ w1.T
        g, u = gu[:, :I], gu[:, I:]
        h = g / (1 + np.exp(-g)) * u
        hd = tab[hq[off:off + m]] * np.repeat(hs[off:off + m], 128, axis=1)
        # fp8 requant of h: relative error per element <= 2^-4 of its block amax
        amax = np.repeat(np.abs(h).reshape(m, -1, 128).max(2), 128, axis=1)
        assert (np.abs(hd - h) <= amax * 2 ** -4 + 1e-30).all()
        w2 = tab[W2[e]].astype(np.float64) * np.kron(W2s[e], np.ones((128, 128)))
        o = hd.astype(np.float64) @ w2.T
        got = orc.bf16_to_f32(out[off:off + m])
        np.testing.assert_allclose(got, o, rtol=2 ** -7, atol=1e-6 * np.abs(o).max())
        off += m
