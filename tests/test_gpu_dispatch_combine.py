"""GPU parity: routing, layout, dispatch (bf16 / int8 / fp8) and combine on
the HIP path vs the CPU oracle, on the same seeded inputs.

Bar: bit-exact for indices, counts, permutation maps, quantised codes and
scales, and the combine output (the combine is specified as an exact fp32
multiply-then-add sequence with RNE to bf16, so it is bit-exact too);
routing gates within 1e-5 relative (expf differs by an ulp between libm and
the GPU).
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import umdk_amd
    return torch.ops.umdk_cam_op_lib


def bits(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.cpu().numpy()


def make_inputs(seed, T, H, E, K, bias_std=0.0, zipf=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).bfloat16()
    logits = torch.randn(T, E, generator=g)
    bias = torch.randn(E, generator=g) * bias_std if bias_std > 0 else None
    return x, logits, bias


def route_both(ops, logits, bias, K):
    idx, w = ops.moe_route(logits.cuda(), None if bias is None else bias.cuda(), K)
    ridx, rw = orc.route(logits.numpy(), None if bias is None else bias.numpy(), K)
    return idx, w, ridx, rw


ROUTE_CASES = [(0, 128, 8, 2, 0.0), (1, 4096, 256, 8, 0.5), (2, 8192, 8, 2, 0.0), (3, 300, 512, 16, 1.0),
               (4, 7, 64, 6, 0.0)]


@pytest.mark.parametrize("seed,T,E,K,bstd", ROUTE_CASES)
def test_route_matches_oracle(ops, seed, T, E, K, bstd):
    print(f"route seed={seed} T={T} E={E} K={K}", flush=True)
    _, logits, bias = make_inputs(seed, 1, 1024, E, K, bstd)
    g = torch.Generator().manual_seed(seed + 100)
    logits = torch.randn(T, E, generator=g)
    idx, w, ridx, rw = route_both(ops, logits, bias, K)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)


def test_route_ties_lower_index(ops):
    rng = np.random.default_rng(7)
    logits = torch.from_numpy(rng.integers(-2, 3, size=(500, 64)).astype(np.float32))
    bias = torch.from_numpy(rng.integers(0, 2, size=64).astype(np.float32))
    idx, w, ridx, rw = route_both(ops, logits, bias, 8)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5)


def _layout_full(topk_idx_i64, E, R):
    """All four layout outputs through the C ABI."""
    from umdk_amd import _lib
    T, K = topk_idx_i64.shape
    dev = topk_idx_i64.device
    ntr = torch.full((R,), -5, dtype=torch.int32, device=dev)
    nte = torch.full((E,), -5, dtype=torch.int32, device=dev)
    itr = torch.full((T, R), -5, dtype=torch.int32, device=dev)
    sti = torch.full((T, K), -5, dtype=torch.int32, device=dev)
    _lib.call("camhipDispatchLayout", _lib.ptr(topk_idx_i64), T, R, E, K, _lib.ptr(ntr), _lib.ptr(nte), _lib.ptr(itr),
              _lib.ptr(sti), device=dev)
    return ntr, nte, itr, sti


LAYOUT_CASES = [(128, 2, 8, 1), (4096, 8, 256, 1), (4096, 8, 256, 8), (8192, 2, 8, 1), (1000, 6, 32, 4),
                (8000, 16, 384, 384), (8000, 16, 512, 128), (1, 1, 1, 1), (3, 16, 512, 2)]


@pytest.mark.parametrize("T,K,E,R", LAYOUT_CASES)
def test_layout_matches_oracle(ops, T, K, E, R):
    print(f"layout T={T} K={K} E={E} R={R}", flush=True)
    rng = np.random.default_rng(T * 31 + K)
    # skewed, with repeated experts within a token and some -1 placeholders
    p = rng.zipf(1.3, size=(T, K)) % E
    ids = p.astype(np.int64)
    ids[rng.random((T, K)) < 0.03] = -1
    ti = torch.from_numpy(ids).cuda()
    got = _layout_full(ti, E, R)
    ref = orc.dispatch_layout(ids, E, R)
    for g, r, name in zip(got, ref, ["per_rank", "per_expert", "is_token_in_rank", "send_token_idx"]):
        assert np.array_equal(g.cpu().numpy(), r), name


def test_layout_op_and_round_robin(ops):
    # test_fused_deep_moe.py:298-302: expert_ids = arange % E -> known counts and ranks
    T, K, E = 16, 8, 16
    ids = (torch.arange(T * K) % E).view(T, K)
    nte, sti = ops.get_dispatch_layout(ids.cuda(), E, 1)
    assert (nte.cpu() == T * K // E).all()
    assert torch.equal(sti.cpu().view(-1), (torch.arange(T * K) // E).int())


def _dispatch(ops, x, idx, E, mode):
    nte, sti = ops.get_dispatch_layout(idx.cuda(), E, 1)
    w = torch.ones(idx.shape, dtype=torch.float32, device="cuda")
    return nte, sti, ops.moe_dispatch_prefill(x.cuda(), idx.cuda(), w, nte, sti, "ep", 0, 1, mode == 2, mode)


DISPATCH_CASES = [(0, 128, 1024, 8, 2), (1, 4096, 7168, 256, 8), (2, 257, 1152, 64, 6), (3, 33, 4096, 16, 16)]


@pytest.mark.parametrize("mode", [0, 2, 3])
@pytest.mark.parametrize("seed,T,H,E,K", DISPATCH_CASES)
def test_dispatch_matches_oracle(ops, seed, T, H, E, K, mode):
    print(f"dispatch seed={seed} T={T} H={H} E={E} K={K} mode={mode}", flush=True)
    x, logits, bias = make_inputs(seed, T, H, E, K, 0.5)
    idx, _ = orc.route(logits.numpy(), bias.numpy(), K)
    idx_t = torch.from_numpy(idx)
    nte, sti, (ex, sc, eidx, rc, rtpe) = _dispatch(ops, x, idx_t, E, mode)
    _, rnte, _, rsti = orc.dispatch_layout(idx.astype(np.int64), E, 1)
    so, rrc, rrtpe, tot = orc.notify_dispatch(rnte)
    assert np.array_equal(nte.cpu().numpy(), rnte) and np.array_equal(sti.cpu().numpy(), rsti)
    assert np.array_equal(rc.cpu().numpy(), rrc) and np.array_equal(rtpe.cpu().numpy(), rrtpe)
    rex, rsc, reidx = orc.dispatch(x.view(torch.int16).numpy().view(np.uint16), idx, so, rsti, E, mode)
    assert ex.shape[0] == tot
    assert np.array_equal(eidx.cpu().numpy().reshape(-1, 3), reidx)
    gx = ex.cpu().view(torch.uint8 if mode else torch.int16).numpy()
    assert np.array_equal(gx.view(rex.dtype), rex)
    if mode:
        assert np.array_equal(sc.cpu().numpy().view(np.uint32), rsc.view(np.uint32))


def test_dispatch_fp8_conversion_exhaustive(ops):
    # block amax 448 gives inv = 1 exactly, so the codes are e4m3(x) for every
    # bf16 x in the block: a sweep over all finite bf16 magnitudes in range
    H = 1024
    vals = torch.arange(0, 0x7F80, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    vals = vals[vals.abs() <= 448]
    vals = torch.cat([vals, -vals])
    per_row = 127 * 8                       # 8 blocks of 127 values + the 448 anchor
    n_rows = (vals.numel() + per_row - 1) // per_row
    pad = torch.zeros(n_rows * per_row)
    pad[:vals.numel()] = vals
    blocks = pad.view(n_rows, 8, 127)
    x = torch.cat([torch.full((n_rows, 8, 1), 448.0), blocks], 2).view(n_rows, H).bfloat16()
    idx = torch.zeros((n_rows, 1), dtype=torch.int32)
    _, _, (ex, sc, _, _, _) = _dispatch(ops, x, idx, 1, 3)
    ref = x.float().to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(ex.cpu().view(torch.uint8), ref)
    assert (sc.cpu() == 1.0).all()


@pytest.mark.parametrize("seed,T,H,E,K", DISPATCH_CASES)
def test_combine_matches_oracle_bit_exact(ops, seed, T, H, E, K):
    print(f"combine seed={seed} T={T} H={H} E={E} K={K}", flush=True)
    x, logits, bias = make_inputs(seed, T, H, E, K, 0.5)
    idx, w = orc.route(logits.numpy(), bias.numpy(), K)
    idx[0, 0] = -1  # a slot that receives no row
    idx_t = torch.from_numpy(idx)
    nte, sti, (ex, sc, eidx, rc, rtpe) = _dispatch(ops, x, idx_t, E, 0)
    g = torch.Generator().manual_seed(seed + 9)
    y = torch.randn(ex.shape, generator=g).bfloat16()          # stand-in expert outputs
    out = ops.moe_combine_prefill(y.cuda(), idx_t.cuda(), torch.from_numpy(w).cuda(), eidx, rc, "ep", 0, 1)
    ref = orc.combine(bits(y), eidx.cpu().numpy(), idx, w, E)
    assert np.array_equal(bits(out), ref)


def test_cfg1_identity_experts_closed_form(ops):
    # benchmark config 1 / test_moe_dispatch_combine_prefill.py:163-168: with
    # identity experts, combine(dispatch(x)) = x * sum_k w_k
    T, H, E, K = 128, 1024, 8, 2
    x, logits, _ = make_inputs(0, T, H, E, K)
    idx, w = ops.moe_route(logits.cuda(), None, K)
    nte, sti = ops.get_dispatch_layout(idx, E, 1)
    ex, sc, eidx, rc, rtpe = ops.moe_dispatch_prefill(x.cuda(), idx, w, nte, sti, "ep", 0, 1, False)
    out = ops.moe_combine_prefill(ex, idx, w, eidx, rc, "ep", 0, 1)
    ref = x.float() * w.cpu().sum(1, keepdim=True)
    torch.testing.assert_close(out.cpu().float(), ref, rtol=2 ** -7, atol=1e-6)
    # calc_diff metric of the reference test (< 5e-5), test_moe_dispatch_combine_prefill.py:84-88
    a, b = out.cpu().double() + 1, ref.double() + 1
    assert (1 - 2 * (a * b).sum() / (a * a + b * b).sum()).item() < 5e-5


def test_int8_roundtrip_per_token_cast_back(ops):
    # examples/utils.py:104-110 per_token_cast_back semantics on the fp8 mode
    T, H, E, K = 64, 2048, 16, 4
    x, logits, _ = make_inputs(5, T, H, E, K)
    idx, w = ops.moe_route(logits.cuda(), None, K)
    nte, sti = ops.get_dispatch_layout(idx, E, 1)
    ex, sc, eidx, rc, _ = ops.moe_dispatch_prefill(x.cuda(), idx, w, nte, sti, "ep", 0, 1, True, 3)
    back = (ex.float().view(ex.shape[0], -1, 128) * sc.view(ex.shape[0], -1, 1)).view(ex.shape)
    src = x.cuda()[eidx.view(-1, 3)[:, 1].long()].float()
    err = (back - src).abs() / src.abs().view(ex.shape[0], -1, 128).amax(2, keepdim=True).repeat_interleave(128, 2).view(ex.shape)
    assert err.max().item() <= 2 ** -4 + 1e-6


def test_error_paths_raise(ops):
    x = torch.zeros(4, 1024, dtype=torch.bfloat16, device="cuda")
    idx = torch.zeros(4, 2, dtype=torch.int32, device="cuda")
    w = torch.ones(4, 2, device="cuda")
    nte, sti = ops.get_dispatch_layout(idx, 8, 1)
    with pytest.raises(RuntimeError, match="one EP rank"):
        ops.moe_dispatch_prefill(x, idx, w, nte, sti, "ep", 0, 2, False)
    with pytest.raises(RuntimeError, match="hidden"):
        ops.moe_dispatch_prefill(torch.zeros(4, 1000, dtype=torch.bfloat16, device="cuda"), idx, w, nte, sti, "ep",
                                 0, 1, False)
    with pytest.raises(RuntimeError, match="numTopk"):
        ops.get_dispatch_layout(torch.zeros(4, 17, dtype=torch.int64, device="cuda"), 32, 1)


def test_diagnose_cost_stats_accumulate(ops):
    # the optional waitRecvCostStats / sendCostStats outputs: entry 0 gains each phase's microseconds,
    # accumulated across calls, and requesting them leaves every other output unchanged
    from umdk_amd.plan import MoePrefillPlan
    T, H, E, K = 4096, 7168, 64, 8
    print(f"diagnose stats T={T} H={H} E={E} K={K}", flush=True)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, H, generator=g).bfloat16().cuda()
    logits = torch.randn(T, E, generator=g).cuda()
    plan = MoePrefillPlan(T, H, E, K, quant_mode=3, device="cuda")
    plan.route(logits)
    plan.layout()
    plan.dispatch(x)
    ref_x, ref_idx = plan.expand_x.clone(), plan.expand_idx.clone()
    y = torch.randn(T * K, H, generator=g).bfloat16().cuda()
    ref_out = plan.combine(y).clone()
    ds = torch.zeros(1, dtype=torch.int32, device="cuda")
    cs = torch.zeros(1, dtype=torch.int32, device="cuda")
    plan.dispatch(x, cost_stats=ds)
    out = plan.combine(y, cost_stats=cs)
    torch.cuda.synchronize()
    d1, c1 = int(ds.item()), int(cs.item())
    assert torch.equal(plan.expand_x.view(torch.uint8), ref_x.view(torch.uint8))
    assert torch.equal(plan.expand_idx, ref_idx) and torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
    # 235 MB written / 470 MB read: tens of microseconds each, and well under a second
    assert 5 <= d1 < 1_000_000 and 5 <= c1 < 1_000_000, (d1, c1)
    plan.dispatch(x, cost_stats=ds)
    plan.combine(y, cost_stats=cs)
    torch.cuda.synchronize()
    assert int(ds.item()) >= d1 + 5 and int(cs.item()) >= c1 + 5

    # the value itself: each call adds the phase's microseconds on the stream, so over n calls the counters
    # track HIP events placed around the same calls (each call truncates to whole microseconds, and the events
    # also hold the two clock-stamp launches)
    n = 20
    ds.zero_()
    cs.zero_()
    st = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n)]
    for e in ev:
        e[0].record(st)
        plan.dispatch(x, cost_stats=ds)
        e[1].record(st)
        e[2].record(st)
        plan.combine(y, cost_stats=cs)
        e[3].record(st)
    torch.cuda.synchronize()
    d_ev = sum(e[0].elapsed_time(e[1]) for e in ev) * 1e3
    c_ev = sum(e[2].elapsed_time(e[3]) for e in ev) * 1e3
    for got, want in ((int(ds.item()), d_ev), (int(cs.item()), c_ev)):
        assert 0.75 * want - n <= got <= want + n, (got, want)


def test_route_int64_copy_of_ids(ops):
    # the optional int64 output of the route op carries the same ids (the layout op's input type)
    from umdk_amd.plan import MoePrefillPlan
    T, H, E, K = 1000, 1024, 256, 8
    print(f"route int64 ids T={T} E={E} K={K}", flush=True)
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(T, E, generator=g).cuda()
    bias = (torch.randn(E, generator=g) * 0.5).cuda()
    plan = MoePrefillPlan(T, H, E, K, quant_mode=0, device="cuda")
    plan.route(logits, bias)
    torch.cuda.synchronize()
    assert torch.equal(plan.topk_idx64, plan.topk_idx.long())
    ref_idx, _ = orc.route(logits.cpu().numpy(), bias.cpu().numpy(), K)
    assert np.array_equal(plan.topk_idx.cpu().numpy(), ref_idx)


@pytest.mark.parametrize("use_quant", [False, True])
def test_reference_prefill_case_identity_experts(ops, use_quant):
    # test_moe_dispatch_combine_prefill.py:73-175 on one rank: x = c, w = c (c stands for the rank id,
    # which would be 0 here), topk from argpartition of |randn| + 1, layout -> dispatch -> (int8:
    # per_token_cast_back) -> combine; out must equal x * sum(w) to calc_diff < 5e-5
    T, E, K, H, c = 32, 16, 8, 7168, 3.0
    print(f"reference prefill case use_quant={use_quant}", flush=True)
    rng = np.random.default_rng(7)
    x_np = np.full((T, H), c, np.float32)
    scores = np.abs(rng.standard_normal((T, E)).astype(np.float32)) + 1
    topk_np = np.argpartition(scores, -K, axis=-1)[:, -K:]
    w_np = np.full((T, K), c, np.float32)
    x = torch.from_numpy(x_np).bfloat16().cuda()
    topk = torch.from_numpy(topk_np.astype(np.int64)).cuda()
    w = torch.from_numpy(w_np).cuda()
    nte, sti = ops.get_dispatch_layout(topk, E, 1)
    recv_x, scales, eidx, rc, _ = ops.moe_dispatch_prefill(x, topk, w, nte, sti, "ep", 0, 1, use_quant)
    if use_quant:   # per_token_cast_back with one scale per row
        recv_x = (recv_x.float().view(recv_x.size(0), -1, 128) * scales.view(-1, 1, 1)).view(recv_x.shape).bfloat16()
    out = ops.moe_combine_prefill(recv_x, topk, w, eidx, rc, "ep", 0, 1)
    check = out.cpu().float().numpy().astype(np.float64) + 1
    ref = (x_np * w_np.sum(1, keepdims=True)).astype(np.float64) + 1
    diff = 1 - 2 * (check * ref).sum() / (check * check + ref * ref).sum()
    assert diff < 5e-5


def test_dispatch_fp8_kmajor_scales_mode(ops):
    # quant mode 5 (C ABI): the same fp8 rows, block scales written k-major [H/128, capacity]
    from umdk_amd import _lib
    print("dispatch fp8 k-major scales", flush=True)
    T, H, E, K = 300, 2048, 32, 6
    x, logits, _ = make_inputs(12, T, H, E, K)
    idx, w = ops.moe_route(logits.cuda(), None, K)
    nte, sti = ops.get_dispatch_layout(idx.long(), E, 1)
    ex, sc, eidx, rc, _ = ops.moe_dispatch_prefill(x.cuda(), idx, w, nte, sti, "ep", 0, 1, True, 3)
    N = ex.shape[0]
    cap = N + 7                                   # a capacity above the row count: the k-major stride
    so = (torch.cumsum(nte, 0) - nte).int()
    ex5 = torch.empty((cap, H), dtype=torch.float8_e4m3fn, device="cuda")
    sc5 = torch.full((H // 128, cap), -1.0, device="cuda")
    ei5 = torch.empty(cap * 3, dtype=torch.int32, device="cuda")
    _lib.call("camhipMoeDispatchNormal", _lib.ptr(x.cuda()), _lib.ptr(idx), _lib.ptr(so), _lib.ptr(sti.int()), None,
              None, T, H, K, 1, 0, E, 5, cap, _lib.ptr(ex5), _lib.ptr(sc5), _lib.ptr(ei5), None, device="cuda")
    assert torch.equal(ex5[:N].view(torch.uint8), ex.view(torch.uint8))
    assert torch.equal(sc5[:, :N].t(), sc)
    assert torch.equal(ei5[:3 * N], eidx)


def test_maximum_sizes_route_dispatch_combine(ops):
    # the largest shapes the C ABI accepts at once: 65536 tokens x top-16 of 512 experts (1,048,576
    # dispatched rows, 32-bit row offsets of 1 GiB fp8 output), with the smallest hidden size so the
    # oracle stays quick; route, layout, fp8 dispatch and combine all bit-exact
    T, H, E, K = 65536, 1024, 512, 16
    print(f"max sizes T={T} H={H} E={E} K={K}", flush=True)
    x, logits, bias = make_inputs(11, T, H, E, K, 0.5)
    idx, w, ridx, rw = route_both(ops, logits, bias, K)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    idx_t = torch.from_numpy(ridx)
    nte, sti, (ex, sc, eidx, rc, rtpe) = _dispatch(ops, x, idx_t, E, 3)
    _, rnte, _, rsti = orc.dispatch_layout(ridx.astype(np.int64), E, 1)
    so, rrc, rrtpe, tot = orc.notify_dispatch(rnte)
    assert tot == T * K and ex.shape[0] == tot
    assert np.array_equal(nte.cpu().numpy(), rnte) and np.array_equal(sti.cpu().numpy(), rsti)
    assert np.array_equal(rc.cpu().numpy(), rrc)
    rex, rsc, reidx = orc.dispatch(x.view(torch.int16).numpy().view(np.uint16), ridx, so, rsti, E, 3)
    assert np.array_equal(eidx.cpu().numpy().reshape(-1, 3), reidx)
    assert np.array_equal(ex.cpu().view(torch.uint8).numpy(), rex)
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), rsc.view(np.uint32))
    del ex, sc, rex, rsc
    g = torch.Generator().manual_seed(12)
    y = torch.randn(tot, H, generator=g).bfloat16()
    out = ops.moe_combine_prefill(y.cuda(), idx_t.cuda(), torch.from_numpy(rw).cuda(), eidx, rc, "ep", 0, 1)
    ref = orc.combine(bits(y), eidx.cpu().numpy(), ridx, rw, E)
    assert np.array_equal(bits(out), ref)
