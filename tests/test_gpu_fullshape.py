"""GPU parity at the benchmarked shapes themselves, against the CPU oracle's chain.

* Config 5 (decode): T=128, H=7168, routed over 256 experts by moe_route, 32 local experts, I=2048, fp8
  fused_deep_moe -- eagerly and as the route + fused-op HIP graph the benchmark replays.
* Config 4 (prefill layer): MoeLayerPlan fp8 at T=4096, H=7168, 32 of 256 experts, I=2048, Zipf(1.1)
  expert popularity.
* Config 3 (Mixtral-8x7B layer, bf16): MoeLayerPlan at T=8192, H=4096, I=14336, 8 experts, top-2, against an fp32
  torch chain of the experts and the combine (the oracle's bf16 GEMM is too slow at this size; routing, counts
  and the dispatched rows are still checked against the oracle).

The oracle runs the reference's chain on the same inputs: route (R0), layout and count exchange
(dispatch_layout.h:112-161, notify_dispatch.h:340-412), fp8 dispatch (Q1/D3), GMM1 + SwiGLU + fp8 requant of
h, GMM2, combine (moe_combine_normal.h:343-377).  Ids, counts, dispatched codes and scales must be bit-exact;
the combined output is within the fp8 GEMM bound (5e-2, max-norm relative).  expert_token_nums must equal
the oracle's counts exactly, as the reference's fused test requires (test_fused_deep_moe.py:443-452).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

H, I, E_ROUTE, K, L = 7168, 2048, 256, 8, 32


@pytest.fixture(scope="module")
def ops():
    import umdk_amd  # noqa: F401
    return torch.ops.umdk_cam_op_lib


def relerr(got, ref):
    got = torch.as_tensor(got, dtype=torch.float64)
    ref = torch.as_tensor(ref, dtype=torch.float64)
    return ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def b16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    return t.cpu().contiguous().view(torch.uint8).numpy()


@pytest.fixture(scope="module")
def weights():
    import bench
    w1, s1, w2, s2 = bench.make_weights(L, H, I, "fp8", torch.device("cuda"), 0)
    host = dict(w1=u8(w1), s1=s1.cpu().numpy(), w2=u8(w2), s2=s2.cpu().numpy())
    return (w1, s1, w2, s2), host


def oracle_layer(x, logits, bias, host):
    """The oracle chain over this rank's L local experts -> (ids, counts, codes, scales, out)."""
    ridx, rw = orc.route(logits.cpu().numpy(), None if bias is None else bias.cpu().numpy(), K)
    rid = np.where(ridx < L, ridx, -1).astype(np.int32)        # non-local experts are not routed on this rank
    _, nte, _, sti = orc.dispatch_layout(rid.astype(np.int64), L, 1)
    so, _, _, _ = orc.notify_dispatch(nte)
    ex, xs, eidx = orc.dispatch(b16(x), rid, so, sti, L, orc.QUANT_FP8)
    cnt = nte.astype(np.int64)
    hq, hs = orc.gmm1_swiglu_fp8(ex, xs, cnt, host["w1"], host["s1"])
    y = orc.gmm2_fp8(hq, hs, cnt, host["w2"], host["s2"])
    out = orc.combine(y, eidx, rid, rw, L)
    return ridx, rw, cnt, ex, xs, orc.bf16_to_f32(out)


def test_decode_config5_fp8_matches_oracle_chain(ops, weights):
    (w1, s1, w2, s2), host = weights
    T = 128
    print(f"config 5 fp8 decode T={T} H={H} I={I} {L} of {E_ROUTE} experts", flush=True)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, H, generator=g).bfloat16().cuda()
    logits = torch.randn(T, E_ROUTE, generator=g).cuda()
    lw1, lw2 = w1.transpose(1, 2), w2.transpose(1, 2)       # logical [L, H, 2I] / [L, I, H] views

    def step():
        ids, wts = ops.moe_route(logits, None, K)
        out, _, etn = ops.fused_deep_moe(x, ids, [lw1], [s1], [lw2], [s2], wts, None, None, None, None, None,
                                         None, None, "ep", 1, 0, L, 0, 0)
        return ids, wts, out, etn

    ids, wts, out, etn = step()
    ridx, rw, cnt, _, _, ref = oracle_layer(x, logits, None, host)
    assert np.array_equal(ids.cpu().numpy(), ridx)
    np.testing.assert_allclose(wts.cpu().numpy(), rw, rtol=1e-5)
    assert np.array_equal(etn.cpu().numpy(), cnt)
    assert int((cnt > 0).sum()) >= 24 and cnt.sum() > 64       # the decode shape: most local experts touched
    assert relerr(out.cpu().float(), ref) < 5e-2

    # the benchmark's graph of the same step: every replay equals the eager result
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        step()
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _, _, gout, getn = step()
    for r in range(3):
        junk = torch.randn(1 << 20, device="cuda") * r
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout.view(torch.int16), out.view(torch.int16)), f"replay {r}"
        assert torch.equal(getn, etn)
        del junk


def test_layer_config4_fp8_matches_oracle_chain(ops, weights):
    import bench
    from umdk_amd.plan import MoeLayerPlan
    (w1, s1, w2, s2), host = weights
    T = 4096
    print(f"config 4 fp8 layer T={T} H={H} I={I} {L} of {E_ROUTE} experts, Zipf 1.1", flush=True)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, H, generator=g).bfloat16().cuda()
    logits = torch.randn(T, E_ROUTE, generator=g).cuda()
    bias = bench.zipf_bias(E_ROUTE, 1.1, 0).cuda()
    plan = MoeLayerPlan(T, H, E_ROUTE, K, L, I, dtype="fp8", device="cuda")
    out = plan.forward(x, logits, bias, w1, s1, w2, s2).clone()
    torch.cuda.synchronize()
    ridx, rw, cnt, ex, xs, ref = oracle_layer(x, logits, bias, host)
    M = int(cnt.sum())
    assert np.array_equal(plan.topk_idx.cpu().numpy(), ridx)
    assert np.array_equal(plan.recv_tokens_per_expert[:L].cpu().numpy(), cnt)
    assert cnt.max() >= 384 and M > 1000                    # Zipf skew: heavy experts take the 256-row tiles
    assert np.array_equal(u8(plan.expand_x[:M]), ex), "fp8 codes differ from the oracle"
    assert np.array_equal(plan.scales[:M].cpu().numpy(), xs), "fp8 block scales differ from the oracle"
    assert relerr(out.cpu().float(), ref) < 5e-2


def test_layer_config3_bf16_matches_fp32_reference(ops):
    # config 3 at its own shape (Mixtral-8x7B: T=8192, H=4096, I=14336, 8 experts, top-2, bf16): MoeLayerPlan
    # against an fp32 torch chain on the same routing (bf16 rounding of h and of the expert outputs, as the
    # layer stores them), 2e-2 max-norm; ids, counts and the dispatched rows checked exactly against the oracle
    import bench
    from umdk_amd.plan import MoeLayerPlan
    T, H3, E3, K3, I3 = 8192, 4096, 8, 2, 14336
    print(f"config 3 bf16 layer T={T} H={H3} I={I3} E={E3} K={K3}", flush=True)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, H3, generator=g).bfloat16().cuda()
    logits = torch.randn(T, E3, generator=g).cuda()
    w1, _, w2, _ = bench.make_weights(E3, H3, I3, "bf16", torch.device("cuda"), 0)
    plan = MoeLayerPlan(T, H3, E3, K3, E3, I3, dtype="bf16", device="cuda")
    out = plan.forward(x, logits, None, w1, None, w2, None).clone()
    torch.cuda.synchronize()
    ridx, rw = orc.route(logits.cpu().numpy(), None, K3)
    assert np.array_equal(plan.topk_idx.cpu().numpy(), ridx)
    _, nte, _, sti = orc.dispatch_layout(ridx.astype(np.int64), E3, 1)
    assert np.array_equal(plan.recv_tokens_per_expert[:E3].cpu().numpy(), nte.astype(np.int64))
    so, _, _, _ = orc.notify_dispatch(nte)
    ex, _, eidx = orc.dispatch(b16(x), ridx, so, sti, E3, orc.QUANT_NONE)
    M = int(nte.sum())
    assert np.array_equal(b16(plan.expand_x[:M]), ex)
    # fp32 reference of the experts and the combine on the GPU's own gates
    ids = plan.topk_idx.long()
    wts = plan.topk_w
    ref = torch.zeros(T, H3, device="cuda")
    for e in range(E3):
        tok, kk = (ids == e).nonzero(as_tuple=True)
        gu = x[tok].float() @ w1[e].float().T
        h = (gu[:, :I3] / (1 + torch.exp(-gu[:, :I3])) * gu[:, I3:]).bfloat16().float()
        y = (h @ w2[e].float().T).bfloat16().float()
        ref.index_add_(0, tok, y * wts[tok, kk].unsqueeze(1))
    assert relerr(out.float(), ref) < 2e-2
