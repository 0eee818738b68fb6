"""GPU tests of the graph-capturable full-layer runner (umdk_amd.plan.MoeLayerPlan): route over E experts, keep
this rank's L local experts, dispatch, GMM1+SwiGLU, GMM2, combine, all capacity-sized with no host reads.

It is compared with the chain of torch ops on the same routing (same kernels on actual-size buffers, so the
result must agree within the GEMM tolerances: 2e-2 bf16, 5e-2 fp8, max-norm), and a captured HIP graph of it is
replayed with new inputs, each replay checked against an eager run (bit-identical: same launches, same data).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import umdk_amd  # noqa: F401
    return torch.ops.umdk_cam_op_lib


def relerr(got, ref):
    return ((got.double() - ref.double()).abs().max() / ref.double().abs().max().clamp_min(1e-30)).item()


def _weights(L, H, I, dtype):
    import bench
    return bench.make_weights(L, H, I, dtype, torch.device("cuda"), 0)


def _chain(ops, plan, x, w1, s1, w2, s2, dtype, E_local):
    # the small-op chain on the plan's own routing (ids of non-local experts are not routed here)
    q = {"bf16": 0, "int8": 2, "fp8": 3}[dtype]
    ids = plan.topk_idx.clone()
    nte, sti = ops.get_dispatch_layout(ids.long(), E_local, 1)
    ex, xs, eidx, rc, rtpe = ops.moe_dispatch_prefill(x, ids, plan.topk_w, nte, sti, "ep", 0, 1, q != 0, q)
    h, hs = ops.grouped_matmul_swiglu(ex, xs if q else None, rtpe, w1, s1, q)
    y = ops.grouped_matmul(h, hs if q else None, rtpe, w2, s2)
    return ops.moe_combine_prefill(y, ids, plan.topk_w, eidx, rc, "ep", 0, 1), rtpe


@pytest.mark.parametrize("dtype", ["bf16", "fp8", "int8"])
def test_layer_plan_matches_op_chain_and_replays(ops, dtype):
    from umdk_amd.plan import MoeLayerPlan
    print(f"layer plan {dtype}", flush=True)
    T, H, E, K, L, I = 512, 2048, 64, 8, 16, 512
    g = torch.Generator(device="cuda").manual_seed(21)
    x = torch.randn(T, H, device="cuda", generator=g).bfloat16()
    logits = torch.randn(T, E, device="cuda", generator=g)
    bias = torch.randn(E, device="cuda", generator=g) * 0.5
    w1, s1, w2, s2 = _weights(L, H, I, dtype)
    plan = MoeLayerPlan(T, H, E, K, L, I, dtype=dtype, device="cuda")
    out = plan.forward(x, logits, bias, w1, s1, w2, s2).clone()
    ref, rtpe = _chain(ops, plan, x, w1, s1, w2, s2, dtype, L)
    assert torch.equal(plan.recv_tokens_per_expert[:L], rtpe)
    routed = (plan.topk_idx < L).any(dim=1)
    assert int(routed.sum()) > 0
    assert relerr(out[routed].float(), ref[routed].float()) < (5e-2 if dtype == "fp8" else 2e-2)
    assert int(out[~routed].view(torch.int16).abs().sum()) == 0          # tokens with no local expert

    # graph capture: replays with new inputs equal eager runs on the same inputs
    xs_in, lg_in = x.clone(), logits.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        plan.forward(xs_in, lg_in, bias, w1, s1, w2, s2)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout = plan.forward(xs_in, lg_in, bias, w1, s1, w2, s2)
    for r in range(3):
        xs_in.copy_(torch.randn(T, H, device="cuda", generator=g).bfloat16())
        lg_in.copy_(torch.randn(T, E, device="cuda", generator=g))
        graph.replay()
        got = gout.clone()
        eager = plan.forward(xs_in, lg_in, bias, w1, s1, w2, s2).clone()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16)), f"replay {r}"
