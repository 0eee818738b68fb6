"""GPU tests of the four-launch prefill step (camhipMoePrefillDispatch + camhipMoePrefillCombine, used by
umdk_amd.plan): its outputs must equal, bit for bit, those of the reference-shaped chain (camhipMoeRoute,
camhipDispatchLayout, camhipNotifyDispatch, camhipMoeDispatchNormal, camhipMoeCombineNormal) and the CPU
oracle's chain (route, dispatch_layout.h:112-161, notify_dispatch.h:340-412, moe_dispatch_normal.h:381-398,
moe_combine_normal.h:343-377) on the same inputs.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

Q = {0: orc.QUANT_NONE, 2: orc.QUANT_INT8, 3: orc.QUANT_FP8}


@pytest.fixture(scope="module")
def lib():
    import umdk_amd  # noqa: F401
    from umdk_amd import _lib
    return _lib


def b16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def raw(t):
    return t.cpu().contiguous().view(torch.uint8).numpy()


# (T, H, E routed, L local, K, quant mode): config 2's shape, a layer rank's share (ids >= L not routed here),
# ragged token counts (not a multiple of the 16-token chunk), K = 16 (256 entries per chunk) and 512 experts
CASES = [(4096, 7168, 256, 256, 8, 3), (4096, 7168, 256, 32, 8, 3), (1000, 1024, 64, 64, 6, 0),
         (333, 2048, 512, 512, 16, 2), (17, 1024, 8, 8, 2, 3), (1, 1024, 16, 4, 3, 0), (4099, 2048, 128, 96, 8, 2),
         (20000, 1024, 64, 64, 4, 0), (9000, 1024, 32, 32, 2, 3)]


@pytest.mark.parametrize("T,H,E,L,K,q", CASES)
def test_prefill_step_matches_op_chain_and_oracle(lib, T, H, E, L, K, q):
    from umdk_amd.plan import MoePrefillPlan
    print(f"prefill step T={T} H={H} E={E} L={L} K={K} q={q}", flush=True)
    g = torch.Generator().manual_seed(T + E + K)
    x = torch.randn(T, H, generator=g).bfloat16()
    logits = torch.randn(T, E, generator=g)
    bias = torch.randn(E, generator=g) * 0.5
    cx, clg, cb = x.cuda(), logits.cuda(), bias.cuda()

    fast = MoePrefillPlan(T, H, L, K, quant_mode=q, device="cuda")
    fast.E_route = E
    fast.dispatch_step(clg, cx, cb)
    ref = MoePrefillPlan(T, H, L, K, quant_mode=q, device="cuda")
    ref.E_route = E
    # the reference-shaped chain over the same routing: route over E, then layout etc. over the L local experts
    lib.launch("camhipMoeRoute", clg.data_ptr(), cb.data_ptr(), T, E, K, ref.topk_idx.data_ptr(),
               ref.topk_w.data_ptr(), ref.topk_idx64.data_ptr(), device=ref.device)
    ref.layout()
    ref.dispatch(cx)
    torch.cuda.synchronize()
    assert torch.equal(fast.topk_idx, ref.topk_idx) and torch.equal(fast.topk_w, ref.topk_w)
    assert torch.equal(fast.recv_count, ref.recv_count)
    assert torch.equal(fast.recv_tokens_per_expert, ref.recv_tokens_per_expert)
    rows = int(ref.recv_count[-1])
    assert torch.equal(fast.expand_idx[:3 * rows], ref.expand_idx[:3 * rows])
    assert np.array_equal(raw(fast.expand_x[:rows]), raw(ref.expand_x[:rows]))
    if q:
        assert torch.equal(fast.scales[:rows], ref.scales[:rows])

    # the oracle chain
    ridx, rw = orc.route(logits.numpy(), bias.numpy(), K)
    assert np.array_equal(fast.topk_idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(fast.topk_w.cpu().numpy(), rw, rtol=1e-5)
    rid = np.where(ridx < L, ridx, -1).astype(np.int32)
    _, nte, _, sti = orc.dispatch_layout(rid.astype(np.int64), L, 1)
    so, rc, rtpe, tot = orc.notify_dispatch(nte)
    assert tot == rows and np.array_equal(fast.recv_count.cpu().numpy(), rc)
    ex, sc, eidx = orc.dispatch(b16(x), rid, so, sti, L, Q[q])
    assert np.array_equal(raw(fast.expand_x[:rows]), ex.view(np.uint8).reshape(rows, H * (2 if q == 0 else 1)))
    assert np.array_equal(fast.expand_idx[:3 * rows].cpu().numpy().reshape(rows, 3), eidx)
    if q:
        assert np.array_equal(fast.scales[:rows].cpu().numpy(), sc)

    # combine of stand-in expert outputs: the step's gather on the dispatch's row map equals the two-phase
    # combine and the oracle
    y = torch.randn(T * K, H, generator=g).bfloat16().cuda()
    out_fast = fast.combine_step(y).clone()
    out_ref = ref.combine(y).clone()
    torch.cuda.synchronize()
    assert torch.equal(out_fast.view(torch.int16), out_ref.view(torch.int16))
    oref = orc.combine(b16(y)[:rows], eidx, rid, fast.topk_w.cpu().numpy(), L)   # GPU gates: expf differs in ulps
    assert np.array_equal(b16(out_fast), oref)


def test_prefill_step_graph_replays(lib):
    # the step captured in a HIP graph, replayed with new inputs: each replay equals an eager step
    from umdk_amd.plan import MoePrefillPlan
    T, H, E, K = 512, 2048, 64, 8
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(T, H, device="cuda", generator=g).bfloat16()
    logits = torch.randn(T, E, device="cuda", generator=g)
    y = torch.randn(T * K, H, device="cuda", generator=g).bfloat16()
    plan = MoePrefillPlan(T, H, E, K, quant_mode=3, device="cuda")
    eager = MoePrefillPlan(T, H, E, K, quant_mode=3, device="cuda")
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        plan.dispatch_step(logits, x)
        plan.combine_step(y)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.dispatch_step(logits, x)
        gout = plan.combine_step(y)
    for r in range(3):
        x.copy_(torch.randn(T, H, device="cuda", generator=g).bfloat16())
        logits.copy_(torch.randn(T, E, device="cuda", generator=g))
        graph.replay()
        got = gout.clone()
        eager.dispatch_step(logits, x)
        ref = eager.combine_step(y)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"replay {r}"
        assert torch.equal(plan.expand_x.view(torch.uint8), eager.expand_x.view(torch.uint8))


def test_prefill_step_rejects_bad_arguments(lib):
    import ctypes
    L_ = lib.lib()
    ws, ex = ctypes.c_uint64(0), ctypes.c_void_p(0)
    P = 0x1000
    st = L_.camhipMoePrefillDispatchGetWorkspaceSize(P, None, P, 16, 1024, 8, 9, 2, 3, 32, P, P, P, P, P, P, P, P,
                                                     ctypes.byref(ws), ctypes.byref(ex))
    assert st == 161001 and "localExperts" in L_.camhipGetLastErrorMsg().decode()
    st = L_.camhipMoePrefillDispatchGetWorkspaceSize(P, None, P, 16, 1024, 8, 8, 2, 3, 33, P, P, P, P, P, P, P, P,
                                                     ctypes.byref(ws), ctypes.byref(ex))
    assert st == 161001 and "recvRowsCapacity" in L_.camhipGetLastErrorMsg().decode()

