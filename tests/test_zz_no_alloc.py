"""GPU test of the allocation-free combine (camhipMoeCombineNormalNoAlloc) through the C ABI.

Its output must be bit-identical to the two-phase combine (camhipMoeCombineNormalGetWorkspaceSize +
camhipMoeCombineNormal) on the same dispatch, on two calls in a row -- the second with a smaller input, so
the row map left in the shared static scratch by the first call must not leak into the second -- and with
the diagnose output requested.
"""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _dispatched(T, H, E, K, seed):
    from umdk_amd.ops import QUANT_NONE
    from umdk_amd.plan import MoePrefillPlan
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(T, H, device="cuda", generator=g).bfloat16()
    logits = torch.randn(T, E, device="cuda", generator=g)
    plan = MoePrefillPlan(T, H, E, K, quant_mode=QUANT_NONE, device="cuda")
    plan.route(logits)
    plan.layout()
    plan.dispatch(x)
    y = (plan.expand_x.float() * 0.5 + 0.25).bfloat16()      # stand-in expert outputs in dispatch order
    return plan, y


def _noalloc(plan, y, out, stats=None):
    from umdk_amd import _lib
    L = _lib.lib()
    st = L.camhipMoeCombineNormalNoAlloc(y.data_ptr(), plan.expand_idx.data_ptr(), plan.N,
                                         plan.recv_count.data_ptr(), plan.topk_w.data_ptr(), plan.T, plan.K, plan.H,
                                         1, 0, plan.E, out.data_ptr(), None if stats is None else stats.data_ptr(),
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, L.camhipGetLastErrorMsg().decode()


@pytest.mark.parametrize("with_stats", [False, True])
def test_noalloc_combine_matches_two_phase_combine(with_stats):
    import umdk_amd  # noqa: F401
    for i, (T, H, E, K) in enumerate([(4096, 7168, 256, 8), (300, 2048, 64, 4)]):
        print(f"noalloc combine call {i}: T={T} H={H} E={E} K={K} stats={with_stats}", flush=True)
        plan, y = _dispatched(T, H, E, K, 40 + i)
        ref = plan.combine(y).clone()                         # the two-phase entry point, caller workspace
        out = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device="cuda")
        stats = torch.zeros(1, dtype=torch.int32, device="cuda") if with_stats else None
        _noalloc(plan, y, out, stats)  # warm-up: the kernels' code is loaded by the first launch
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        if stats is not None:
            stats.zero_()
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        free_before = torch.cuda.mem_get_info()[0]  # the device's free bytes (hipMemGetInfo): any allocation
        _noalloc(plan, y, out, stats)
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        assert torch.cuda.mem_get_info()[0] == free_before, "device memory was allocated"
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"call {i}"
        if with_stats:
            assert int(stats.item()) >= 0
