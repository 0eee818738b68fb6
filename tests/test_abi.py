"""CPU checks of the C-ABI library: it loads, exports every entry point that
include/camhip.h declares, and rejects invalid arguments with the documented
status codes and messages (the reference's tiling range checks,
dispatch_layout_tiling.cpp:98-122, moe_dispatch_normal_tiling.cpp:72-94).
No kernel is launched: only GetWorkspaceSize and the workspace check of the
second phase run, which never touch a GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "camhip.h")


@pytest.fixture(scope="module")
def L():
    from umdk_amd import _lib
    return _lib.lib()


def declared():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"CAMHIP_API\s+[^;(]*?\b(camhip\w+)\s*\(", txt)))


def test_header_declares_entry_points():
    names = declared()
    assert "camhipDispatchLayoutGetWorkspaceSize" in names and "camhipMoeCombineNormal" in names
    assert len(names) >= 12


def test_library_exports_every_declared_symbol(L):
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing


def test_python_binding_covers_every_two_phase_pair():
    from umdk_amd import _lib
    two_phase = {n[: -len("GetWorkspaceSize")] for n in declared() if n.endswith("GetWorkspaceSize")}
    assert two_phase == set(_lib.SIGNATURES)


def _ws(L, name, *args):
    ws = ctypes.c_uint64(0)
    ex = ctypes.c_void_p(0)
    st = getattr(L, name + "GetWorkspaceSize")(*args, ctypes.byref(ws), ctypes.byref(ex))
    return st, ws.value, ex, L.camhipGetLastErrorMsg().decode()


P = 0x1000  # a non-NULL stand-in pointer: never dereferenced by the first phase


@pytest.mark.parametrize("T,R,E,K,frag", [
    (10, 0, 8, 2, "numRanks"), (10, 385, 768, 2, "numRanks"), (10, 1, 513, 2, "numExperts"),
    (10, 3, 8, 2, "divisible"), (10, 1, 8, 17, "numTopk"), (10, 1, 8, 0, "numTopk"), (70000, 1, 8, 2, "numTokens"),
])
def test_layout_rejects_out_of_range(L, T, R, E, K, frag):
    st, _, _, msg = _ws(L, "camhipDispatchLayout", P, T, R, E, K, P, P, P, P)
    assert st == 161001 and frag in msg


def test_layout_null_output_is_rejected(L):
    st, _, _, msg = _ws(L, "camhipDispatchLayout", P, 10, 1, 8, 2, None, None, None, P)
    assert st == 161002 and "numTokensPerExpert" in msg


def test_layout_workspace_size_and_short_workspace(L):
    st, ws, ex, _ = _ws(L, "camhipDispatchLayout", P, 4096, 1, 256, 8, P, P, P, P)
    assert st == 0
    assert ws == 4 * 128 * (256 + 1)   # 128 chunks of 256 entries, E+R counters each
    # second phase with a short workspace: rejected before any launch, executor freed
    st2 = L.camhipDispatchLayout(None, 0, ex, None)
    assert st2 == 161003 and "workspace" in L.camhipGetLastErrorMsg().decode()


@pytest.mark.parametrize("H,q,frag", [(1000, 0, "hidden"), (8192, 0, "hidden"), (1040, 3, "128"), (1040, 5, "128"),
                                     (1024, 1, "quantMode"), (1024, 4, "quantMode")])
def test_dispatch_rejects_bad_hidden_and_quant(L, H, q, frag):
    st, _, _, msg = _ws(L, "camhipMoeDispatchNormal", P, P, P, P, None, None, 4, H, 2, 1, 0, 8, q, 8, P, P, P, None)
    assert st == 161001 and frag in msg


def test_dispatch_and_combine_need_single_rank(L):
    st, _, _, msg = _ws(L, "camhipMoeDispatchNormal", P, P, P, P, None, None, 4, 1024, 2, 2, 0, 8, 0, 8, P, P, P, None)
    assert st == 161001 and "one EP rank" in msg
    st, _, _, msg = _ws(L, "camhipMoeCombineNormal", P, P, 8, P, P, 4, 2, 1024, 2, 1, 8, P, None)
    assert st == 161001 and "one EP rank" in msg
    st, _, _, msg = _ws(L, "camhipNotifyDispatch", P, 8, 4, 2, 0, P, P, P, P, P, P)
    assert st == 161001 and "one EP rank" in msg


def test_route_limits(L):
    st, _, _, msg = _ws(L, "camhipMoeRoute", P, None, 4, 8, 9, P, P, None)
    assert st == 161001 and "topK" in msg
    st, ws, ex, _ = _ws(L, "camhipMoeRoute", P, None, 4, 8, 2, P, P, None)
    assert st == 0 and ws == 0
    assert L.camhipMoeRoute(None, 0, None, None) == 161002  # NULL executor


def test_reference_import_name():
    # the reference's call sites import the extension by its module name, then use torch.ops.umdk_cam_op_lib.*
    # (test_fused_deep_moe.py:24, 219); both work unchanged
    import torch
    import umdk_cam_op_lib
    for name in ("fused_deep_moe", "get_dispatch_layout", "moe_dispatch_prefill", "moe_combine_prefill"):
        assert callable(getattr(umdk_cam_op_lib, name))
        assert hasattr(torch.ops.umdk_cam_op_lib, name)


def test_ops_refuse_cpu_tensors():
    import torch
    import umdk_amd  # noqa: F401
    with pytest.raises(Exception):
        torch.ops.umdk_cam_op_lib.get_dispatch_layout(torch.zeros(4, 2, dtype=torch.int64), 8, 1)


def test_diagnose_outputs_take_workspace(L):
    # the optional cost-stats outputs add an 8-byte clock stamp to the workspace
    st, ws0, ex, _ = _ws(L, "camhipMoeDispatchNormal", P, P, P, P, None, None, 4, 1024, 2, 1, 0, 8, 0, 8, P, P, P, None)
    L.camhipReleaseExecutor(ex)
    st1, ws1, ex, _ = _ws(L, "camhipMoeDispatchNormal", P, P, P, P, None, None, 4, 1024, 2, 1, 0, 8, 0, 8, P, P, P, P)
    L.camhipReleaseExecutor(ex)
    assert st == 0 and st1 == 0 and ws0 == 0 and ws1 == 8
    st, wc0, ex, _ = _ws(L, "camhipMoeCombineNormal", P, P, 8, P, P, 4, 2, 1024, 1, 0, 8, P, None)
    L.camhipReleaseExecutor(ex)
    st1, wc1, ex, _ = _ws(L, "camhipMoeCombineNormal", P, P, 8, P, P, 4, 2, 1024, 1, 0, 8, P, P)
    L.camhipReleaseExecutor(ex)
    assert st == 0 and st1 == 0 and wc0 == 4 * 4 * 2 and wc1 == wc0 + 8


# grouped GEMMs: "ppp iiii pp iii pp" (SwiGLU) / "ppp iiii pp ii p" (plain)
def _gmm1(L, m=1024, k=1024, n=512, dt=3, lay=0, oq=3, xs=P, ws=P, groups=4):
    return _ws(L, "camhipGroupedMatmulSwiglu", P, xs, P, groups, m, k, n, P, ws, dt, lay, oq, P, P)


def _gmm2(L, m=1024, k=512, n=1024, dt=3, lay=0, xs=P, ws=P, groups=4):
    return _ws(L, "camhipGroupedMatmul", P, xs, P, groups, m, k, n, P, ws, dt, lay, P)


@pytest.mark.parametrize("kw,frag", [
    (dict(dt=1), "dtype"), (dict(groups=0), "numGroups"), (dict(groups=513), "numGroups"), (dict(m=0), "m "),
    (dict(k=1000), "multiple"), (dict(n=384), "I a multiple of 128"), (dict(lay=2), "xScaleLayout"),
    (dict(xs=None), "xScale"), (dict(ws=None), "weightScale"), (dict(dt=2, oq=3), "outQuant 2"),
    (dict(dt=0, oq=3), "fp8 h needs fp8 inputs"),
])
def test_gmm1_rejects_bad_arguments(L, kw, frag):
    st, _, ex, msg = _gmm1(L, **kw)
    assert st != 0 and frag in msg, msg


@pytest.mark.parametrize("kw,frag", [(dict(n=640), "multiple of 256"), (dict(k=96, dt=0), "multiple of 64"),
                                     (dict(lay=-1), "xScaleLayout")])
def test_gmm2_rejects_bad_arguments(L, kw, frag):
    st, _, ex, msg = _gmm2(L, **kw)
    assert st != 0 and frag in msg, msg


def test_gmm_workspace_sizes(L):
    # fp8 with row-major activation scales: their k-major copy, m * (k/128) floats
    st, ws, ex, _ = _gmm1(L, m=1024, k=1024, lay=0)
    L.camhipReleaseExecutor(ex)
    assert st == 0 and ws == 1024 * 8 * 4
    # k-major scales (as GMM1 writes h_scale for GMM2) and bf16 need none
    for args in (dict(lay=1), dict(dt=0, oq=0, xs=None, ws=None)):
        st, ws, ex, _ = _gmm1(L, **args)
        L.camhipReleaseExecutor(ex)
        assert st == 0 and ws == 0, args
    st, ws, ex, _ = _gmm2(L, lay=1)
    L.camhipReleaseExecutor(ex)
    assert st == 0 and ws == 0
    # int8 SwiGLU: fp32 h and the row maxima before the per-token requantisation
    st, ws, ex, _ = _gmm1(L, m=1000, k=1024, n=512, dt=2, oq=2)
    L.camhipReleaseExecutor(ex)
    assert st == 0 and ws == ((1000 * 256 * 4 + 255) & ~255) + 1000 * (256 // 32) * 4   # h, then I/32 maxima per row


def test_weight_pointer_tables_cached():
    # separated fused_deep_moe weights go to the kernels as device arrays of per-expert pointers; the
    # table for one set of pointers is built once and reused (host logic only: CPU tensors stand in)
    import torch
    from umdk_amd import ops
    ts = [torch.zeros(4) for _ in range(3)]
    t1 = ops._ptr_table(ts, "cpu")
    assert t1.dtype == torch.int64 and t1.tolist() == [t.data_ptr() for t in ts]
    assert ops._ptr_table(ts, "cpu") is t1
    assert ops._ptr_table(ts[::-1], "cpu").tolist() == [t.data_ptr() for t in ts[::-1]]


def test_converted_weights_cached_per_source():
    import torch
    # a weight in the reference's contiguous [k, n] layout is transposed once per source tensor; the copy is
    # reused while the source is unchanged, redone after an in-place update, and dropped with the source
    from umdk_amd import ops
    w = torch.arange(12, dtype=torch.float32).view(3, 4)       # logical [k=3, n=4]
    a = ops._kmajor(w, 4, 3, "w")
    assert a.is_contiguous() and torch.equal(a, w.t())
    assert ops._kmajor(w, 4, 3, "w") is a
    w.add_(1)
    b = ops._kmajor(w, 4, 3, "w")
    assert b is a and b.data_ptr() == a.data_ptr() and torch.equal(b, w.t())   # refreshed in place
    v = w.t().contiguous().t()                                  # k-contiguous storage underneath: no copy
    assert ops._kmajor(v, 4, 3, "v").data_ptr() == v.data_ptr()
    n = len(ops._CONVERTED)
    del w, a, b
    assert len(ops._CONVERTED) == n - 1
    s = torch.ones(2, 3, dtype=torch.float64)
    c = ops._contig(s, "s", torch.float32)
    assert c.dtype == torch.float32 and ops._contig(s, "s", torch.float32) is c
    f = torch.ones(2, 3)
    assert ops._contig(f, "f", torch.float32) is f


def test_combine_noalloc_rejects_beyond_its_scratch(L):
    # 65536 tokens x top-8 = 524288 row slots: past the static scratch (262144 slots); rejected before any launch
    st = L.camhipMoeCombineNormalNoAlloc(P, P, 8, None, P, 65536, 8, 1024, 1, 0, 8, P, None, None)
    assert st == 161001 and "static scratch" in L.camhipGetLastErrorMsg().decode()
    st = L.camhipMoeCombineNormalNoAlloc(P, P, 8, None, P, 4, 2, 1000, 1, 0, 8, P, None, None)
    assert st == 161001 and "hidden" in L.camhipGetLastErrorMsg().decode()


@pytest.mark.parametrize("i2", [600064, 262144])
def test_fused_rejects_operands_past_32bit_offsets(L, i2):
    # one expert's fp8 weights (2I x H) or h (batch*topk x I) of 4 GiB or more: the grouped GEMMs address
    # an operand with 32-bit byte offsets
    st, _, ex, msg = _ws(L, "camhipFusedDeepMoe", P, P, P, P, P, P, P, None, None, None, None, None, None, None,
                         4096, 7168, 8, i2, 0, 3, 1, 0, 32, 0, 0, P, None, P)
    assert st != 0 and "4 GiB" in msg, msg
    st, _, ex, msg = _ws(L, "camhipFusedDeepMoe", P, P, P, P, P, P, P, None, None, None, None, None, None, None,
                         4096, 7168, 8, 4096, 0, 3, 1, 0, 32, 0, 0, P, None, P)
    assert st == 0, msg
    L.camhipReleaseExecutor(ex)



@pytest.mark.parametrize("T,K,H,Lx,cap,frag", [
    (0, 8, 1024, 8, 8, "numTokens"), (4, 8, 1024, 0, 8, "localExperts"), (4, 2, 1024, 8, 9, "recvRowsCapacity"),
    (4, 2, 1024, 8, 0, "recvRowsCapacity"), (4, 17, 1024, 8, 8, "topK"), (4, 2, 1000, 8, 8, "hidden"),
])
def test_prefill_combine_rejects_out_of_range(L, T, K, H, Lx, cap, frag):
    st, _, _, msg = _ws(L, "camhipMoePrefillCombine", P, P, P, P, P, T, K, H, Lx, cap, P)
    assert st == 161001 and frag in msg, msg


def test_prefill_combine_null_pointers_are_rejected(L):
    st, _, _, msg = _ws(L, "camhipMoePrefillCombine", P, P, None, P, P, 4, 2, 1024, 8, 8, P)
    assert st == 161002 and "combineRowMap" in msg, msg
    st, ws, ex, msg = _ws(L, "camhipMoePrefillCombine", P, P, P, P, P, 4, 2, 1024, 8, 8, P)
    assert st == 0 and ws == 0, msg
    L.camhipReleaseExecutor(ex)


@pytest.mark.parametrize("dt,H,I2,frag", [(2, 1024, 512, "dtype"), (3, 1000, 512, "k"), (3, 1024, 300, "I")])
def test_moe_experts_rejects_bad_arguments(L, dt, H, I2, frag):
    st, _, _, msg = _ws(L, "camhipMoeExperts", P, P, P, 8, 64, H, I2, P, P, P, P, dt, 1, P, P, P)
    assert st == 161001 and frag in msg, msg


def test_moe_experts_workspace_holds_the_counters(L):
    # decode-sized groups (<= 48 rows per group): the chained launch's readiness counters, cleared by the call
    st, ws, ex, msg = _ws(L, "camhipMoeExperts", P, P, P, 32, 1024, 7168, 4096, P, P, P, P, 3, 1, P, P, P)
    assert st == 0 and ws >= 4 * (1024 // 32 + 32), msg
    L.camhipReleaseExecutor(ex)
    st, _, _, msg = _ws(L, "camhipMoeExperts", P, P, P, 32, 1024, 7168, 4096, P, P, P, P, 3, 1, P, None, P)
    assert st != 0, "fp8 h scales are required"
