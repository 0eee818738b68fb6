"""GPU tests of the fused decode entry (torch.ops.umdk_cam_op_lib.fused_deep_moe).

The reference checks its fused op against the chain of small ops
(test/cam/ut/fused_deep_moe/test_fused_deep_moe.py:102-240, expert_token_nums
exactly equal at :450-452).  Here the fused op is compared with (1) the chain of
this build's own small ops -- bit-identical, since it runs the same kernels in
the same order -- and (2) the CPU oracle's chain (layout, dispatch, grouped
GEMMs, combine) within the GEMM tolerances (2e-2 bf16, 5e-2 fp8, max-norm).
expert_token_nums must match the oracle's counts exactly.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


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


def fp8_w(w):
    L, n, k = w.shape
    wv = w.float().view(L, n // 128, 128, k // 128, 128)
    amax = wv.abs().amax(dim=(2, 4)).clamp(min=1e-6)
    q = (wv / (amax / 448.0)[:, :, None, :, None]).to(torch.float8_e4m3fn)
    return q.view(L, n, k), (amax / 448.0).contiguous()


def make(seed, bs, H, I, E, K, dtype, ish=0, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(bs, H, generator=g) * 10 - 5).bfloat16()       # U(-5,5) as test_fused_deep_moe.py:276-344
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(bs)]).int()
    scales = torch.rand(bs, K, generator=g)
    w1 = torch.randn(E, 2 * I, H, generator=g) * 0.02                # physical [L, 2I, H]
    w2 = torch.randn(E, H, I, generator=g) * 0.02
    d = dict(x=x, ids=ids, scales=scales)
    if dtype == "bf16":
        d.update(w1=w1.bfloat16(), w2=w2.bfloat16(), s1=None, s2=None)
    else:
        q1, s1 = fp8_w(w1)
        q2, s2 = fp8_w(w2)
        d.update(w1=q1, w2=q2, s1=s1, s2=s2)
    if ish:
        sw1 = torch.randn(1, 2 * ish, H, generator=g) * 0.02
        sw2 = torch.randn(1, H, ish, generator=g) * 0.02
        if dtype == "bf16":
            d.update(sw1=sw1[0].bfloat16(), sw2=sw2[0].bfloat16(), ss1=None, ss2=None)
        else:
            q1, s1 = fp8_w(sw1)
            q2, s2 = fp8_w(sw2)
            d.update(sw1=q1[0], sw2=q2[0], ss1=s1[0], ss2=s2[0])
    return {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in d.items()}


def call_fused(ops, d, E, mask=None, separated=False):
    # logical reference shapes: gmm1 [L, H, 2I], gmm2 [L, I, H] -- transposed views of the k-contiguous storage
    w1 = d["w1"].transpose(1, 2)
    w2 = d["w2"].transpose(1, 2)
    g1 = list(w1.unbind(0)) if separated else [w1]
    g2 = list(w2.unbind(0)) if separated else [w2]
    s1 = [d["s1"]] if d["s1"] is not None else []
    s2 = [d["s2"]] if d["s2"] is not None else []
    sw1 = d.get("sw1")
    return ops.fused_deep_moe(d["x"], d["ids"], g1, s1, g2, s2, d["scales"],
                              None if sw1 is None else sw1.T, d.get("ss1"),
                              None if sw1 is None else d["sw2"].T, d.get("ss2"),
                              None, None, mask, "ep", 1, 0, E, 0, 0)


def chain_small_ops(ops, d, E, K):
    fp8 = d["s1"] is not None
    nte, sti = ops.get_dispatch_layout(d["ids"], E, 1)
    ex, xs, eidx, rc, rtpe = ops.moe_dispatch_prefill(d["x"], d["ids"], d["scales"], nte, sti, "ep", 0, 1, fp8,
                                                      3 if fp8 else 0)
    h, hs = ops.grouped_matmul_swiglu(ex, xs if fp8 else None, rtpe, d["w1"], d["s1"], 3 if fp8 else 0)
    y = ops.grouped_matmul(h, hs if fp8 else None, rtpe, d["w2"], d["s2"])
    out = ops.moe_combine_prefill(y, d["ids"], d["scales"], eidx, rc, "ep", 0, 1)
    return out, rtpe


@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
# up to 2048 (token, k) entries the layout runs inside the dispatch launch (256 x 8: the limit; 512 experts);
# 300 x 8 takes the single-block layout launch, 1100 x 8 > 8192 entries the prefill-sized bookkeeping path
@pytest.mark.parametrize("bs,H,I,E,K", [(16, 7168, 1024, 16, 8), (128, 2048, 512, 32, 8), (3, 1024, 128, 8, 2),
                                        (256, 1024, 128, 16, 8), (64, 1024, 128, 512, 8), (300, 1024, 128, 16, 8),
                                        (1100, 1024, 128, 16, 8)])
def test_fused_equals_small_op_chain(ops, dtype, bs, H, I, E, K):
    print(f"fused vs chain {dtype} bs={bs} H={H} I={I} E={E} K={K}", flush=True)
    d = make(bs + H, bs, H, I, E, K, dtype)
    out, _, etn = call_fused(ops, d, E)
    ref, rtpe = chain_small_ops(ops, d, E, K)
    assert torch.equal(etn, rtpe)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("H", [1024, 512])   # 512: the reference fused op's smallest token length
@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_fused_matches_oracle_chain(ops, dtype, H):
    bs, I, E, K = 12, 128, 8, 3
    d = make(11, bs, H, I, E, K, dtype)
    ids = d["ids"].clone()
    ids[2, 1] = -1                       # placeholder slot
    mask = torch.ones(bs, dtype=torch.bool, device="cuda")
    mask[9:] = False                     # true-prefix active mask
    d["ids"] = ids
    out, _, etn = call_fused(ops, d, E, mask=mask)
    # oracle chain on the same inputs
    rid = ids.cpu().numpy().copy()
    rid[9:] = -1
    _, nte, _, sti = orc.dispatch_layout(rid.astype(np.int64), E, 1)
    so, _, _, _ = orc.notify_dispatch(nte)
    assert np.array_equal(etn.cpu().numpy(), nte.astype(np.int64))
    cnt = nte.astype(np.int64)
    if dtype == "bf16":
        ex, _, eidx = orc.dispatch(b16(d["x"]), rid, so, sti, E, orc.QUANT_NONE)
        h = orc.gmm1_swiglu_bf16(ex, cnt, b16(d["w1"]))
        y = orc.gmm2_bf16(h, cnt, b16(d["w2"]))
        tol = 2e-2
    else:
        ex, xs, eidx = orc.dispatch(b16(d["x"]), rid, so, sti, E, orc.QUANT_FP8)
        hq, hs = orc.gmm1_swiglu_fp8(ex, xs, cnt, u8(d["w1"]), d["s1"].cpu().numpy())
        y = orc.gmm2_fp8(hq, hs, cnt, u8(d["w2"]), d["s2"].cpu().numpy())
        tol = 5e-2
    ref = orc.combine(y, eidx, rid, d["scales"].cpu().numpy(), E)
    got = out.cpu().float()
    assert relerr(got[:9], orc.bf16_to_f32(ref)[:9]) < tol
    assert (got[9:] == 0).all()          # inactive tokens receive nothing


@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_fused_shared_expert_and_separated_weights(ops, dtype):
    bs, H, I, E, K, ish = 32, 2048, 256, 16, 4, 512
    d = make(5, bs, H, I, E, K, dtype, ish=ish)
    out_c, sh_c, etn_c = call_fused(ops, d, E)
    out_s, sh_s, etn_s = call_fused(ops, d, E, separated=True)
    assert torch.equal(out_c.view(torch.int16), out_s.view(torch.int16)) and torch.equal(etn_c, etn_s)
    assert torch.equal(sh_c.view(torch.int16), sh_s.view(torch.int16))
    # shared expert: dense SwiGLU FFN of every token, checked against the oracle's chain for one expert that
    # receives every token (dispatch with the fused op's quantiser, GMM1+SwiGLU with the fp8 requant of h, GMM2)
    ids1 = np.zeros((bs, 1), np.int32)
    sti1 = np.arange(bs, dtype=np.int32)[:, None]
    so1 = np.zeros(1, np.int32)
    cnt = np.array([bs], np.int64)
    if dtype == "bf16":
        ex, _, _ = orc.dispatch(b16(d["x"]), ids1, so1, sti1, 1, orc.QUANT_NONE)
        h = orc.gmm1_swiglu_bf16(ex, cnt, b16(d["sw1"])[None])
        ref = orc.gmm2_bf16(h, cnt, b16(d["sw2"])[None])
    else:
        ex, xs, _ = orc.dispatch(b16(d["x"]), ids1, so1, sti1, 1, orc.QUANT_FP8)
        hq, hs = orc.gmm1_swiglu_fp8(ex, xs, cnt, u8(d["sw1"])[None], d["ss1"].cpu().numpy()[None])
        ref = orc.gmm2_fp8(hq, hs, cnt, u8(d["sw2"])[None], d["ss2"].cpu().numpy()[None])
    assert relerr(sh_c.cpu().float(), orc.bf16_to_f32(ref)) < (2e-2 if dtype == "bf16" else 5e-2)


def test_fused_graph_capture_replays(ops):
    # decode step captured in a HIP graph; every replay must equal the eager result, with eager
    # work and synchronisations between replays
    bs, H, I, E, K = 128, 7168, 256, 32, 8
    d = make(3, bs, H, I, E, K, "fp8")
    eager, _, etn0 = call_fused(ops, d, E)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            call_fused(ops, d, E)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout, _, getn = call_fused(ops, d, E)
    for r in range(4):
        junk = torch.randn(1 << 20, device="cuda") * r   # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout.view(torch.int16), eager.view(torch.int16)), f"replay {r}"
        assert torch.equal(getn, etn0)
        del junk


@pytest.mark.parametrize("layout", ["kmajor_view", "reference_contiguous"])
@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_fused_separated_allocations_in_place(ops, dtype, layout):
    # dynamic-EPLB weights (test_fused_deep_moe.py:256-269): one allocation per expert, made in a
    # scrambled order, weights and scales both as lists.  "kmajor_view": transposed views of k-contiguous
    # storage, read in place through device pointer tables (no copy at all).  "reference_contiguous": the
    # reference's own contiguous [k, n] per-expert tensors (what its clone() produces), converted once and
    # cached on the source tensors, so later calls and a captured graph make no copy.  Both are
    # bit-identical to the coupled call and a graph captured on the lists replays correctly.
    bs, H, I, E, K = 128, 7168, 256, 32, 8
    d = make(7, bs, H, I, E, K, dtype)
    ref, _, etn_ref = call_fused(ops, d, E)
    order = torch.randperm(E, generator=torch.Generator().manual_seed(1)).tolist()
    g1, g2, s1, s2 = [None] * E, [None] * E, [None] * E, [None] * E
    for e in order:
        if layout == "kmajor_view":
            g1[e] = d["w1"][e].clone().transpose(0, 1)       # logical [H, 2I] over k-contiguous storage
            g2[e] = d["w2"][e].clone().transpose(0, 1)
        else:
            g1[e] = d["w1"][e].transpose(0, 1).contiguous()  # logical [H, 2I], contiguous
            g2[e] = d["w2"][e].transpose(0, 1).contiguous()
        if dtype == "fp8":
            s1[e] = d["s1"][e].clone()
            s2[e] = d["s2"][e].clone()
    if dtype != "fp8":
        s1 = s2 = []
    call = lambda: ops.fused_deep_moe(d["x"], d["ids"], g1, s1, g2, s2, d["scales"], None, None, None, None,  # noqa: E731
                                      None, None, None, "ep", 1, 0, E, 0, 0)
    torch.cuda.synchronize()
    wbytes = sum(t.numel() * t.element_size() for t in g1 + g2)
    if layout == "reference_contiguous":
        call()                       # the one conversion per source tensor
        torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    out, _, etn = call()
    torch.cuda.synchronize()
    assert torch.cuda.max_memory_allocated() - base < wbytes // 4   # workspace and outputs only
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)) and torch.equal(etn, etn_ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            call()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout, _, getn = call()
    for r in range(3):
        junk = torch.randn(1 << 20, device="cuda") * r
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout.view(torch.int16), ref.view(torch.int16)), f"replay {r}"
        assert torch.equal(getn, etn_ref)
        del junk
    if layout == "reference_contiguous":
        # an in-place update of a source tensor (a new expert placement) is picked up by the next eager call
        g1[0].zero_()
        out2, _, _ = call()
        torch.cuda.synchronize()
        assert not torch.equal(out2.view(torch.int16), ref.view(torch.int16))


def test_fused_rejects_bad_weight_lists(ops):
    d = make(2, 8, 1024, 128, 8, 2, "bf16")
    g1 = list(d["w1"].transpose(1, 2).unbind(0))
    g2 = list(d["w2"].transpose(1, 2).unbind(0))
    with pytest.raises(RuntimeError, match="per-expert tensors"):
        ops.fused_deep_moe(d["x"], d["ids"], g1[:7], [], g2, [], d["scales"], None, None, None, None, None, None,
                           None, "ep", 1, 0, 8, 0, 0)
    with pytest.raises(RuntimeError, match="logical shape"):
        bad = g1[:7] + [torch.zeros(1024, 128, dtype=torch.bfloat16, device="cuda")]
        ops.fused_deep_moe(d["x"], d["ids"], bad, [], g2, [], d["scales"], None, None, None, None, None, None,
                           None, "ep", 1, 0, 8, 0, 0)


def test_fused_rejects_unsupported(ops):
    d = make(1, 4, 1024, 128, 8, 2, "bf16")
    with pytest.raises(RuntimeError, match="one EP rank"):
        ops.fused_deep_moe(d["x"], d["ids"], [d["w1"].transpose(1, 2)], [], [d["w2"].transpose(1, 2)], [],
                           d["scales"], None, None, None, None, None, None, None, "ep", 2, 0, 8, 0, 0)
    with pytest.raises(RuntimeError, match="not supported"):
        w = torch.zeros(8, 1024, 256, dtype=torch.float16, device="cuda")
        ops.fused_deep_moe(d["x"], d["ids"], [w], [], [w], [], d["scales"], None, None, None, None, None, None,
                           None, "ep", 1, 0, 8, 0, 0)
    with pytest.raises(RuntimeError, match="need int8 weights"):
        sm = torch.ones(8, 1024, device="cuda")
        ops.fused_deep_moe(d["x"], d["ids"], [d["w1"].transpose(1, 2)], [], [d["w2"].transpose(1, 2)], [],
                           d["scales"], None, None, None, None, sm, None, None, "ep", 1, 0, 8, 0, 0)


def test_fused_decode_fresh_inputs_and_forced_give_up(ops):
    """The decode path (layout and dispatch in one launch, then the chained GEMMs, whose GMM2 tiles read h
    written by other blocks of the same launch): consecutive calls on new activations and ids each time equal
    the small-op chain (a row of the previous call read from a stale cache would show); then, with every
    readiness wait made unreachable from the host and a 20 us bound, the call ends normally and reports through
    the sync status, and the next call is exact again."""
    from umdk_amd import _lib
    bs, H, I, E, K = 128, 2048, 256, 32, 8
    for seed in range(3):
        print(f"fused decode, fresh inputs: seed {seed}", flush=True)
        d = make(40 + seed, bs, H, I, E, K, "fp8")
        out, _, etn = call_fused(ops, d, E)
        ref, rtpe = chain_small_ops(ops, d, E, K)
        assert torch.equal(etn, rtpe)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    print("fused decode, forced give-up", flush=True)
    torch.cuda.synchronize()
    _lib.sync_status(clear=True)
    L = _lib.lib()
    L.camhipDebugSetSyncWait(2000, 1)
    try:
        call_fused(ops, d, E)
        torch.cuda.synchronize()
    finally:
        L.camhipDebugSetSyncWait(0, 0)
    assert _lib.sync_status(clear=True) != 0, "an unreachable wait did not report"
    out, _, etn = call_fused(ops, d, E)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)) and torch.equal(etn, rtpe)
    assert _lib.sync_status() == 0
