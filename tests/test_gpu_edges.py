"""GPU edge cases of the prefill ops and the fused entry: no tokens, every row on one expert, a fully
masked batch, and a grouped GEMM whose rows all belong to one group.

Expected values are closed forms: with identity experts and gates of 1/8 the combine returns x exactly
(x * 0.125 is exact and eight equal fp32 addends sum exactly); tokens that are masked or not routed
contribute nothing (the fused path skips expert ids < 0, cam_moe_distribute_combine.h:667-671).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import umdk_amd  # noqa: F401
    return torch.ops.umdk_cam_op_lib


def test_zero_tokens_through_the_prefill_ops(ops):
    print("edges: zero tokens", flush=True)
    E, K, H = 16, 4, 1024
    logits = torch.empty(0, E, device="cuda")
    idx, w = ops.moe_route(logits, None, K)
    assert tuple(idx.shape) == (0, K) and tuple(w.shape) == (0, K)
    nte, sti = ops.get_dispatch_layout(idx.long(), E, 1)
    assert torch.equal(nte.cpu(), torch.zeros(E, dtype=nte.dtype)) and sti.numel() == 0
    x = torch.empty(0, H, dtype=torch.bfloat16, device="cuda")
    for use_quant, mode in ((False, 0), (True, 3)):
        ex, sc, eidx, rc, rtpe = ops.moe_dispatch_prefill(x, idx, w, nte, sti, "ep", 0, 1, use_quant, mode)
        # as the reference binding: one placeholder row when nothing is received (moe_dispatch_prefill.cpp:111)
        assert ex.shape[0] == 1 and eidx.numel() == 3
        assert int(rc.cpu().sum()) == 0 and int(rtpe.cpu().sum()) == 0
        y = torch.zeros(1, H, dtype=torch.bfloat16, device="cuda")
        out = ops.moe_combine_prefill(y, idx, w, eidx, rc, "ep", 0, 1)
        assert tuple(out.shape) == (0, H)


def test_every_row_on_one_expert(ops):
    print("edges: all rows on expert 7", flush=True)
    T, H, E, K = 4096, 1024, 256, 8
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, H, generator=g).bfloat16().cuda()
    idx = torch.full((T, K), 7, dtype=torch.int32, device="cuda")
    w = torch.full((T, K), 0.125, dtype=torch.float32, device="cuda")
    nte, sti = ops.get_dispatch_layout(idx.long(), E, 1)
    assert int(nte[7]) == T * K and int(nte.sum()) == T * K
    assert torch.equal(sti.view(-1).cpu(), torch.arange(T * K, dtype=sti.dtype))   # stable rank = (t,k) order
    ex, _, eidx, rc, rtpe = ops.moe_dispatch_prefill(x, idx, w, nte, sti, "ep", 0, 1, False, 0)
    assert torch.equal(ex.view(T, K, H)[:, 3].view(torch.int16), x.view(torch.int16))
    out = ops.moe_combine_prefill(ex, idx, w, eidx, rc, "ep", 0, 1)               # identity experts
    assert torch.equal(out.view(torch.int16), x.view(torch.int16))


@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_grouped_gemm_all_rows_in_one_group(ops, dtype):
    print(f"edges: one group holds every row ({dtype})", flush=True)
    L, M, H, I = 32, 1536, 4096, 256
    g = torch.Generator(device="cuda").manual_seed(5)
    gl = torch.zeros(L, dtype=torch.int64, device="cuda")
    gl[19] = M                                  # GMM1: the 256-row tile class (>= 384 rows, >= 32 k-steps)
    x = torch.randn(M, H, device="cuda", generator=g)
    w1 = torch.randn(L, 2 * I, H, device="cuda", generator=g) * 0.03
    w2 = torch.randn(L, H, I, device="cuda", generator=g) * 0.03
    if dtype == "bf16":
        h, _ = ops.grouped_matmul_swiglu(x.bfloat16(), None, gl, w1.bfloat16(), None, 0)
        out = ops.grouped_matmul(h, None, gl, w2.bfloat16(), None)
        xr, w1r, w2r, tol = x.bfloat16().float(), w1[19].bfloat16().float(), w2[19].bfloat16().float(), 2e-2
        hr_in = h.float()
    else:
        def q_rows(t):
            v = t.view(t.shape[0], -1, 128)
            a = v.abs().amax(2).clamp(min=1e-4)
            return (v * (448.0 / a).unsqueeze(2)).to(torch.float8_e4m3fn).view_as(t), a / 448.0

        def q_w(t):
            n, k = t.shape[-2:]
            v = t.view(L, n // 128, 128, k // 128, 128)
            a = v.abs().amax((2, 4)).clamp(min=1e-4)
            q = (v * (448.0 / a)[:, :, None, :, None]).to(torch.float8_e4m3fn).view(L, n, k)
            return q, a / 448.0

        xq, xs = q_rows(x)
        w1q, w1s = q_w(w1)
        w2q, w2s = q_w(w2)
        h, hs = ops.grouped_matmul_swiglu(xq, xs, gl, w1q, w1s, 3)
        out = ops.grouped_matmul(h, hs, gl, w2q, w2s)
        xr = (xq.float().view(M, -1, 128) * xs.unsqueeze(2)).view(M, H)
        w1r = (w1q[19].float().view(2 * I // 128, 128, H // 128, 128) * w1s[19][:, None, :, None]).view(2 * I, H)
        w2r = (w2q[19].float().view(H // 128, 128, I // 128, 128) * w2s[19][:, None, :, None]).view(H, I)
        hr_in = (h.float().view(M, -1, 128) * hs.reshape(M, -1, 1)).view(M, I)
        tol = 5e-2
    gu = xr @ w1r.T
    hr = gu[:, :I] / (1 + torch.exp(-gu[:, :I])) * gu[:, I:]
    assert ((hr_in - hr).abs().max() / hr.abs().max()).item() < tol
    yr = hr_in @ w2r.T
    assert ((out.float() - yr).abs().max() / yr.abs().max()).item() < tol


@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_fused_fully_masked_batch(ops, dtype):
    print(f"edges: fused op with every token masked ({dtype})", flush=True)
    from tests.test_gpu_fused import call_fused, make
    bs, H, I, E, K = 24, 1024, 128, 8, 2
    d = make(7, bs, H, I, E, K, dtype)
    mask = torch.zeros(bs, dtype=torch.bool, device="cuda")
    out, _, etn = call_fused(ops, d, E, mask=mask)
    assert int(etn.abs().sum()) == 0
    assert int(out.view(torch.int16).abs().sum()) == 0 and out.shape == (bs, H)
