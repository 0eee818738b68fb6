"""Writes tests/golden/*.npz: small input/output vectors for the CAM MoE path,
computed with library routines only (torch.topk, torch.softmax, numpy stable
argsort, torch's float8_e4m3fn / bfloat16 casts, float64 matmul) -- not with
the oracle under test.  The reference ships no data files and no golden
vectors for this path (its tests draw unseeded random data at run time), so
these vectors restate the reference's own closed forms:

  * routing      -- the examples' torch.topk routing
                    (src/cam/examples/moe_dispatch_combine_prefill_sample.py:87-93)
  * layout       -- stable per-expert rank (dispatch_layout.h:112-161) ==
                    position of (t,k) in a stable sort of the flat topk_idx by expert
  * round robin  -- expert_ids = arange % E (test/cam/ut/fused_deep_moe/test_fused_deep_moe.py:298-302)
  * fp8 quant    -- DeepSeek-V3 per_token_cast_to_fp8 (1x128 blocks, amax clamp 1e-4)
  * int8 quant   -- moe_dispatch_normal.h:295-332 closed form rint(x*127/(amax+1e-12))
  * combine      -- identity experts: out = x * sum_k w (test_moe_dispatch_combine_prefill.py:163-168)
  * gemm         -- float64 matmul of dequantised operands, SwiGLU silu(g)*u

Run:  python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def route_ref(logits, bias, K):
    score = logits + bias if bias is not None else logits
    # stable descending order: sort by (-score, index)
    order = torch.sort(-score, dim=1, stable=True).indices[:, :K]
    p = torch.softmax(logits.double(), dim=1)
    w = torch.gather(p, 1, order)
    w = w / w.sum(1, keepdim=True)
    return order.int(), w.float()


def layout_ref(topk_idx, E):
    flat = topk_idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=E).astype(np.int32)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    pos = np.empty_like(order)
    pos[order] = np.arange(flat.size)
    sti = (pos - starts[flat]).astype(np.int32).reshape(topk_idx.shape)
    return counts, sti, pos.reshape(topk_idx.shape).astype(np.int32)


def fp8_quant_ref(x_bf16, H):
    x = x_bf16.float().view(x_bf16.shape[0], H // 128, 128)
    amax = x.abs().amax(dim=2).clamp(min=1e-4)
    # true IEEE division (torch's `448.0 / tensor` is reciprocal-then-multiply,
    # which differs in the last bit and flips RNE ties)
    inv = torch.div(torch.full_like(amax, 448.0), amax)
    q = (x * inv.unsqueeze(2)).to(torch.float8_e4m3fn)
    scale = torch.div(amax, torch.full_like(amax, 448.0))
    return q.view(x_bf16.shape[0], H).view(torch.uint8).numpy(), scale.numpy().astype(np.float32)


def int8_quant_ref(x_bf16):
    x = x_bf16.float()
    amax = x.abs().amax(dim=1, keepdim=True)
    s = torch.tensor(127.0) / (amax + torch.tensor(1e-12))
    q = torch.round(x * s).to(torch.int8)  # torch.round is half-to-even
    return q.numpy().view(np.uint8), (1.0 / s).squeeze(1).numpy().astype(np.float32)


def case_route_layout_dispatch(seed, T, H, E, K, with_bias):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).bfloat16()
    logits = torch.randn(T, E, generator=g)
    bias = (torch.randn(E, generator=g) * 0.5) if with_bias else None
    idx, w = route_ref(logits, bias, K)
    counts, sti, pos = layout_ref(idx.numpy().astype(np.int64), E)
    q8, s8 = fp8_quant_ref(x, H)
    qi, si = int8_quant_ref(x)
    # identity experts: y = dispatched bf16 rows, combine -> x * sum(w) rounded from fp32
    wsum = w.sum(1, keepdim=True)
    ident = (x.float() * wsum).bfloat16()
    out = dict(x=bf16_bits(x), logits=logits.numpy(), idx=idx.numpy(), w=w.numpy(),
               counts=counts, send_token_idx=sti, row_of=pos, fp8_codes=q8, fp8_scales=s8,
               int8_codes=qi, int8_scales=si, ident_out=bf16_bits(ident))
    if bias is not None:
        out["bias"] = bias.numpy()
    return out


def case_round_robin(T, E, K):
    ids = (np.arange(T * K) % E).reshape(T, K).astype(np.int64)
    counts = np.full(E, T * K // E, np.int32)
    counts[: (T * K) % E] += 1
    return dict(idx=ids, counts=counts)


def case_gemm(seed, Ms, H, I):
    g = torch.Generator().manual_seed(seed)
    L = len(Ms)
    M = sum(Ms)
    A = torch.randn(M, H, generator=g).bfloat16()
    W1 = (torch.randn(L, 2 * I, H, generator=g) * 0.02).bfloat16()
    W2 = (torch.randn(L, H, I, generator=g) * 0.02).bfloat16()
    hs, outs = [], []
    off = 0
    for e, m in enumerate(Ms):
        a = A[off:off + m].double()
        gu = a @ W1[e].double().T
        gg, uu = gu[:, :I].float(), gu[:, I:].float()
        h = (gg / (1 + torch.exp(-gg)) * uu).bfloat16()
        o = (h.double() @ W2[e].double().T).float().bfloat16()
        hs.append(h)
        outs.append(o)
        off += m
    return dict(A=bf16_bits(A), W1=bf16_bits(W1), W2=bf16_bits(W2), counts=np.array(Ms, np.int64),
                h=bf16_bits(torch.cat(hs)), out=bf16_bits(torch.cat(outs)))


def main():
    np.savez_compressed(os.path.join(HERE, "cfg1_tiny.npz"),
                        **case_route_layout_dispatch(1, 128, 1024, 8, 2, False))
    np.savez_compressed(os.path.join(HERE, "skew_bias.npz"),
                        **case_route_layout_dispatch(2, 64, 256, 64, 8, True))
    np.savez_compressed(os.path.join(HERE, "round_robin.npz"), **case_round_robin(16, 16, 8))
    np.savez_compressed(os.path.join(HERE, "gemm_bf16_small.npz"), **case_gemm(3, [5, 0, 17, 9], 256, 128))


if __name__ == "__main__":
    main()
