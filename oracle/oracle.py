"""ctypes wrapper around the C oracle (oracle/cam_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product package umdk_amd
never imports this module.

Arrays are numpy; bf16 tensors travel as uint16 bit patterns and fp8 e4m3fn
tensors as uint8 codes.  Each function cites the reference file:line its C
counterpart restates (see the header of cam_oracle.c).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libcamoracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_f32_to_e4m3.restype = ctypes.c_uint8
        _lib.orc_f32_to_e4m3.argtypes = [ctypes.c_float]
        _lib.orc_e4m3_to_f32.restype = ctypes.c_float
        _lib.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        _lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        _lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else ctypes.c_void_p(0)


def num_threads():
    """Threads of the oracle's token-parallel loops (route, dispatch, combine)."""
    return int(lib().orc_num_threads())


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def route(logits, bias, K):
    """R0: top-K of logit+bias (ties -> lower index), renormalised softmax gates."""
    logits = _c(logits, np.float32)
    T, E = logits.shape
    bias = None if bias is None else _c(bias, np.float32)
    idx = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float32)
    lib().orc_route(_p(logits), _p(bias), T, E, K, _p(idx), _p(w))
    return idx, w


def dispatch_layout(topk_idx, E, R):
    """D1 (dispatch_layout.h:112-161) -> (per_rank, per_expert, is_token_in_rank, send_token_idx)."""
    ti = _c(topk_idx, np.int64)
    T, K = ti.shape
    ntr = np.empty(R, np.int32)
    nte = np.empty(E, np.int32)
    itr = np.empty((T, R), np.int32)
    sti = np.empty((T, K), np.int32)
    lib().orc_dispatch_layout(_p(ti), T, K, E, R, _p(ntr), _p(nte), _p(itr), _p(sti))
    return ntr, nte, itr, sti


def notify_dispatch(counts):
    """D2 (notify_dispatch.h:143-152,340-360,389-412), one rank."""
    c = _c(counts, np.int32)
    E = c.shape[0]
    so = np.empty(E, np.int32)
    rc = np.empty(E, np.int32)
    rtpe = np.empty(E, np.int64)
    tot = np.zeros(1, np.int32)
    lib().orc_notify_dispatch(_p(c), E, _p(so), _p(rc), _p(rtpe), _p(tot))
    return so, rc, rtpe, int(tot[0])


QUANT_NONE, QUANT_INT8, QUANT_FP8 = 0, 2, 3


def dispatch(x_bf16, topk_idx, send_offset, send_token_idx, E, quant_mode, n_rows=None, rank=0):
    """D3 + Q1/Q2 (moe_dispatch_normal.h:295-332,335-344,381-398,545-591)."""
    x = _c(x_bf16, np.uint16)
    T, H = x.shape
    ti = _c(topk_idx, np.int32)
    K = ti.shape[1]
    if n_rows is None:
        n_rows = int(((ti >= 0) & (ti < E)).sum())
    if quant_mode == QUANT_NONE:
        ex = np.zeros((n_rows, H), np.uint16)
        sc = np.zeros(n_rows, np.float32)
    elif quant_mode == QUANT_INT8:
        ex = np.zeros((n_rows, H), np.uint8)
        sc = np.zeros(n_rows, np.float32)
    else:
        ex = np.zeros((n_rows, H), np.uint8)
        sc = np.zeros((n_rows, H // 128), np.float32)
    eidx = np.full((n_rows, 3), -7, np.int32)
    lib().orc_dispatch(_p(x), _p(ti), _p(_c(send_offset, np.int32)), _p(_c(send_token_idx, np.int32)),
                       T, H, K, E, rank, quant_mode, _p(ex), _p(sc), _p(eidx))
    return ex, sc, eidx


def dispatch_int8_fused(x_bf16, topk_idx, send_offset, send_token_idx, E, smooth=None, n_rows=None):
    """Fused-op int8 dispatch (cam_moe_distribute_dispatch.h:640-681): per destination row,
    optional smooth[e] multiply, s = 127/amax, q = rint(f*s), scale = 1/s -> (q, scale, expand_idx)."""
    x = _c(x_bf16, np.uint16)
    T, H = x.shape
    ti = _c(topk_idx, np.int32)
    K = ti.shape[1]
    if n_rows is None:
        n_rows = int(((ti >= 0) & (ti < E)).sum())
    ex = np.zeros((n_rows, H), np.int8)
    sc = np.zeros(n_rows, np.float32)
    eidx = np.full((n_rows, 3), -7, np.int32)
    sm = None if smooth is None else _c(smooth, np.float32)
    lib().orc_dispatch_int8_fused(_p(x), _p(ti), _p(_c(send_offset, np.int32)), _p(_c(send_token_idx, np.int32)),
                                  T, H, K, E, _p(sm), _p(ex), _p(sc), _p(eidx))
    return ex, sc, eidx


def combine(y_bf16, expand_idx, topk_idx, topk_w, E):
    """C1 (moe_combine_normal.h:343-377; cam_moe_distribute_combine.h:654-716)."""
    y = _c(y_bf16, np.uint16)
    N, H = y.shape
    ei = _c(expand_idx, np.int32).reshape(-1, 3)
    ti = _c(topk_idx, np.int32)
    w = _c(topk_w, np.float32)
    T, K = ti.shape
    out = np.empty((T, H), np.uint16)
    lib().orc_combine(_p(y), _p(ei), ei.shape[0], _p(ti), _p(w), T, K, E, H, _p(out))
    return out


def gmm1_swiglu_bf16(A, counts, W1):
    """G1+G2 bf16: W1 [L,2I,H] (gate rows then up rows), A [M,H] -> h [M,I] bf16."""
    A = _c(A, np.uint16)
    W1 = _c(W1, np.uint16)
    L, I2, H = W1.shape
    cnt = _c(counts, np.int64)
    M = int(cnt.sum())
    h = np.zeros((A.shape[0], I2 // 2), np.uint16)
    assert A.shape[0] >= M
    lib().orc_gmm1_swiglu_bf16(_p(A), _p(cnt), L, _p(W1), H, I2 // 2, _p(h))
    return h


def gmm2_bf16(Hin, counts, W2):
    """G3 bf16: W2 [L,H,I], Hin [M,I] -> out [M,H] bf16."""
    Hin = _c(Hin, np.uint16)
    W2 = _c(W2, np.uint16)
    L, H, I = W2.shape
    cnt = _c(counts, np.int64)
    out = np.zeros((Hin.shape[0], H), np.uint16)
    lib().orc_gmm2_bf16(_p(Hin), _p(cnt), L, _p(W2), I, H, _p(out))
    return out


def gmm1_swiglu_fp8(A, As, counts, W1, W1s):
    """G1+G2 fp8 block-scaled -> (hq [M,I] e4m3, hs [M,I/128])."""
    A = _c(A, np.uint8)
    As = _c(As, np.float32)
    W1 = _c(W1, np.uint8)
    W1s = _c(W1s, np.float32)
    L, I2, H = W1.shape
    I = I2 // 2
    cnt = _c(counts, np.int64)
    hq = np.zeros((A.shape[0], I), np.uint8)
    hs = np.zeros((A.shape[0], I // 128), np.float32)
    lib().orc_gmm1_swiglu_fp8(_p(A), _p(As), _p(cnt), L, _p(W1), _p(W1s), H, I, _p(hq), _p(hs))
    return hq, hs


def gmm2_fp8(Hq, Hs, counts, W2, W2s):
    """G3 fp8 block-scaled -> out [M,H] bf16."""
    Hq = _c(Hq, np.uint8)
    Hs = _c(Hs, np.float32)
    W2 = _c(W2, np.uint8)
    W2s = _c(W2s, np.float32)
    L, H, I = W2.shape
    cnt = _c(counts, np.int64)
    out = np.zeros((Hq.shape[0], H), np.uint16)
    lib().orc_gmm2_fp8(_p(Hq), _p(Hs), _p(cnt), L, _p(W2), _p(W2s), I, H, _p(out))
    return out


def f32_to_e4m3(x):
    return lib().orc_f32_to_e4m3(float(x))


def e4m3_to_f32(c):
    return lib().orc_e4m3_to_f32(int(c))


def bf16_to_f32(u16):
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f):
    """Vectorised RNE fp32 -> bf16 bits (NaN-free inputs)."""
    u = np.asarray(f, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def e4m3_table():
    """All 256 e4m3fn codes decoded to float32 (NaN at 0x7f/0xff)."""
    return np.array([lib().orc_e4m3_to_f32(c) for c in range(256)], np.float32)


def gmm1_swiglu_int8(A, As, counts, W1, W1s):
    """int8 GMM1 + SwiGLU with per-channel / per-token dequant -> h fp32 [M, I]."""
    A = _c(A, np.int8)
    W1 = _c(W1, np.int8)
    L, I2, H = W1.shape
    h = np.zeros((A.shape[0], I2 // 2), np.float32)
    lib().orc_gmm1_swiglu_int8(_p(A), _p(_c(As, np.float32)), _p(_c(counts, np.int64)), L, _p(W1),
                               _p(_c(W1s, np.float32)), H, I2 // 2, _p(h))
    return h


def quant_rows_int8(h):
    """Per-token int8 requant of h (post_swiglu_dynamic_quant.h:164-231) -> (q int8, scale)."""
    h = _c(h, np.float32)
    M, I = h.shape
    q = np.zeros((M, I), np.int8)
    s = np.zeros(M, np.float32)
    lib().orc_quant_rows_int8(_p(h), M, I, _p(q), _p(s))
    return q, s


def gmm2_int8(Hq, Hs, counts, W2, W2s):
    """int8 GMM2 with per-channel / per-token dequant -> bf16 [M, H]."""
    Hq = _c(Hq, np.int8)
    W2 = _c(W2, np.int8)
    L, H, I = W2.shape
    out = np.zeros((Hq.shape[0], H), np.uint16)
    lib().orc_gmm2_int8(_p(Hq), _p(_c(Hs, np.float32)), _p(_c(counts, np.int64)), L, _p(W2),
                        _p(_c(W2s, np.float32)), I, H, _p(out))
    return out
