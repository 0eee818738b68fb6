"""torch.ops.umdk_cam_op_lib -- CAM's operator surface on MI355X.

Same library name, op names, argument names, order and defaults as the
reference's TORCH_LIBRARY block (src/cam/comm_operator/pybind/pybind.cpp:21-36),
registered for the GPU dispatch key and backed by libcamhip.so through its C
ABI.  Like the reference bindings (pybind/get_dispatch_layout.cpp:33-60,
moe_dispatch_prefill.cpp:38-127, moe_combine_prefill.cpp:28-64), each op
casts index/weight dtypes, checks shapes, allocates outputs and launches on
the current stream; a failed check raises RuntimeError, as TORCH_BIND_ASSERT
raises TorchBindException (torch_bind_exception.h:20-40).

Differences, all documented in the op docstrings:
  * num_ranks must be 1 (one EP rank per GPU, no collectives); the reference
    requires 2..384.
  * moe_dispatch_prefill takes an extra trailing `quant_mode` (default -1 =
    follow use_quant as the reference does: 2 if use_quant else 0); 3 selects
    FP8 e4m3fn rows with [rows, hidden/128] fp32 block scales.
  * moe_route (routing) and grouped expert GEMM ops are additions with no
    reference counterpart.
"""
import weakref

import torch

from . import _lib

LIB_NAME = "umdk_cam_op_lib"

_def = torch.library.Library(LIB_NAME, "DEF")
_def.define("get_dispatch_layout(Tensor topk_idx, int num_experts, int num_ranks) -> (Tensor, Tensor)")
_def.define(
    "moe_dispatch_prefill(Tensor x, Tensor topk_idx, Tensor topk_weights, Tensor num_tokens_per_expert, "
    "Tensor send_token_idx_small, str group_ep, int rank, int num_ranks, bool use_quant, int quant_mode=-1) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")
_def.define(
    "moe_combine_prefill(Tensor x, Tensor topk_idx, Tensor topk_weights, Tensor src_idx, Tensor send_head, "
    "str group_ep, int rank, int num_ranks) -> Tensor")
_def.define("moe_route(Tensor logits, Tensor? bias, int topk) -> (Tensor, Tensor)")
_def.define("grouped_matmul_swiglu(Tensor x, Tensor? x_scale, Tensor group_list, Tensor weight, "
            "Tensor? weight_scale, int out_quant=0) -> (Tensor, Tensor)")
_def.define("grouped_matmul(Tensor x, Tensor? x_scale, Tensor group_list, Tensor weight, Tensor? weight_scale) "
            "-> Tensor")

_def.define(
    "fused_deep_moe(Tensor x, Tensor expert_ids, Tensor[] gmm1_weight, Tensor[] gmm1_weight_scale, "
    "Tensor[] gmm2_weight, Tensor[] gmm2_weight_scale, Tensor expert_scales, "
    "Tensor? share_gmm1_weight, Tensor? share_gmm1_weight_scale, "
    "Tensor? share_gmm2_weight, Tensor? share_gmm2_weight_scale, "
    "Tensor? expert_smooth_scales, Tensor? share_smooth_scales, Tensor? x_active_mask, "
    "str group_ep, int ep_rank_size, int ep_rank_id, int moe_expert_num, "
    "int quant_mode, int global_bs) -> Tensor[]")

_impl = torch.library.Library(LIB_NAME, "IMPL", "CUDA")
_meta = torch.library.Library(LIB_NAME, "IMPL", "Meta")

QUANT_NONE, QUANT_INT8_TOKEN, QUANT_FP8_BLOCK = 0, 2, 3
WEIGHT_LIST = 0x100  # OR'ed into the fused entry's weight dtype: per-expert weight pointer tables
QUANT_FP8_BLOCK_KMAJOR = 5  # C-ABI dispatch only: fp8 rows with k-major block scales (the GEMMs' layout)


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _single_rank(rank, num_ranks, op):
    _check(num_ranks == 1 and rank == 0,
           f"{op}: this build runs one EP rank per GPU without collectives; "
           f"num_ranks must be 1 and rank 0 (got num_ranks={num_ranks}, rank={rank})")


def get_dispatch_layout(topk_idx, num_experts, num_ranks):
    """Per-expert token counts and stable per-expert rank of every (t,k).

    Mirrors GetDispatchLayoutImplNpu (pybind/get_dispatch_layout.cpp:33-60):
    returns (num_tokens_per_expert [E] int32, send_token_idx [T,K] int32)."""
    ti = topk_idx if topk_idx.dtype == torch.int64 else topk_idx.to(torch.int64)
    _check(ti.dim() == 2, "get_dispatch_layout: topk_idx must be 2-D")
    _check(ti.is_contiguous(), "get_dispatch_layout: topk_idx must be contiguous")
    _check(num_experts > 0, "get_dispatch_layout: num_experts must be > 0")
    T, K = ti.shape
    dev = ti.device
    nte = torch.empty(num_experts, dtype=torch.int32, device=dev)
    sti = torch.empty((T, K), dtype=torch.int32, device=dev)
    _lib.call("camhipDispatchLayout", _lib.ptr(ti), T, num_ranks, num_experts, K, None, _lib.ptr(nte), None,
              _lib.ptr(sti), device=dev)
    return nte, sti


def _notify(num_tokens_per_expert, T, device):
    E = num_tokens_per_expert.shape[0]
    i32 = dict(dtype=torch.int32, device=device)
    send_offset = torch.empty(E, **i32)
    total = torch.empty(1, **i32)
    recv_count = torch.empty(E, **i32)
    recv_offset = torch.empty(E, **i32)
    max_bs = torch.empty(1, **i32)
    rtpe = torch.empty(E, dtype=torch.int64, device=device)
    _lib.call("camhipNotifyDispatch", _lib.ptr(num_tokens_per_expert), E, T, 1, 0, _lib.ptr(send_offset),
              _lib.ptr(total), _lib.ptr(recv_count), _lib.ptr(recv_offset), _lib.ptr(max_bs), _lib.ptr(rtpe),
              device=device)
    return send_offset, total, recv_count, recv_offset, rtpe


def moe_dispatch_prefill(x, topk_idx, topk_weights, num_tokens_per_expert, send_token_idx_small, group_ep, rank,
                         num_ranks, use_quant, quant_mode=-1):
    """Permute tokens by expert (with optional fused quantisation).

    Mirrors MoeDispatchPrefillImplNpu (pybind/moe_dispatch_prefill.cpp:38-127):
    count exchange, a host read of the received row count to size the outputs
    (as the reference does at :110-111), then the dispatch kernel.  Returns
    (expand_x [N,H], dynamic_scales, expand_idx [3N] int32, recv_count [E]
    int32, recv_tokens_per_expert [E] int64).  quant_mode: -1 follows
    use_quant (2 if set, else 0); 0 bf16 rows; 2 int8 rows + [N] scales; 3 fp8
    e4m3fn rows + [N, H/128] scales."""
    ti = topk_idx if topk_idx.dtype == torch.int32 else topk_idx.to(torch.int32)
    if quant_mode < 0:
        quant_mode = QUANT_INT8_TOKEN if use_quant else QUANT_NONE
    _check(quant_mode in (QUANT_NONE, QUANT_INT8_TOKEN, QUANT_FP8_BLOCK),
           f"moe_dispatch_prefill: quant_mode {quant_mode} not supported")
    _check(num_tokens_per_expert.dtype == torch.int32, "moe_dispatch_prefill: num_tokens_per_expert must be int32")
    _single_rank(rank, num_ranks, "moe_dispatch_prefill")
    _check(x.dim() == 2 and x.is_contiguous(), "moe_dispatch_prefill: x must be 2-D and contiguous")
    _check(x.dtype == torch.bfloat16, "moe_dispatch_prefill: x must be bfloat16")
    _check(num_tokens_per_expert.dim() == 1 and num_tokens_per_expert.is_contiguous(),
           "moe_dispatch_prefill: num_tokens_per_expert must be 1-D and contiguous")
    _check(num_tokens_per_expert.shape[0] % num_ranks == 0,
           "moe_dispatch_prefill: num_experts must be divisible by num_ranks")
    T, H = x.shape
    E = num_tokens_per_expert.shape[0]
    _check(E > 0, "moe_dispatch_prefill: num_experts must be > 0")
    _check(ti.dim() == 2 and ti.is_contiguous(), "moe_dispatch_prefill: topk_idx must be 2-D and contiguous")
    _check(topk_weights.dim() == 2 and topk_weights.is_contiguous(),
           "moe_dispatch_prefill: topk_weights must be 2-D and contiguous")
    K = ti.shape[1]
    _check(ti.shape[0] == T and send_token_idx_small.shape[0] == T, "moe_dispatch_prefill: token count mismatch")
    _check(topk_weights.shape[1] == K and send_token_idx_small.shape[1] == K, "moe_dispatch_prefill: topk mismatch")
    dev = x.device
    send_offset, total, recv_count, recv_offset, rtpe = _notify(num_tokens_per_expert, T, dev)
    n_recv = int(total.item())
    n_rows = max(n_recv, 1)
    if quant_mode == QUANT_NONE:
        expand_x = torch.empty((n_rows, H), dtype=x.dtype, device=dev)
        scales = torch.empty(n_rows, dtype=torch.float32, device=dev)
    elif quant_mode == QUANT_INT8_TOKEN:
        expand_x = torch.empty((n_rows, H), dtype=torch.int8, device=dev)
        scales = torch.empty(n_rows, dtype=torch.float32, device=dev)
    else:
        expand_x = torch.empty((n_rows, H), dtype=torch.float8_e4m3fn, device=dev)
        scales = torch.empty((n_rows, H // 128), dtype=torch.float32, device=dev)
    expand_idx = torch.empty(n_rows * 3, dtype=torch.int32, device=dev)
    sti = send_token_idx_small if send_token_idx_small.dtype == torch.int32 else send_token_idx_small.to(torch.int32)
    _lib.call("camhipMoeDispatchNormal", _lib.ptr(x), _lib.ptr(ti), _lib.ptr(send_offset), _lib.ptr(sti.contiguous()),
              _lib.ptr(recv_offset), _lib.ptr(recv_count), T, H, K, 1, 0, E, quant_mode, n_rows, _lib.ptr(expand_x),
              _lib.ptr(scales), _lib.ptr(expand_idx), None, device=dev)
    return expand_x, scales, expand_idx, recv_count, rtpe


def moe_combine_prefill(x, topk_idx, topk_weights, src_idx, send_head, group_ep, rank, num_ranks):
    """Weighted unpermute back to token order.

    Mirrors MoeCombinePrefillImplNpu (pybind/moe_combine_prefill.cpp:28-64):
    x [N,H] bf16 expert outputs in dispatch order, src_idx = expand_idx from
    dispatch, send_head = recv_count; returns [T,H] with
    out[t] = bf16(sum_k x[row(t,k)] * w[t,k]) accumulated in fp32."""
    _single_rank(rank, num_ranks, "moe_combine_prefill")
    _check(x.dim() == 2 and x.is_contiguous(), "moe_combine_prefill: x must be 2-D and contiguous")
    _check(x.dtype == torch.bfloat16, "moe_combine_prefill: x must be bfloat16")
    w = topk_weights if topk_weights.dtype == torch.float32 else topk_weights.to(torch.float32)
    w = w.contiguous()
    T, K = w.shape
    N, H = x.shape
    _check(src_idx.numel() >= 3 * N, "moe_combine_prefill: src_idx must hold 3 ints per row")
    _check(src_idx.dtype == torch.int32, "moe_combine_prefill: src_idx must be int32")
    E = send_head.shape[0]
    out = torch.empty((T, H), dtype=x.dtype, device=x.device)
    sh = send_head if send_head.dtype == torch.int32 else send_head.to(torch.int32)
    _lib.call("camhipMoeCombineNormal", _lib.ptr(x), _lib.ptr(src_idx.contiguous()), N, _lib.ptr(sh.contiguous()),
              _lib.ptr(w), T, K, H, 1, 0, E, _lib.ptr(out), None, device=x.device)
    return out


def moe_route(logits, bias, topk):
    """Top-K routing (addition; no reference counterpart): returns
    (topk_idx [T,K] int32, topk_weights [T,K] fp32); ties go to the lower id."""
    _check(logits.dim() == 2 and logits.dtype == torch.float32, "moe_route: logits must be [T,E] float32")
    lg = logits.contiguous()
    T, E = lg.shape
    b = None
    if bias is not None:
        _check(bias.dtype == torch.float32 and bias.numel() == E, "moe_route: bias must be [E] float32")
        b = bias.contiguous()
    idx = torch.empty((T, topk), dtype=torch.int32, device=lg.device)
    w = torch.empty((T, topk), dtype=torch.float32, device=lg.device)
    _lib.call("camhipMoeRoute", _lib.ptr(lg), _lib.ptr(b), T, E, topk, _lib.ptr(idx), _lib.ptr(w), None,
              device=lg.device)
    return idx, w


def _gmm_common(x, x_scale, group_list, weight, weight_scale, op):
    _check(x.dim() == 2 and x.is_contiguous(), f"{op}: x must be 2-D and contiguous")
    _check(weight.dim() == 3 and weight.is_contiguous(), f"{op}: weight must be [groups, n, k] contiguous")
    _check(group_list.dtype == torch.int64 and group_list.dim() == 1, f"{op}: group_list must be 1-D int64")
    L, n, k = weight.shape
    _check(group_list.numel() == L, f"{op}: group_list has {group_list.numel()} groups, weight {L}")
    _check(x.shape[1] == k, f"{op}: x has {x.shape[1]} columns, weight k = {k}")
    if x.dtype == torch.bfloat16:
        _check(weight.dtype == torch.bfloat16, f"{op}: bf16 x needs bf16 weight")
        dt = 0
    elif x.dtype == torch.int8:
        _check(weight.dtype == torch.int8, f"{op}: int8 x needs int8 weight")
        _check(x_scale is not None and weight_scale is not None, f"{op}: int8 needs x_scale and weight_scale")
        _check(x_scale.dtype == torch.float32 and tuple(x_scale.shape) == (x.shape[0],),
               f"{op}: int8 x_scale must be float32 [m] (per token)")
        _check(weight_scale.dtype == torch.float32 and tuple(weight_scale.shape) == (L, n),
               f"{op}: int8 weight_scale must be float32 [groups, n] (per channel)")
        dt = 2
    else:
        _check(x.dtype == torch.float8_e4m3fn and weight.dtype == torch.float8_e4m3fn,
               f"{op}: x and weight must both be bfloat16, int8 or float8_e4m3fn")
        _check(x_scale is not None and weight_scale is not None, f"{op}: fp8 needs x_scale and weight_scale")
        _check(x_scale.dtype == torch.float32 and tuple(x_scale.shape) == (x.shape[0], k // 128),
               f"{op}: x_scale must be float32 [m, k/128]")
        _check(x_scale.is_contiguous() or x_scale.t().is_contiguous(),
               f"{op}: x_scale must be row-major [m, k/128] or the transpose of a contiguous [k/128, m]")
        _check(weight_scale.dtype == torch.float32 and tuple(weight_scale.shape) == (L, n // 128, k // 128),
               f"{op}: weight_scale must be float32 [groups, n/128, k/128]")
        dt = 3
    return dt, L, n, k


def _x_scale_layout(x_scale):
    # 1: fp8 block scales stored k-major ([k/128, m] contiguous, the layout the kernels read); 0: row-major
    if x_scale is None or x_scale.dim() != 2 or x_scale.is_contiguous():
        return 0
    return 1


def grouped_matmul_swiglu(x, x_scale, group_list, weight, weight_scale, out_quant=0):
    """GMM1 + SwiGLU over ragged expert groups (addition; the reference runs
    this stage inside fused_deep_moe, grouped_matmul_slice_m_per_token_dequant_
    swiglu_quant_multistage_workspace.h:299-455).  weight [L, 2I, k]: rows
    [0,I) gate, [I,2I) up.  Returns (h [m, I], h_scale): bf16 h and an empty
    scale for out_quant=0; fp8 h and [m, I/128] scales for out_quant=3; for int8
    x and weights (per-token x_scale [m], per-channel weight_scale [L, 2I]),
    out_quant must be 2: int8 h requantised per token with scales [m]
    (post_swiglu_dynamic_quant.h:164-231).  fp8 x_scale may be row-major or
    the transpose of a contiguous [k/128, m]; the fp8 h_scale is returned as
    such a transpose (k-major storage, which grouped_matmul reads directly)."""
    dt, L, n, k = _gmm_common(x, x_scale, group_list, weight, weight_scale, "grouped_matmul_swiglu")
    m = x.shape[0]
    I = n // 2
    if dt == 2:
        _check(out_quant == QUANT_INT8_TOKEN, "grouped_matmul_swiglu: int8 inputs need out_quant=2")
        h = torch.empty((m, I), dtype=torch.int8, device=x.device)
        hs = torch.empty((m,), dtype=torch.float32, device=x.device)
    elif out_quant == QUANT_FP8_BLOCK:
        h = torch.empty((m, I), dtype=torch.float8_e4m3fn, device=x.device)
        hs = torch.empty((I // 128, m), dtype=torch.float32, device=x.device).t()
    else:
        _check(out_quant == QUANT_NONE, "grouped_matmul_swiglu: out_quant must be 0 or 3")
        h = torch.empty((m, I), dtype=torch.bfloat16, device=x.device)
        hs = torch.empty(0, dtype=torch.float32, device=x.device)
    _lib.call("camhipGroupedMatmulSwiglu", _lib.ptr(x), _lib.ptr(x_scale, True), _lib.ptr(group_list), L, m, k, n,
              _lib.ptr(weight), _lib.ptr(weight_scale), dt, _x_scale_layout(x_scale), out_quant, _lib.ptr(h),
              _lib.ptr(hs, True) if out_quant else None, device=x.device)
    return h, hs


def grouped_matmul(x, x_scale, group_list, weight, weight_scale):
    """GMM2 over ragged expert groups: out[m, n] = bf16(x W^T) (addition; the
    reference's grouped_matmul_slice_m_per_token_dequant_multistage_workspace.h:141-292).
    int8: out = bf16(((float)acc * weight_scale[g, n]) * x_scale[m])."""
    dt, L, n, k = _gmm_common(x, x_scale, group_list, weight, weight_scale, "grouped_matmul")
    m = x.shape[0]
    out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    _lib.call("camhipGroupedMatmul", _lib.ptr(x), _lib.ptr(x_scale, True), _lib.ptr(group_list), L, m, k, n,
              _lib.ptr(weight), _lib.ptr(weight_scale), dt, _x_scale_layout(x_scale), _lib.ptr(out),
              device=x.device)
    return out


def prepack_weight(w_lkn):
    """Reference logical layout [L, k, n] (e.g. W1 [L, H, 2I], API guide
    doc/en/cam/CAM API Guide.md:183-186) -> the [L, n, k] k-contiguous layout
    the grouped GEMMs read.  A one-time copy at weight load."""
    return w_lkn.transpose(1, 2).contiguous()


_CONVERTED = {}


def _converted(src, tag, make):
    """A layout or dtype conversion of a weight-like input, made once per source tensor.

    The result is cached on the source tensor object and its version counter, so a caller that passes
    the same weights on every step (the reference's dynamic-EPLB lists, test_fused_deep_moe.py:256-269)
    pays the copy once and keeps one stable device address (a captured graph reads it).  After the source is
    modified in place, the next eager call refreshes the copy in place (same address, so graphs captured on it
    replay the new values from then on; the refresh first waits for the device, so no replay in flight reads a
    half-updated copy).  The entry is dropped when the source is freed.  A conversion first
    needed inside graph capture is refused: the copy would land in the graph's private pool."""
    key = (id(src), tag)
    ent = _CONVERTED.get(key)
    if ent is not None and ent[0]() is src and ent[1] == src._version:
        return ent[2]
    _check(not (src.is_cuda and torch.cuda.is_current_stream_capturing()),
           f"fused_deep_moe: {tag} needs a converted copy (layout or dtype) that cannot be made inside graph "
           "capture; run the call once eagerly before capturing, or pass the kernels' own layout")
    if ent is not None and ent[0]() is src:
        # the source changed in place: refresh the copy in place, so graphs captured on it see the new values.
        # A graph replay still reading the copy may be in flight on any stream of the device: wait for the
        # device first, so the replay never reads a half-updated weight (a rare path: weights change rarely)
        out = ent[2]
        if out.is_cuda:
            torch.cuda.synchronize(out.device)
        out.copy_(make())
        _CONVERTED[key] = (ent[0], src._version, out)
        return out
    out = make()

    def _drop(_ref, key=key):
        _CONVERTED.pop(key, None)

    _CONVERTED[key] = (weakref.ref(src, _drop), src._version, out)
    return out


def _contig(t, tag, dtype=None):
    """t as a contiguous tensor of `dtype` (default: its own), converted once per source (see _converted)."""
    dtype = t.dtype if dtype is None else dtype
    if t.dtype == dtype and t.is_contiguous():
        return t
    return _converted(t, tag, lambda: t.to(dtype).contiguous())


def _kmajor(w, n, k, what):
    """A weight given in the reference's logical [..., k, n] shape -> contiguous storage with k contiguous
    ([..., n, k]).  A transposed view of such storage is used as is; a contiguous [..., k, n] tensor is
    transposed once per source tensor (a cached copy, see _converted)."""
    if tuple(w.shape[-2:]) == (k, n):
        t = w.transpose(-1, -2)
        if t.is_contiguous():
            return t                       # already k-contiguous underneath: no copy
        return _converted(w, what, lambda: t.contiguous())
    raise RuntimeError(f"fused_deep_moe: {what} must have logical shape [..., {k}, {n}], got {tuple(w.shape)}")


def _is_coupled(ws):
    return len(ws) == 1 and ws[0].dim() == 3


def _coupled(ws, L, n, k, what):
    w = _kmajor(ws[0], n, k, what)
    _check(tuple(w.shape) == (L, n, k), f"fused_deep_moe: {what} shape mismatch")
    return w


def _scales(ss, L, n, k, what):
    """fp8 128x128 block scales [L, n/128, k/128] (one coupled tensor)."""
    if not ss or ss[0] is None:
        return None
    s = ss[0]
    _check(s.dim() == 3 and s.dtype == torch.float32 and tuple(s.shape) == (L, n // 128, k // 128),
           f"fused_deep_moe: {what} must be float32 [{L}, {n // 128}, {k // 128}] (128x128 block scales)")
    return _contig(s, what)


def _channel_scales(ss, L, n, what):
    """int8 per-channel scales [L, n] (one coupled tensor); cast to float32 as the reference's
    test builds them in float (test_fused_deep_moe.py:309-312)."""
    _check(bool(ss) and ss[0] is not None, f"fused_deep_moe: int8 weights need {what}")
    s = ss[0]
    _check(s.dim() == 2 and tuple(s.shape) == (L, n), f"fused_deep_moe: {what} must be [{L}, {n}] per-channel scales")
    return _contig(s, what, torch.float32)


def _per_expert(ws, L, what, coupled_dim):
    """The L per-expert tensors of a weight argument: the reference's separated lists as given, or
    the slices of one coupled tensor (views, no copy)."""
    _check(bool(ws) and ws[0] is not None, f"fused_deep_moe: {what} missing")
    if len(ws) == 1 and ws[0].dim() == coupled_dim:
        _check(ws[0].shape[0] == L, f"fused_deep_moe: {what} holds {ws[0].shape[0]} experts, need {L}")
        return list(ws[0].unbind(0))
    _check(len(ws) == L, f"fused_deep_moe: {what} needs 1 coupled tensor or {L} per-expert tensors, got {len(ws)}")
    return list(ws)


_PTR_TABLES = {}
_PTR_PINNED = set()   # tables a captured graph may read: never freed


def _ptr_table(ts, device):
    """Device array of the tensors' data pointers (int64), cached by the pointer values so that a
    steady caller (and a captured graph) reuses one table.  A table used during graph capture is
    kept for the life of the process; other tables are dropped when the cache fills."""
    key = (str(device),) + tuple(t.data_ptr() for t in ts)
    tab = _PTR_TABLES.get(key)
    capturing = torch.device(device).type == "cuda" and torch.cuda.is_current_stream_capturing()
    if tab is None:
        _check(not capturing, "fused_deep_moe: separated weights first seen inside graph capture; "
               "run the call once before capturing (its pointer table is built eagerly)")
        if len(_PTR_TABLES) >= 256:
            for k in [k for k in _PTR_TABLES if k not in _PTR_PINNED]:
                del _PTR_TABLES[k]
        tab = torch.tensor(key[1:], dtype=torch.int64).to(device)
        _PTR_TABLES[key] = tab
    if capturing:
        _PTR_PINNED.add(key)
    elif tab.is_cuda:
        # a cached table may be reused from another stream: the allocator must not hand its memory out
        # again (after the cache drops it) before that stream's reads are done
        tab.record_stream(torch.cuda.current_stream(tab.device))
    return tab


def _separated(ws, ss, L, n, k, fp8, int8, what, device):
    """Separated mode (the reference's per-expert TensorList weights, dynamic EPLB:
    test_fused_deep_moe.py:256-269): no stacking copy; the kernels read each expert through a
    device pointer table.  Returns (weight table, scale table or None, tensors to keep alive)."""
    we = [_kmajor(t, n, k, what) for t in _per_expert(ws, L, what, 3)]
    for t in we:
        _check(tuple(t.shape) == (n, k) and t.is_contiguous() and t.device == device,
               f"fused_deep_moe: each {what} must be [{k}, {n}] with one expert per tensor on {device}")
    keep = list(we)
    st = None
    if fp8 or int8:
        sname = what + "_scale"
        se = _per_expert(ss, L, sname, 3 if fp8 else 2)
        if fp8:
            se = [_contig(t, sname) for t in se]
            for t in se:
                _check(t.dtype == torch.float32 and tuple(t.shape) == (n // 128, k // 128),
                       f"fused_deep_moe: each {sname} must be float32 [{n // 128}, {k // 128}]")
        else:
            se = [_contig(t, sname, torch.float32).view(-1) for t in se]
            for t in se:
                _check(t.numel() == n, f"fused_deep_moe: each {sname} must have {n} per-channel scales")
        keep += se
        st = _ptr_table(se, device)
    return _ptr_table(we, device), st, keep


def fused_deep_moe(x, expert_ids, gmm1_weight, gmm1_weight_scale, gmm2_weight, gmm2_weight_scale, expert_scales,
                   share_gmm1_weight, share_gmm1_weight_scale, share_gmm2_weight, share_gmm2_weight_scale,
                   expert_smooth_scales, share_smooth_scales, x_active_mask, group_ep, ep_rank_size, ep_rank_id,
                   moe_expert_num, quant_mode, global_bs):
    """Decode MoE layer in one call: dispatch + GMM1 + SwiGLU + GMM2 + combine
    (+ shared expert), returning [output, share_output, expert_token_nums].

    Mirrors FusedDeepMoeImplNpu (pybind/fused_deep_moe.cpp:30-83) and the API
    guide (doc/en/cam/CAM API Guide.md:177-226): weights in the logical
    [L, H, 2I] / [L, I, H] shapes (one coupled tensor, or L separated ones
    read in place through device pointer tables; a transposed view of
    k-contiguous storage avoids a copy), expert_ids
    int32 with -1 placeholders, x_active_mask a true-prefix bool mask.
    Weights are int8 with per-channel scales [L, 2I] / [L, H] -- the
    reference's own mode, with optional smooth-quant scales
    expert_smooth_scales [moe_expert_num, H] and share_smooth_scales [H] --,
    bf16, or float8_e4m3fn with 128x128 block scales [L, n/128, k/128].
    Output shapes are fixed by the inputs, so the op can be captured in a
    graph."""
    _check(x.dim() == 2 and x.dtype == torch.bfloat16 and x.is_contiguous(),
           "fused_deep_moe: x must be a contiguous [batch, hidden] bfloat16 tensor")
    _check(expert_ids.dim() == 2, "fused_deep_moe: expert_ids must be 2-D")
    _single_rank(ep_rank_id, ep_rank_size, "fused_deep_moe")
    bs, h = x.shape
    k = expert_ids.shape[1]
    L = moe_expert_num // ep_rank_size
    dt = gmm1_weight[0].dtype
    _check(dt in (torch.bfloat16, torch.int8, torch.float8_e4m3fn),
           f"fused_deep_moe: weight dtype {dt} not supported (int8, bfloat16 or float8_e4m3fn)")
    w1_logical = gmm1_weight[0].shape
    n1 = w1_logical[-1]
    I = n1 // 2
    fp8 = dt == torch.float8_e4m3fn
    int8 = dt == torch.int8
    separated = not (_is_coupled(gmm1_weight) and _is_coupled(gmm2_weight))
    s1 = s2 = None
    keep = []
    if separated:
        w1, s1, k1 = _separated(gmm1_weight, gmm1_weight_scale, L, n1, h, fp8, int8, "gmm1_weight", x.device)
        w2, s2, k2 = _separated(gmm2_weight, gmm2_weight_scale, L, h, I, fp8, int8, "gmm2_weight", x.device)
        keep = k1 + k2  # noqa: F841 -- per-expert tensors stay alive until the launch is queued
    else:
        w1 = _coupled(gmm1_weight, L, n1, h, "gmm1_weight")
        w2 = _coupled(gmm2_weight, L, h, I, "gmm2_weight")
    if separated:
        pass  # tables built above
    elif fp8:
        s1 = _scales(gmm1_weight_scale, L, n1, h, "gmm1_weight_scale")
        s2 = _scales(gmm2_weight_scale, L, h, I, "gmm2_weight_scale")
    elif int8:
        s1 = _channel_scales(gmm1_weight_scale, L, n1, "gmm1_weight_scale")
        s2 = _channel_scales(gmm2_weight_scale, L, h, "gmm2_weight_scale")
    smooth = share_smooth = None
    if expert_smooth_scales is not None:
        _check(int8, "fused_deep_moe: expert_smooth_scales need int8 weights")
        _check(tuple(expert_smooth_scales.shape) == (moe_expert_num, h),
               f"fused_deep_moe: expert_smooth_scales must be [{moe_expert_num}, {h}]")
        smooth = _contig(expert_smooth_scales, "expert_smooth_scales", torch.float32)
    if share_smooth_scales is not None and share_gmm1_weight is not None:   # ignored without a shared expert
        _check(int8, "fused_deep_moe: share_smooth_scales need int8 weights")
        _check(share_smooth_scales.numel() == h, f"fused_deep_moe: share_smooth_scales must have {h} elements")
        share_smooth = _contig(share_smooth_scales, "share_smooth_scales", torch.float32).view(h)
    shared = share_gmm1_weight is not None
    sw1 = sw2 = ss1 = ss2 = None
    nsh = 0
    if shared:
        _check(share_gmm2_weight is not None, "fused_deep_moe: share_gmm2_weight missing")
        nsh = share_gmm1_weight.shape[-1]
        sw1 = _kmajor(share_gmm1_weight, nsh, h, "share_gmm1_weight")
        sw2 = _kmajor(share_gmm2_weight, h, nsh // 2, "share_gmm2_weight")
        if fp8:
            ss1 = _contig(share_gmm1_weight_scale, "share_gmm1_weight_scale")
            ss2 = _contig(share_gmm2_weight_scale, "share_gmm2_weight_scale")
        elif int8:
            _check(share_gmm1_weight_scale is not None and share_gmm2_weight_scale is not None,
                   "fused_deep_moe: int8 shared expert needs share_gmm1/2_weight_scale")
            _check(share_gmm1_weight_scale.numel() == nsh and share_gmm2_weight_scale.numel() == h,
                   f"fused_deep_moe: int8 shared scales must be [{nsh}] and [{h}]")
            ss1 = _contig(share_gmm1_weight_scale, "share_gmm1_weight_scale", torch.float32).view(nsh)
            ss2 = _contig(share_gmm2_weight_scale, "share_gmm2_weight_scale", torch.float32).view(h)
    ids = expert_ids if expert_ids.dtype == torch.int32 else expert_ids.to(torch.int32)
    ids = ids.contiguous()
    es = expert_scales if expert_scales.dtype == torch.float32 else expert_scales.to(torch.float32)
    es = es.contiguous()
    mask = None
    if x_active_mask is not None:
        mask = x_active_mask.to(torch.bool).contiguous().view(torch.uint8)
    out = torch.empty_like(x)
    share_out = torch.empty_like(x)
    etn = torch.empty(L, dtype=torch.int64, device=x.device)
    _lib.call("camhipFusedDeepMoe", _lib.ptr(x), _lib.ptr(ids), _lib.ptr(w1), _lib.ptr(s1), _lib.ptr(w2),
              _lib.ptr(s2), _lib.ptr(es), _lib.ptr(sw1), _lib.ptr(ss1), _lib.ptr(sw2), _lib.ptr(ss2),
              _lib.ptr(smooth), _lib.ptr(share_smooth), _lib.ptr(mask), bs, h, k, n1, nsh,
              (3 if fp8 else 2 if int8 else 0) | (WEIGHT_LIST if separated else 0), ep_rank_size, ep_rank_id, moe_expert_num, quant_mode, global_bs, _lib.ptr(out),
              _lib.ptr(share_out), _lib.ptr(etn), device=x.device)
    return [out, share_out, etn]


def fused_deep_moe_meta(x, expert_ids, gmm1_weight, gmm1_weight_scale, gmm2_weight, gmm2_weight_scale,
                        expert_scales, share_gmm1_weight, share_gmm1_weight_scale, share_gmm2_weight,
                        share_gmm2_weight_scale, expert_smooth_scales, share_smooth_scales, x_active_mask, group_ep,
                        ep_rank_size, ep_rank_id, moe_expert_num, quant_mode, global_bs):
    """Shape function (pybind/fused_deep_moe.cpp:91-124)."""
    L = moe_expert_num // ep_rank_size
    return [torch.empty_like(x), torch.empty_like(x), torch.empty(L, dtype=torch.int64, device=x.device)]


_impl.impl("fused_deep_moe", fused_deep_moe)
_meta.impl("fused_deep_moe", fused_deep_moe_meta)
_impl.impl("grouped_matmul_swiglu", grouped_matmul_swiglu)
_impl.impl("grouped_matmul", grouped_matmul)
_impl.impl("get_dispatch_layout", get_dispatch_layout)
_impl.impl("moe_dispatch_prefill", moe_dispatch_prefill)
_impl.impl("moe_combine_prefill", moe_combine_prefill)
_impl.impl("moe_route", moe_route)
