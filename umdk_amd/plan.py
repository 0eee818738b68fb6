"""Capacity-sized, host-sync-free runner of the prefill path
(route -> layout -> count exchange -> dispatch -> [experts] -> combine).

The torch ops mirror the reference bindings, including the host read of the
received row count (moe_dispatch_prefill.cpp:110-111) that sizes their
outputs.  This plan instead sizes every buffer for the worst case (T*K rows on
one rank) once, so a step never synchronises with the host, allocates nothing
and can be captured in a HIP graph.  Rows past recv_count[-1] are unused.
"""
import torch

from . import _lib
from .ops import QUANT_FP8_BLOCK, QUANT_FP8_BLOCK_KMAJOR, QUANT_INT8_TOKEN, QUANT_NONE


class MoePrefillPlan:
    def __init__(self, T, H, E, K, quant_mode=QUANT_FP8_BLOCK, device="cuda"):
        self.T, self.H, self.E, self.K, self.q = T, H, E, K, quant_mode
        self.device = torch.device(device)
        dev = self.device
        i32 = dict(dtype=torch.int32, device=dev)
        N = T * K
        self.N = N
        self.topk_idx = torch.empty((T, K), **i32)
        self.topk_idx64 = torch.empty((T, K), dtype=torch.int64, device=dev)
        self.topk_w = torch.empty((T, K), dtype=torch.float32, device=dev)
        self.num_tokens_per_expert = torch.empty(E, **i32)
        self.send_token_idx = torch.empty((T, K), **i32)
        self.send_offset = torch.empty(E, **i32)
        self.total_recv = torch.empty(1, **i32)
        self.recv_count = torch.empty(E, **i32)
        self.recv_offset = torch.empty(E, **i32)
        self.max_bs = torch.empty(1, **i32)
        self.recv_tokens_per_expert = torch.empty(E, dtype=torch.int64, device=dev)
        xdt = {QUANT_NONE: torch.bfloat16, QUANT_INT8_TOKEN: torch.int8, QUANT_FP8_BLOCK: torch.float8_e4m3fn}[quant_mode]
        self.expand_x = torch.empty((N, H), dtype=xdt, device=dev)
        self.scales = torch.empty((N, H // 128) if quant_mode == QUANT_FP8_BLOCK else (N,), dtype=torch.float32,
                                  device=dev)
        self.expand_idx = torch.empty(N * 3, **i32)
        self.out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
        ws_layout = _lib.workspace_size("camhipDispatchLayout", 1, T, 1, E, K, None, 1, None, 1)
        # sized with the diagnose output requested (the larger workspace), so either call fits
        ws_combine = _lib.workspace_size("camhipMoeCombineNormal", 1, 1, N, None, 1, T, K, H, 1, 0, E, 1, 1)
        ws_dispatch = _lib.workspace_size("camhipMoeDispatchNormal", 1, 1, 1, 1, None, None, T, H, K, 1, 0, E,
                                          quant_mode, N, 1, 1, 1, 1)
        self.ws_layout = torch.empty(max(ws_layout, 1), dtype=torch.uint8, device=dev)
        # the four-launch step (camhipMoePrefillDispatch / camhipMoePrefillCombine): the combine's row map
        # comes from the dispatch
        self.combine_row_map = torch.empty((T, K), **i32)
        self.E_route = E
        ws_step = _lib.workspace_size("camhipMoePrefillDispatch", 1, None, 1, T, H, E, E, K, quant_mode, N,
                                      1, 1, 1, 1, 1, 1, 1, 1)
        self.ws_step = torch.empty(max(ws_step, 1), dtype=torch.uint8, device=dev)
        self.ws_combine = torch.empty(max(ws_combine, 1), dtype=torch.uint8, device=dev)
        self.ws_dispatch = torch.empty(max(ws_dispatch, 1), dtype=torch.uint8, device=dev)

    # -- stages ---------------------------------------------------------
    def route(self, logits, bias=None, stream=None):
        # the int64 copy of the ids feeds the layout op (int64 topk_idx, as aclnnDispatchLayout)
        _lib.launch("camhipMoeRoute", logits.data_ptr(), None if bias is None else bias.data_ptr(), self.T, self.E,
                    self.K, self.topk_idx.data_ptr(), self.topk_w.data_ptr(), self.topk_idx64.data_ptr(),
                    stream=stream, device=self.device)

    def layout(self, stream=None):
        _lib.launch("camhipDispatchLayout", self.topk_idx64.data_ptr(), self.T, 1, self.E, self.K, None,
                    self.num_tokens_per_expert.data_ptr(), None, self.send_token_idx.data_ptr(),
                    workspace=self.ws_layout, stream=stream, device=self.device)
        _lib.launch("camhipNotifyDispatch", self.num_tokens_per_expert.data_ptr(), self.E, self.T, 1, 0,
                    self.send_offset.data_ptr(), self.total_recv.data_ptr(), self.recv_count.data_ptr(),
                    self.recv_offset.data_ptr(), self.max_bs.data_ptr(), self.recv_tokens_per_expert.data_ptr(),
                    stream=stream, device=self.device)

    def dispatch(self, x, stream=None, cost_stats=None):
        """cost_stats: optional [1] int32 device tensor; gains the dispatch phase's microseconds
        (the reference's waitRecvCostStats diagnose output)."""
        _lib.launch("camhipMoeDispatchNormal", x.data_ptr(), self.topk_idx.data_ptr(), self.send_offset.data_ptr(),
                    self.send_token_idx.data_ptr(), self.recv_offset.data_ptr(), self.recv_count.data_ptr(), self.T,
                    self.H, self.K, 1, 0, self.E, self.q, self.N, self.expand_x.data_ptr(), self.scales.data_ptr(),
                    self.expand_idx.data_ptr(), None if cost_stats is None else cost_stats.data_ptr(),
                    workspace=self.ws_dispatch, stream=stream, device=self.device)

    def combine(self, y, stream=None, cost_stats=None):
        """y: [N, H] bf16 expert outputs in dispatch order.  cost_stats: optional [1] int32 device
        tensor; gains the combine phase's microseconds (the reference's sendCostStats)."""
        _lib.launch("camhipMoeCombineNormal", y.data_ptr(), self.expand_idx.data_ptr(), self.N,
                    self.recv_count.data_ptr(), self.topk_w.data_ptr(), self.T, self.K, self.H, 1, 0, self.E,
                    self.out.data_ptr(), None if cost_stats is None else cost_stats.data_ptr(),
                    workspace=self.ws_combine, stream=stream, device=self.device)
        return self.out


    # -- the step in four launches ------------------------------------------------
    def dispatch_step(self, logits, x, bias=None, stream=None):
        """route (over E_route experts) + layout + count exchange + dispatch (over the local experts) in three
        launches; the same results as route(), layout() and dispatch() (send_token_idx and num_tokens_per_expert
        are not produced), plus the combine's row map."""
        _lib.launch("camhipMoePrefillDispatch", logits.data_ptr(), None if bias is None else bias.data_ptr(),
                    x.data_ptr(), self.T, self.H, self.E_route, self.E, self.K, self.q, self.N,
                    self.topk_idx.data_ptr(), self.topk_w.data_ptr(), self.expand_x.data_ptr(),
                    None if self.q == QUANT_NONE else self.scales.data_ptr(), self.expand_idx.data_ptr(),
                    self.recv_count.data_ptr(), self.recv_tokens_per_expert.data_ptr(),
                    self.combine_row_map.data_ptr(), workspace=self.ws_step, stream=stream, device=self.device)

    def combine_step(self, y, stream=None):
        """combine() after dispatch_step(): one gather launch on the dispatch's row map."""
        _lib.launch("camhipMoePrefillCombine", y.data_ptr(), self.expand_idx.data_ptr(),
                    self.combine_row_map.data_ptr(), self.recv_count.data_ptr(), self.topk_w.data_ptr(), self.T,
                    self.K, self.H, self.E, self.N, self.out.data_ptr(), stream=stream, device=self.device)
        return self.out


class MoeLayerPlan(MoePrefillPlan):
    """Full expert layer on one EP rank: route over `E` experts, keep the
    (t,k) pairs whose expert is one of this rank's `L` local experts (ids
    0..L-1; the others would be sent to other ranks and are not routed here),
    dispatch them, run GMM1+SwiGLU and GMM2 per local expert, and combine.

    dtype "bf16": bf16 rows and weights, bf16 h.  dtype "fp8": fp8 e4m3fn rows
    with 1x128 scales, fp8 weights with 128x128 scales, fp8 h with 1x128
    scales.  dtype "int8": the reference's int8 prefill numerics -- int8 rows
    with per-token scales (the use_quant recipe, moe_dispatch_normal.h:295-332),
    int8 weights with per-output-channel scales [L, 2I] / [L, H], int8 h
    requantised per token.  The output is bf16 in every mode.  Weights are
    [L, 2I, H] and [L, H, I] with the reduction dimension contiguous.
    """

    def __init__(self, T, H, E, K, L, I, dtype="fp8", device="cuda"):
        _check = {"bf16": QUANT_NONE, "fp8": QUANT_FP8_BLOCK, "int8": QUANT_INT8_TOKEN}
        if dtype not in _check:
            raise ValueError(f"MoeLayerPlan: dtype must be bf16, fp8 or int8 (got {dtype})")
        q = _check[dtype]
        super().__init__(T, H, L, K, quant_mode=q, device=device)
        self.E_route = E
        self.L, self.I, self.dtype = L, I, dtype
        dev = self.device
        N = self.N
        if dtype == "fp8":
            # the dispatch writes the block scales k-major ([H/128, N] storage), the layout GMM1 reads directly
            self.q = QUANT_FP8_BLOCK_KMAJOR
            self.scales = torch.empty((H // 128, N), dtype=torch.float32, device=dev).t()
            self.h = torch.empty((N, I), dtype=torch.float8_e4m3fn, device=dev)
            # k-major h scales ([I/128, N] storage): GMM1 writes and GMM2 reads this layout
            self.h_scale = torch.empty((I // 128, N), dtype=torch.float32, device=dev).t()
        elif dtype == "int8":
            self.h = torch.empty((N, I), dtype=torch.int8, device=dev)
            self.h_scale = torch.empty(N, dtype=torch.float32, device=dev)
        else:
            self.h = torch.empty((N, I), dtype=torch.bfloat16, device=dev)
            self.h_scale = None
        self.y = torch.empty((N, H), dtype=torch.bfloat16, device=dev)
        # int8 GMM1 keeps its fp32 h and partial row maxima in a workspace until the per-token requantisation
        ws1 = _lib.workspace_size("camhipGroupedMatmulSwiglu", 1, 1, 1, L, N, H, 2 * I, 1, 1, self._dt(), 0,
                                  self._out_quant(), 1, 1)
        self.ws_gmm1 = torch.empty(max(ws1, 1), dtype=torch.uint8, device=dev) if ws1 else None
        # both GEMMs in one call (camhipMoeExperts: one chained launch where the kernel exists); int8 keeps
        # the two calls (its h is requantised per token in a launch of its own)
        self.ws_experts = None
        if dtype != "int8":
            wsx = _lib.workspace_size("camhipMoeExperts", 1, 1, 1, L, N, H, 2 * I, 1, 1, 1, 1, self._dt(), 1, 1, 1,
                                      1)
            self.ws_experts = torch.empty(max(wsx, 1), dtype=torch.uint8, device=dev)
        self.topk_idx = torch.empty((T, K), dtype=torch.int32, device=dev)

    def route(self, logits, bias=None, stream=None):
        _lib.launch("camhipMoeRoute", logits.data_ptr(), None if bias is None else bias.data_ptr(), self.T,
                    self.E_route, self.K, self.topk_idx.data_ptr(), self.topk_w.data_ptr(),
                    self.topk_idx64.data_ptr(), stream=stream, device=self.device)

    def experts(self, w1, w1_scale, w2, w2_scale, stream=None):
        """GMM1 + SwiGLU and GMM2 over the dispatched rows -> self.y (bit-identical to gmm1() then gmm2())."""
        if self.ws_experts is None:
            self.gmm1(w1, w1_scale, stream)
            return self.gmm2(w2, w2_scale, stream)
        dt = self._dt()
        p = lambda t: None if t is None else t.data_ptr()
        _lib.launch("camhipMoeExperts", self.expand_x.data_ptr(), self.scales.data_ptr() if dt else None,
                    self.recv_tokens_per_expert.data_ptr(), self.L, self.N, self.H, 2 * self.I, w1.data_ptr(),
                    p(w1_scale), w2.data_ptr(), p(w2_scale), dt, 1, self.h.data_ptr(), p(self.h_scale),
                    self.y.data_ptr(), workspace=self.ws_experts, stream=stream, device=self.device)
        return self.y

    def _dt(self):
        return {"bf16": 0, "int8": 2, "fp8": 3}[self.dtype]

    def _out_quant(self):
        return {"bf16": QUANT_NONE, "int8": QUANT_INT8_TOKEN, "fp8": QUANT_FP8_BLOCK}[self.dtype]

    def gmm1(self, w1, w1_scale, stream=None):
        dt = self._dt()
        xs = self.scales.data_ptr() if dt else None
        _lib.launch("camhipGroupedMatmulSwiglu", self.expand_x.data_ptr(), xs,
                    self.recv_tokens_per_expert.data_ptr(), self.L, self.N, self.H, 2 * self.I, w1.data_ptr(),
                    None if w1_scale is None else w1_scale.data_ptr(), dt, 1 if dt == 3 else 0, self._out_quant(),
                    self.h.data_ptr(), None if self.h_scale is None else self.h_scale.data_ptr(),
                    workspace=self.ws_gmm1, stream=stream, device=self.device)
        return self.h

    def gmm2(self, w2, w2_scale, stream=None):
        dt = self._dt()
        _lib.launch("camhipGroupedMatmul", self.h.data_ptr(),
                    None if self.h_scale is None else self.h_scale.data_ptr(),
                    self.recv_tokens_per_expert.data_ptr(), self.L, self.N, self.I, self.H, w2.data_ptr(),
                    None if w2_scale is None else w2_scale.data_ptr(), dt, 1 if dt == 3 else 0, self.y.data_ptr(),
                    stream=stream, device=self.device)
        return self.y

    def forward(self, x, logits, bias, w1, w1_scale, w2, w2_scale, stream=None):
        """The whole layer: dispatch_step, GMM1 + SwiGLU, GMM2, combine_step (six launches for fp8/bf16)."""
        self.dispatch_step(logits, x, bias, stream)
        self.experts(w1, w1_scale, w2, w2_scale, stream)
        return self.combine_step(self.y, stream)

    def forward_op_chain(self, x, logits, bias, w1, w1_scale, w2, w2_scale, stream=None):
        """The same layer through the reference-shaped calls (route, layout, count exchange, dispatch, ..., combine)."""
        self.route(logits, bias, stream)
        self.layout(stream)
        self.dispatch(x, stream)
        self.experts(w1, w1_scale, w2, w2_scale, stream)
        return self.combine(self.y, stream)
