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
from .ops import QUANT_FP8_BLOCK, QUANT_INT8_TOKEN, QUANT_NONE


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
        ws_combine = _lib.workspace_size("camhipMoeCombineNormal", 1, 1, N, None, 1, T, K, H, 1, 0, E, 1)
        self.ws_layout = torch.empty(max(ws_layout, 1), dtype=torch.uint8, device=dev)
        self.ws_combine = torch.empty(max(ws_combine, 1), dtype=torch.uint8, device=dev)

    # -- stages ---------------------------------------------------------
    def route(self, logits, bias=None, stream=None):
        _lib.launch("camhipMoeRoute", logits.data_ptr(), None if bias is None else bias.data_ptr(), self.T, self.E,
                    self.K, self.topk_idx.data_ptr(), self.topk_w.data_ptr(), stream=stream, device=self.device)

    def layout(self, stream=None):
        self.topk_idx64.copy_(self.topk_idx)
        _lib.launch("camhipDispatchLayout", self.topk_idx64.data_ptr(), self.T, 1, self.E, self.K, None,
                    self.num_tokens_per_expert.data_ptr(), None, self.send_token_idx.data_ptr(),
                    workspace=self.ws_layout, stream=stream, device=self.device)
        _lib.launch("camhipNotifyDispatch", self.num_tokens_per_expert.data_ptr(), self.E, self.T, 1, 0,
                    self.send_offset.data_ptr(), self.total_recv.data_ptr(), self.recv_count.data_ptr(),
                    self.recv_offset.data_ptr(), self.max_bs.data_ptr(), self.recv_tokens_per_expert.data_ptr(),
                    stream=stream, device=self.device)

    def dispatch(self, x, stream=None):
        _lib.launch("camhipMoeDispatchNormal", x.data_ptr(), self.topk_idx.data_ptr(), self.send_offset.data_ptr(),
                    self.send_token_idx.data_ptr(), self.recv_offset.data_ptr(), self.recv_count.data_ptr(), self.T,
                    self.H, self.K, 1, 0, self.E, self.q, self.N, self.expand_x.data_ptr(), self.scales.data_ptr(),
                    self.expand_idx.data_ptr(), stream=stream, device=self.device)

    def combine(self, y, stream=None):
        """y: [N, H] bf16 expert outputs in dispatch order."""
        _lib.launch("camhipMoeCombineNormal", y.data_ptr(), self.expand_idx.data_ptr(), self.N,
                    self.recv_count.data_ptr(), self.topk_w.data_ptr(), self.T, self.K, self.H, 1, 0, self.E,
                    self.out.data_ptr(), workspace=self.ws_combine, stream=stream, device=self.device)
        return self.out
