"""umdk_amd -- MI355X (gfx950) implementation of UMDK CAM's MoE hot path.

Importing the package registers torch.ops.umdk_cam_op_lib.* (the reference's
operator library name) and exposes the same module-level functions as the
reference's pybind module (src/cam/comm_operator/pybind/pybind.cpp:13-19).
"""
from . import ops  # noqa: F401  (registers torch.ops.umdk_cam_op_lib)
from .ops import (fused_deep_moe, get_dispatch_layout, grouped_matmul, grouped_matmul_swiglu, moe_combine_prefill,  # noqa: F401
                  moe_dispatch_prefill, moe_route, prepack_weight)

__all__ = ["fused_deep_moe", "get_dispatch_layout", "moe_dispatch_prefill", "moe_combine_prefill", "moe_route", "grouped_matmul_swiglu",
           "grouped_matmul", "prepack_weight"]
