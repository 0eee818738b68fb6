"""The reference's extension module name, for call sites written against it.

CAM's callers import `umdk_cam_op_lib` (the pybind module, src/cam/comm_operator/pybind/pybind.cpp:13-19) and then
call `torch.ops.umdk_cam_op_lib.*`.  Importing this module registers those operators from the MI355X build
(umdk_amd) and exposes the same module-level functions, so such call sites run without edits.
"""
from umdk_amd import fused_deep_moe, get_dispatch_layout, moe_combine_prefill, moe_dispatch_prefill  # noqa: F401

__all__ = ["fused_deep_moe", "get_dispatch_layout", "moe_dispatch_prefill", "moe_combine_prefill"]
