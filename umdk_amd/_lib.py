"""Loader for libcamhip.so and a thin two-phase caller over its C ABI.

The library must already be built (``python -m umdk_amd.build`` or
``__graft_entry__.build()``); there is no fallback path: a missing library or
a non-GPU tensor raises.
"""
import ctypes
import os

import torch  # loads the HIP runtime first, so libcamhip binds to the same one

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libcamhip.so")

_P = ctypes.c_void_p
_I = ctypes.c_int64
_U64P = ctypes.POINTER(ctypes.c_uint64)
_EXP = ctypes.POINTER(ctypes.c_void_p)

# argument kinds of each *GetWorkspaceSize entry point ('p' pointer, 'i' int64)
SIGNATURES = {
    "camhipMoeRoute": "pp iii ppp",
    "camhipDispatchLayout": "p iiii pppp",
    "camhipNotifyDispatch": "p iiii pppppp",
    "camhipMoeDispatchNormal": "pppppp iiiiiiii pppp",
    "camhipMoeCombineNormal": "pp i pp iiiiii pp",
    "camhipGroupedMatmulSwiglu": "ppp iiii pp iii pp",
    "camhipGroupedMatmul": "ppp iiii pp ii p",
    "camhipFusedDeepMoe": "pppppp p pppp ppp iiiiii iiiii ppp",
    "camhipMoePrefillDispatch": "ppp iiiiiii pppppppp",
    "camhipMoePrefillCombine": "ppppp iiiii p",
    "camhipMoeExperts": "ppp iiii pppp ii ppp",
}

_lib = None


class CamHipError(RuntimeError):
    pass


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m umdk_amd.build` (there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        L.camhipGetLastErrorMsg.restype = ctypes.c_char_p
        L.camhipGetVersion.restype = ctypes.c_char_p
        L.camhipReleaseExecutor.restype = None
        L.camhipReleaseExecutor.argtypes = [_P]
        for name, sig in SIGNATURES.items():
            kinds = sig.replace(" ", "")
            f = getattr(L, name + "GetWorkspaceSize")
            f.restype = ctypes.c_int
            f.argtypes = [(_P if k == "p" else _I) for k in kinds] + [_U64P, _EXP]
            g = getattr(L, name)
            g.restype = ctypes.c_int
            g.argtypes = [_P, ctypes.c_uint64, _P, _P]
        # the allocation-free combine: the combine's GetWorkspaceSize arguments without the workspace
        # outputs, then the stream
        L.camhipMoeCombineNormalNoAlloc.restype = ctypes.c_int
        L.camhipMoeCombineNormalNoAlloc.argtypes = [_P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P]
        L.camhipGetSyncStatus.restype = ctypes.c_int
        L.camhipGetSyncStatus.argtypes = [ctypes.POINTER(ctypes.c_int32), ctypes.c_int32]
        L.camhipDebugSetSyncWait.restype = None
        L.camhipDebugSetSyncWait.argtypes = [_I, ctypes.c_int32]
        _lib = L
    return _lib


def exported_symbols():
    return [n + s for n in SIGNATURES for s in ("GetWorkspaceSize", "")] + [
        "camhipGetLastErrorMsg", "camhipGetVersion"]


def ptr(t, transposed_ok=False):
    """Device pointer of a tensor (None -> NULL).  transposed_ok also accepts
    the transpose of a contiguous 2-D tensor (k-major scale storage)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise CamHipError("umdk_cam_op_lib ops run on the GPU only; got a tensor on " + str(t.device))
    if not (t.is_contiguous() or (transposed_ok and t.dim() == 2 and t.t().is_contiguous())):
        raise CamHipError("umdk_cam_op_lib ops need contiguous tensors")
    return t.data_ptr()


def call(name, *args, device=None, stream=None):
    """Runs one two-phase entry point: size the workspace, allocate it from
    torch's caching allocator on `device`, launch on the current stream."""
    L = lib()
    ws = ctypes.c_uint64(0)
    ex = ctypes.c_void_p(0)
    st = getattr(L, name + "GetWorkspaceSize")(*args, ctypes.byref(ws), ctypes.byref(ex))
    if st != 0:
        raise CamHipError(f"{name}GetWorkspaceSize failed ({st}): {L.camhipGetLastErrorMsg().decode()}")
    buf = None
    if ws.value > 0:
        buf = torch.empty(ws.value, dtype=torch.uint8, device=device)
    if stream is None:
        stream = torch.cuda.current_stream(device).cuda_stream
    st = getattr(L, name)(buf.data_ptr() if buf is not None else None, ws.value, ex, stream)
    if st != 0:
        raise CamHipError(f"{name} failed ({st}): {L.camhipGetLastErrorMsg().decode()}")
    return buf


def launch(name, *args, workspace=None, stream=None, device=None):
    """Like call(), but with a caller-owned workspace tensor (no allocation:
    safe inside a captured graph once the workspace is large enough)."""
    L = lib()
    ws = ctypes.c_uint64(0)
    ex = ctypes.c_void_p(0)
    st = getattr(L, name + "GetWorkspaceSize")(*args, ctypes.byref(ws), ctypes.byref(ex))
    if st != 0:
        raise CamHipError(f"{name}GetWorkspaceSize failed ({st}): {L.camhipGetLastErrorMsg().decode()}")
    have = workspace.numel() * workspace.element_size() if workspace is not None else 0
    if stream is None:
        stream = torch.cuda.current_stream(device).cuda_stream
    st = getattr(L, name)(workspace.data_ptr() if workspace is not None else None, have, ex, stream)
    if st != 0:
        raise CamHipError(f"{name} failed ({st}): {L.camhipGetLastErrorMsg().decode()}")


def sync_status(clear=False):
    """The current device's sync status of the chained GEMM launches (0: no readiness wait gave up);
    synchronous, call after the launches have completed."""
    L = lib()
    v = ctypes.c_int32(0)
    st = L.camhipGetSyncStatus(ctypes.byref(v), 1 if clear else 0)
    if st != 0:
        raise CamHipError(f"camhipGetSyncStatus failed ({st}): {L.camhipGetLastErrorMsg().decode()}")
    return v.value


def workspace_size(name, *args):
    """First phase only; the executor is released by a zero-size second call."""
    L = lib()
    ws = ctypes.c_uint64(0)
    ex = ctypes.c_void_p(0)
    st = getattr(L, name + "GetWorkspaceSize")(*args, ctypes.byref(ws), ctypes.byref(ex))
    if st != 0:
        raise CamHipError(f"{name}GetWorkspaceSize failed ({st}): {L.camhipGetLastErrorMsg().decode()}")
    L.camhipReleaseExecutor(ex)
    return ws.value
