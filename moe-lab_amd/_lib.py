"""ctypes binding of libmoe_mi355x.so (the C ABI declared in include/moe_mi355x.h).

The library is built in-tree by ``__graft_entry__.build()`` (moe-lab_amd/csrc/Makefile). There is no
fallback: if the library is missing or cannot be loaded, every GPU entry point raises.
torch is imported first so the library binds to the HIP runtime torch already loaded (both carry the
soname libamdhip64.so.7), sharing its device context and streams.
"""
import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime before the library)

HERE = os.path.dirname(os.path.abspath(__file__))
# MOELAB_AMD_LIB names another build of the same library (e.g. one compiled with different tuning macros)
LIB_PATH = os.environ.get("MOELAB_AMD_LIB") or os.path.join(HERE, "libmoe_mi355x.so")

MOE_OK, MOE_ERR_ARG, MOE_ERR_DTYPE, MOE_ERR_WORKSPACE, MOE_ERR_LAUNCH, MOE_ERR_ALIGN = 0, -1, -2, -3, -4, -5
DTYPE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
FMT_INT4_G64, FMT_MXFP4 = 0, 1
PATH_AUTO, PATH_SLOTS, PATH_GROUPED = 0, 1, 2
ACT_SWIGLU, ACT_GEGLU, ACT_GPTOSS = 0, 1, 2

EXPORTS = ("moe_router", "moe_router_counter_count", "moe_topk", "moe_group", "moe_experts_run",
           "moe_experts_run_stages", "moe_experts_workspace_bytes", "moe_row_bytes", "moe_tile_bytes",
           "moe_tiles_pack", "moe_shared_experts_run", "moe_shared_experts_workspace_bytes", "moe_version",
           "moe_experts_run_static", "moe_layer_run", "moe_layer_workspace_bytes", "moe_experts_run_shared",
           "moe_experts_shared_workspace_bytes", "moe_router_group", "moe_layer_run_shared",
           "moe_layer_shared_workspace_bytes", "moe_probe_read")
PROBE_SINK = 1024   # MOE_PROBE_SINK
STATIC_SCRATCH_BYTES = 32 << 20   # MOE_STATIC_SCRATCH_BYTES: the workspace array of moe_experts_run_static
STAGE_GATE_UP, STAGE_DOWN, STAGE_ALL = 1, 2, 3

_ERRORS = {
    MOE_ERR_ARG: "invalid argument (shape, size or pointer)",
    MOE_ERR_DTYPE: "unsupported dtype or weight format",
    MOE_ERR_WORKSPACE: "workspace missing or too small",
    MOE_ERR_LAUNCH: "HIP launch failed",
    MOE_ERR_ALIGN: "pointer not 16-byte aligned",
}


class MoeError(RuntimeError):
    def __init__(self, fn, rc):
        super().__init__(f"{fn}: {_ERRORS.get(rc, 'error')} (rc={rc})")
        self.rc = rc


class Proj(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("tiles", ctypes.c_void_p)]


class Experts(ctypes.Structure):
    _fields_ = [("fmt", ctypes.c_int32), ("E", ctypes.c_int32), ("d", ctypes.c_int32), ("F", ctypes.c_int32),
                ("gate", Proj), ("up", Proj), ("down", Proj)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        vp, i, f, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
        L.moe_router.argtypes = [vp, vp, vp, i, i, i, i, i, f, vp, vp, vp, vp, vp]
        L.moe_router_counter_count.argtypes = [i]
        L.moe_topk.argtypes = [vp, i, i, i, i, i, f, vp, vp, vp]
        L.moe_group.argtypes = [vp, i, i, vp, vp, vp, vp, vp, vp]
        L.moe_experts_run.argtypes = [ctypes.POINTER(Experts), vp, i, vp, vp, i, i, i, i, i, vp, i, vp, vp, sz, vp]
        L.moe_experts_run_stages.argtypes = [ctypes.POINTER(Experts), vp, i, vp, vp, i, i, i, i, i, vp, i, vp, vp,
                                             sz, i, vp]
        L.moe_experts_run_static.argtypes = [ctypes.POINTER(Experts), vp, i, vp, vp, i, i, i, i, i, vp, i, vp, vp]
        L.moe_experts_workspace_bytes.argtypes = [ctypes.POINTER(Experts), i, i, i]
        L.moe_experts_workspace_bytes.restype = sz
        L.moe_router_group.argtypes = [vp, vp, vp, i, i, i, i, i, f, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        L.moe_layer_run.argtypes = [ctypes.POINTER(Experts), vp, i, vp, vp, i, i, i, f, i, vp, vp, vp, i, vp, vp, sz,
                                    vp]
        L.moe_layer_run_shared.argtypes = [ctypes.POINTER(Experts), i, vp, i, vp, vp, vp, i, i, i, f, i, vp, vp, vp, i,
                                           vp, vp, sz, vp]
        L.moe_layer_shared_workspace_bytes.argtypes = [ctypes.POINTER(Experts), i, i, i]
        L.moe_layer_shared_workspace_bytes.restype = sz
        L.moe_layer_workspace_bytes.argtypes = [ctypes.POINTER(Experts), i, i]
        L.moe_layer_workspace_bytes.restype = sz
        L.moe_version.restype = ctypes.c_char_p
        L.moe_probe_read.argtypes = [vp, sz, vp, vp]
        L.moe_row_bytes.argtypes = [i, i]
        L.moe_row_bytes.restype = sz
        L.moe_tile_bytes.argtypes = [i, i, i]
        L.moe_tile_bytes.restype = sz
        L.moe_tiles_pack.argtypes = [i, i, i, i, vp, vp, vp]
        L.moe_shared_experts_run.argtypes = [ctypes.POINTER(Experts), vp, i, i, i, vp, vp, i, vp, vp, sz, vp]
        L.moe_shared_experts_workspace_bytes.argtypes = [ctypes.POINTER(Experts), i]
        L.moe_shared_experts_workspace_bytes.restype = sz
        L.moe_experts_run_shared.argtypes = [ctypes.POINTER(Experts), i, vp, i, vp, vp, i, i, i, i, vp, vp, i, vp,
                                             vp, sz, vp]
        L.moe_experts_shared_workspace_bytes.argtypes = [ctypes.POINTER(Experts), i, i, i, i]
        L.moe_experts_shared_workspace_bytes.restype = sz
        for n in ("moe_router", "moe_router_counter_count", "moe_topk", "moe_group", "moe_experts_run",
                  "moe_experts_run_stages", "moe_tiles_pack", "moe_shared_experts_run", "moe_experts_run_static",
                  "moe_layer_run", "moe_experts_run_shared", "moe_router_group", "moe_layer_run_shared",
                  "moe_probe_read"):
            getattr(L, n).restype = ctypes.c_int
        _lib = L
    return _lib


def check(fn, rc):
    if rc != MOE_OK:
        raise MoeError(fn, rc)


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_device(t, name="tensor"):
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (the HIP path has no CPU fallback)")


_WS = {}        # device index -> the current scratch buffer of that device
_RETIRED = []   # buffers replaced by larger ones: never freed (a captured HIP graph keeps their raw pointers)


def grow(table, key, nbytes, make, what):
    """The buffer table[key] with at least nbytes, replaced by a new one (at least twice the old size, so at
    most log2 of the largest size is ever retired) when it is smaller. A replaced buffer is kept alive for the
    process: a HIP graph captured with it still writes there. Growing during stream capture raises instead:
    the new buffer would come from the graph's private pool."""
    buf = table.get(key)
    if buf is not None and buf.numel() >= nbytes:
        return buf
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"{what} would grow from {0 if buf is None else buf.numel()} to {nbytes} during "
                           f"HIP graph capture: call reserve() with the largest call's sizes before capturing")
    if buf is not None:
        _RETIRED.append(buf)
    buf = make(max(int(nbytes), 2 * (0 if buf is None else buf.numel())))
    table[key] = buf
    return buf


def workspace(device, nbytes):
    """Per-device scratch buffer of the expert calls (uint8, at least nbytes; the calls need no particular
    contents). Grows on demand (see grow)."""
    device = torch.device(device)
    return grow(_WS, device.index, max(int(nbytes), 256),
                lambda n: torch.empty(n, dtype=torch.uint8, device=device), "the expert workspace")
