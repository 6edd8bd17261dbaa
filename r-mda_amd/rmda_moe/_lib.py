"""ctypes binding of librmda_moe.so (built from r-mda_amd/csrc by its Makefile).

Loading fails loudly when the library is missing: there is no CPU fallback
anywhere in this package.
"""
import ctypes
import os
import re

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT_DIR = os.path.dirname(PKG_DIR)              # r-mda_amd/
REPO_DIR = os.path.dirname(ROOT_DIR)
CSRC_DIR = os.path.join(ROOT_DIR, "csrc")
LIB_PATH = os.path.join(CSRC_DIR, "librmda_moe.so")
# A partial build of the library in its place (the sanitized safetensors
# reader of tests/asan): only the entry points it exports get bound.
PARTIAL_LIB = os.environ.get("RMDA_MOE_PARTIAL_LIB")
HEADER_PATH = os.path.join(REPO_DIR, "include", "rmda_moe.h")

_u32 = ctypes.c_uint32
_p = ctypes.c_void_p

OK = 0
ERRORS = {
    -1: "RMDA_ERR_ARG", -2: "RMDA_ERR_SHAPE", -3: "RMDA_ERR_CAPACITY", -4: "RMDA_ERR_HIP",
    -5: "RMDA_ERR_STICKY", -6: "RMDA_ERR_WORKSPACE", -7: "RMDA_ERR_DEVICE",
}
NONE = 0xFFFFFFFF
NO_SLOT = 0xFFFFFFFF
MAX_EXPERTS = 512
MAX_TOPK = 16
MM_TILE = 128
CTX_MAX_PAIRS = 1 << 21
PROF_STAGES = 7
PROF_RING = 64


class RoutePC(ctypes.Structure):
    _fields_ = [("rows", _u32), ("experts", _u32), ("topk", _u32), ("stride", _u32)]


class ScanPC(ctypes.Structure):
    _fields_ = [("experts", _u32), ("tile", _u32)]


class ScatterPC(ctypes.Structure):
    _fields_ = [("rows", _u32), ("topk", _u32), ("d8", _u32)]


class MmPC(ctypes.Structure):
    _fields_ = [("m", _u32), ("n", _u32), ("k", _u32), ("sa", _u32), ("sb", _u32)]


class CombinePC(ctypes.Structure):
    _fields_ = [("rows", _u32), ("d", _u32), ("topk", _u32), ("pstride", _u32), ("sg_off", _u32),
                ("inj_stride", _u32), ("inj_off", _u32), ("hc", _u32)]


class ElemPC(ctypes.Structure):
    _fields_ = [("rows", _u32), ("n", _u32), ("astride", _u32), ("ao", _u32), ("bo", _u32),
                ("op", _u32), ("scale", ctypes.c_float)]


class SlotPC(ctypes.Structure):
    _fields_ = [("n", _u32), ("slot", _u32)]


class Bf16PC(ctypes.Structure):
    _fields_ = [("n", _u32)]


class RouterPC(ctypes.Structure):
    _fields_ = [("rows", _u32), ("d", _u32), ("cols", _u32), ("stride", _u32), ("nbias", _u32)]


class Shape(ctypes.Structure):
    _fields_ = [("rows", _u32), ("d", _u32), ("experts", _u32), ("topk", _u32), ("inter", _u32),
                ("shared", _u32)]


class LayerArgs(ctypes.Structure):
    _fields_ = [("x", _p), ("w_router", _p), ("bias", _p), ("w_gate_up", _p), ("w_down", _p),
                ("w_sh_gate_up", _p), ("w_sh_down", _p), ("out", _p), ("workspace", _p),
                ("workspace_bytes", ctypes.c_size_t), ("packed", _p), ("h", _p), ("inj", _p),
                ("inj_stride", _u32), ("inj_off", _u32), ("hc", _u32), ("x32", _p)]


ST_BF16, ST_F16, ST_F32, ST_I64, ST_I32, ST_U8, ST_OTHER = 0, 1, 2, 3, 4, 5, 15
ST_MAX_DIMS = 4


class StTensor(ctypes.Structure):
    _fields_ = [("data", _p), ("bytes", ctypes.c_uint64), ("dtype", _u32), ("ndim", _u32),
                ("shape", ctypes.c_uint64 * ST_MAX_DIMS), ("file", _u32)]


class WsLayout(ctypes.Structure):
    _fields_ = [("proj", ctypes.c_size_t), ("idx", ctypes.c_size_t), ("wt", ctypes.c_size_t),
                ("count", ctypes.c_size_t), ("off", ctypes.c_size_t), ("slot", ctypes.c_size_t),
                ("total", ctypes.c_size_t), ("proj_stride", _u32), ("items", ctypes.c_size_t),
                ("n_items", ctypes.c_size_t), ("n_items_hot", ctypes.c_size_t)]


class QwenMoe(ctypes.Structure):
    _fields_ = [("ctx", _p), ("d", _u32), ("experts", _u32), ("topk", _u32), ("inter", _u32), ("shared", _u32),
                ("hc", _u32), ("hc_rank", _u32), ("inj_stride", _u32), ("w_router", _p), ("w_gate_up", _p),
                ("w_down", _p), ("w_sh_gate_up", _p), ("w_sh_down", _p), ("max_rows", _u32), ("scratch", _p),
                ("scratch_bytes", ctypes.c_size_t), ("n_slots", _u32)]


class QwenLayout(ctypes.Structure):
    _fields_ = [("p", ctypes.c_size_t), ("idx", ctypes.c_size_t), ("wt", ctypes.c_size_t),
                ("count", ctypes.c_size_t), ("off", ctypes.c_size_t), ("slot", ctypes.c_size_t),
                ("xp", ctypes.c_size_t), ("amax", ctypes.c_size_t), ("total", ctypes.c_size_t),
                ("p_stride", _u32), ("hp", ctypes.c_size_t), ("hp16", ctypes.c_size_t), ("tiles", ctypes.c_size_t)]


# name -> (restype, argtypes)
SIGNATURES = {
    "rmda_moe_ctx_create": (ctypes.c_int, [ctypes.POINTER(_p), ctypes.c_int, _p]),
    "rmda_moe_ctx_destroy": (None, [_p]),
    "rmda_moe_set_stream": (ctypes.c_int, [_p, _p]),
    "rmda_moe_set_hot_rows": (ctypes.c_int, [_p, _u32]),
    "rmda_moe_set_tile_policy": (ctypes.c_int, [_p, ctypes.c_int]),
    "rmda_moe_set_fused_combine": (ctypes.c_int, [_p, ctypes.c_int]),
    "rmda_moe_set_route_in_rank": (ctypes.c_int, [_p, ctypes.c_int]),
    "rmda_moe_ctx_error": (ctypes.c_int, [_p]),
    "rmda_moe_ctx_message": (ctypes.c_char_p, [_p]),
    "rmda_moe_ctx_clear_error": (None, [_p]),
    "rmda_moe_sync": (ctypes.c_int, [_p]),
    "rmda_moe_version": (ctypes.c_char_p, []),
    "rmda_moe_abi_version": (ctypes.c_int, []),
    "rmda_moe_route": (ctypes.c_int, [_p, _p, _p, _p, _p, _p]),
    "rmda_moe_scan": (ctypes.c_int, [_p, _p, _p, _p, _p, _u32]),
    "rmda_moe_scatter": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _p]),
    "rmda_moe_scatter_experts": (ctypes.c_int, [_p, _u32]),
    "rmda_moe_mm": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p]),
    "rmda_moe_combine": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "rmda_moe_combine_plain": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _p]),
    "rmda_qwen_elem": (ctypes.c_int, [_p, _p, _p, _p]),
    "rmda_absmax": (ctypes.c_int, [_p, _p, _p, _p]),
    "rmda_cast_f16": (ctypes.c_int, [_p, _p, _p, _p, _p]),
    "rmda_qwen_bf16": (ctypes.c_int, [_p, _p, _p]),
    "rmda_moe_router": (ctypes.c_int, [_p, _p, _p, _p, _p, _p]),
    "rmda_moe_router_slot": (ctypes.c_int, [_p, _p, _p, _u32, _p, _p, _p, _p]),
    "rmda_moe_workspace_bytes": (ctypes.c_size_t, [_p]),
    "rmda_moe_workspace_bytes_x32": (ctypes.c_size_t, [_p]),
    "rmda_moe_workspace_layout": (ctypes.c_int, [_p, _p]),
    "rmda_moe_layer": (ctypes.c_int, [_p, _p, _p]),
    "rmda_moe_packed_bytes": (ctypes.c_size_t, [_p]),
    "rmda_moe_layer_static": (ctypes.c_int, [_p, _p, _p]),
    "rmda_moe_pack_weights": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, ctypes.c_int, _p]),
    "rmda_moe_prof_begin": (ctypes.c_int, [_p]),
    "rmda_moe_prof_end": (ctypes.c_int, [_p, _p, _p]),
    "rmda_moe_prof_empty_ms": (ctypes.c_int, [_p, _p]),
    "rmda_moe_prof_stage_name": (ctypes.c_char_p, [_u32]),
    "rmda_moe_fill_normal_f16": (ctypes.c_int, [_p, _p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64,
                                                ctypes.c_float]),
    "rmda_moe_fill_normal_f32": (ctypes.c_int, [_p, _p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64,
                                                ctypes.c_float]),
    "rmda_st_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_p)]),
    "rmda_st_close": (None, [_p]),
    "rmda_st_message": (ctypes.c_char_p, []),
    "rmda_st_count": (_u32, [_p]),
    "rmda_st_name": (ctypes.c_char_p, [_p, _u32]),
    "rmda_st_find": (ctypes.c_int, [_p, ctypes.c_char_p, _p]),
    "rmda_moe_upload_layer": (ctypes.c_int, [_p, _p, ctypes.c_char_p, _p, _p]),
    "rmda_moe_upload_wait": (ctypes.c_int, [_p]),
    "rmda_qwen_moe_scratch_bytes": (ctypes.c_size_t, [_p]),
    "rmda_qwen_moe_layout": (ctypes.c_int, [_p, _p]),
    "rmda_qwen_moe_mm": (ctypes.c_int, [_p, _p, _u32, _p, _p, _u32, _u32, _u32]),
    "rmda_qwen_route_rec": (ctypes.c_int, [_p, _u32, _u32]),
    "rmda_qwen_moe_rec": (ctypes.c_int, [_p, _p, _p, _p, _p, _u32]),
}

_LIB = None


def header_functions(path=HEADER_PATH):
    """Names of every function the C header declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rmda_\w+)\s*\(", text)))


def lib():
    """The loaded library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("librmda_moe.so is missing at %s: build it with __graft_entry__.build() "
                               "(there is no CPU fallback)" % LIB_PATH)
        L = ctypes.CDLL(PARTIAL_LIB or LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            if PARTIAL_LIB and not hasattr(L, name):
                continue
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB
