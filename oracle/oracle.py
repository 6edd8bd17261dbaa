"""ctypes view of the CPU oracle (oracle/libmoe_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.  Every function
restates a reference shader; the citations are in moe_oracle.c.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# RMDA_ORACLE_LIB: another build of the same source (the sanitized one of tests/asan)
LIB_PATH = os.environ.get("RMDA_ORACLE_LIB") or os.path.join(HERE, "libmoe_oracle.so")
REF_HASH_PATH = os.path.join(HERE, "_ref", "libref_hash.so")
REF_SAFET_PATH = os.path.join(HERE, "_ref", "libref_safet.so")

NONE = 0xFFFFFFFF
NO_SLOT = 0xFFFFFFFF

_u32 = ctypes.c_uint32
_p = ctypes.c_void_p


class RouterPC(ctypes.Structure):
    _fields_ = [("rows", _u32), ("d", _u32), ("cols", _u32), ("stride", _u32), ("nbias", _u32)]


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


class Shape(ctypes.Structure):
    _fields_ = [("rows", _u32), ("d", _u32), ("experts", _u32), ("topk", _u32), ("inter", _u32),
                ("shared", _u32)]


class Layer(ctypes.Structure):
    _fields_ = [("shape", Shape), ("tile", _u32), ("hp_scale", ctypes.c_int), ("x_scale", ctypes.c_int),
                ("threads", ctypes.c_int),
                ("x", _p), ("w_router", _p), ("bias", _p), ("w_gate_up", _p), ("w_down", _p),
                ("w_sh_gate_up", _p), ("w_sh_down", _p), ("rows_sel", _p), ("n_sel", _u32),
                ("out", _p), ("proj", _p), ("idx", _p), ("wt", _p), ("slot", _p), ("count", _p),
                ("off", _p), ("ye16", ctypes.c_int), ("stage_ms", _p), ("x32", _p)]

LAYER_STAGES = ("router", "route", "scan", "scatter", "gate_up", "down", "shared", "combine")


def build():
    """Compile the oracle (and oracle/_ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if os.path.isdir("/root/reference/src"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_h2f.restype = ctypes.c_float
        L.orc_h2f.argtypes = [ctypes.c_uint16]
        L.orc_f2h.restype = ctypes.c_uint16
        L.orc_f2h.argtypes = [ctypes.c_float]
        L.orc_hash_u64.restype = ctypes.c_uint64
        L.orc_hash_u64.argtypes = [ctypes.c_uint64] * 3
        L.orc_normal.restype = ctypes.c_float
        L.orc_normal.argtypes = [ctypes.c_uint64] * 3 + [ctypes.c_float]
        L.orc_slot_scale.restype = ctypes.c_float
        L.orc_slot_scale.argtypes = [_p, _u32]
        L.orc_proj_stride.restype = _u32
        L.orc_moe_layer.restype = ctypes.c_int
        for name in ["orc_h2f_n", "orc_f2h_n"]:
            getattr(L, name).argtypes = [_p, _p, ctypes.c_size_t]
        L.orc_fill_normal_f16.argtypes = [_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float]
        L.orc_fill_normal_f32.argtypes = [_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float]
        L.orc_router.argtypes = [_p, _p, _p, _p, _p, ctypes.c_int]
        L.orc_router_scaled.argtypes = [_p, _p, _p, _p, ctypes.c_float, _p, ctypes.c_int]
        L.orc_moe_route.argtypes = [_p, _p, _p, _p, _p]
        L.orc_moe_scan.argtypes = [_p, _p, _p, _p, _u32]
        L.orc_moe_scatter.argtypes = [_p] * 7
        L.orc_moe_mm.argtypes = [_p] * 6 + [ctypes.c_int]
        L.orc_moe_combine.argtypes = [_p] * 8
        L.orc_moe_combine_plain.argtypes = [_p] * 7
        L.orc_qwen_elem.argtypes = [_p, _p, _p]
        L.orc_absmax.argtypes = [_p, _p, _p]
        L.orc_cast_f16.argtypes = [_p, _p, _p, _p]
        L.orc_qwen_bf16.argtypes = [_p, _p]
        L.orc_moe_layer.argtypes = [_p]
        _LIB = L
    return _LIB


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(_p)


def _ref(s):
    return ctypes.byref(s)


def _nthreads(threads):
    if threads is None:
        threads = min(os.cpu_count() or 1, 16)
    return int(threads)


# ---- generator -----------------------------------------------------------

def fill_normal_f16(n, stream, seed, std):
    out = np.empty(n, np.uint16)
    lib().orc_fill_normal_f16(_ptr(out), n, stream, seed, std)
    return out


def fill_normal_f32(n, stream, seed, std):
    out = np.empty(n, np.float32)
    lib().orc_fill_normal_f32(_ptr(out), n, stream, seed, std)
    return out


def hash_u64(stream, key, i):
    return lib().orc_hash_u64(stream, key, i)


def f2h(a):
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().orc_f2h_n(_ptr(a), _ptr(out), a.size)
    return out


def h2f(a):
    a = np.ascontiguousarray(a, np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().orc_h2f_n(_ptr(a), _ptr(out), a.size)
    return out


# ---- per-stage -----------------------------------------------------------

def router(x16, w, bias=None, nbias=None, stride=None, threads=None, post=None):
    """proj = x16 . w^T (+ bias) in the canonical order.  x16 uint16 [T,d], w f32 [cols,d].
    With `post`, every chunk sum is multiplied by it before the bias
    (orc_router_scaled: the router on a slot-scaled x16 with 1/scale)."""
    T, d = x16.shape
    cols = w.shape[0]
    stride = cols if stride is None else stride
    nbias = (0 if bias is None else bias.shape[0]) if nbias is None else nbias
    proj = np.zeros((T, stride), np.float32)
    pc = RouterPC(T, d, cols, stride, nbias)
    args = (_ptr(np.ascontiguousarray(x16)), _ptr(np.ascontiguousarray(w)),
            _ptr(None if bias is None else np.ascontiguousarray(bias, np.float32)))
    if post is None:
        lib().orc_router(_ref(pc), *args, _ptr(proj), _nthreads(threads))
    else:
        lib().orc_router_scaled(_ref(pc), *args, post, _ptr(proj), _nthreads(threads))
    return proj


def route(proj, experts, topk, rows=None):
    rows = proj.shape[0] if rows is None else rows
    stride = proj.shape[1]
    idx = np.zeros(rows * topk, np.uint32)
    wt = np.zeros(rows * topk, np.float32)
    count = np.zeros(experts, np.uint32)
    pc = RoutePC(rows, experts, topk, stride)
    lib().orc_moe_route(_ref(pc), _ptr(np.ascontiguousarray(proj, np.float32)), _ptr(idx), _ptr(wt),
                        _ptr(count))
    return idx, wt, count


def scan(count, tile, n_tiles):
    experts = count.shape[0]
    off = np.zeros(experts, np.uint32)
    tiles = np.zeros(max(n_tiles, 1), np.uint32)
    pc = ScanPC(experts, tile)
    lib().orc_moe_scan(_ref(pc), _ptr(np.ascontiguousarray(count, np.uint32)), _ptr(off), _ptr(tiles),
                       n_tiles)
    return off, tiles[:n_tiles]


def scatter(idx, off, x16, topk, xp_rows):
    rows, d = x16.shape
    fill = np.zeros(off.shape[0], np.uint32)
    xp = np.zeros((xp_rows, d), np.uint16)
    slot = np.zeros(rows * topk, np.uint32)
    pc = ScatterPC(rows, topk, d // 8)
    lib().orc_moe_scatter(_ref(pc), _ptr(np.ascontiguousarray(idx, np.uint32)),
                          _ptr(np.ascontiguousarray(off, np.uint32)), _ptr(fill),
                          _ptr(np.ascontiguousarray(x16)), _ptr(xp), _ptr(slot))
    return xp, slot, fill


def moe_mm(a, b, tiles, n, k, sa=NO_SLOT, sb=NO_SLOT, amax=None, c_init=None, threads=None):
    m = a.shape[0]
    c = np.zeros((m, n), np.float32) if c_init is None else np.array(c_init, np.float32, copy=True)
    pc = MmPC(m, n, k, sa, sb)
    lib().orc_moe_mm(_ref(pc), _ptr(np.ascontiguousarray(a)), _ptr(np.ascontiguousarray(b)), _ptr(c),
                     _ptr(None if amax is None else np.ascontiguousarray(amax, np.uint32)),
                     _ptr(np.ascontiguousarray(tiles, np.uint32)), _nthreads(threads))
    return c


def combine(pc_fields, wt, slot, y, proj, sh, inj, h):
    pc = CombinePC(*pc_fields)
    h = np.array(h, np.float32, copy=True)
    lib().orc_moe_combine(_ref(pc), _ptr(wt), _ptr(slot), _ptr(y), _ptr(proj), _ptr(sh), _ptr(inj), _ptr(h))
    return h


def combine_plain(pc_fields, wt, slot, y, proj, sh):
    pc = CombinePC(*pc_fields)
    out = np.zeros((pc.rows, pc.d), np.float32)
    lib().orc_moe_combine_plain(_ref(pc), _ptr(wt), _ptr(slot), _ptr(y), _ptr(proj), _ptr(sh), _ptr(out))
    return out


def qwen_elem(a, rows, n, astride, ao, bo, op, scale=1.0):
    pc = ElemPC(rows, n, astride, ao, bo, op, scale)
    y = np.zeros(rows * n, np.float32)
    lib().orc_qwen_elem(_ref(pc), _ptr(np.ascontiguousarray(a, np.float32)), _ptr(y))
    return y


def absmax(x, amax, slot):
    amax = np.array(amax, np.uint32, copy=True)
    pc = SlotPC(x.size, slot)
    lib().orc_absmax(_ref(pc), _ptr(np.ascontiguousarray(x, np.float32)), _ptr(amax))
    return amax


def cast_f16(src, amax, slot):
    pc = SlotPC(src.size, slot)
    dst = np.zeros(src.size, np.uint16)
    lib().orc_cast_f16(_ref(pc), _ptr(np.ascontiguousarray(src, np.float32)), _ptr(dst),
                       _ptr(None if amax is None else np.ascontiguousarray(amax, np.uint32)))
    return dst


def slot_scale(amax, slot):
    amax = None if amax is None else np.ascontiguousarray(amax, np.uint32)
    return lib().orc_slot_scale(_ptr(amax), slot)


def qwen_bf16(w):
    w = np.array(w, np.uint32, copy=True)
    pc = Bf16PC(w.size)
    lib().orc_qwen_bf16(_ref(pc), _ptr(w))
    return w


def proj_stride(experts, shared):
    return experts + (1 if shared > 0 else 0)


def layer(inp, tile=1, hp_scale=1, x_scale=1, rows_sel=None, threads=None, ye16=False):
    """Whole layer in the reference order (plain output, fp32).

    `inp` is a dict of host numpy arrays (see rmda_moe.inputs): x, w_router,
    bias, w_gate_up, w_down, w_sh_gate_up, w_sh_down and the shape fields;
    an fp32 "x32" in place of x runs the reference's slot-scaled cast of x.
    ye16 rounds every expert output row to fp16 before the combine (the
    fused GPU layer's storage).  Returns a dict with out, the routing
    intermediates and stage_ms (wall-clock ms per stage, LAYER_STAGES).
    """
    s = inp["shape"]
    T, d, E, K = s["rows"], s["d"], s["experts"], s["topk"]
    ps = proj_stride(E, s["shared"])
    sel = None if rows_sel is None else np.ascontiguousarray(rows_sel, np.uint32)
    n_out = T if sel is None else sel.shape[0]
    res = {
        "out": np.zeros((n_out, d), np.float32),
        "proj": np.zeros((T, ps), np.float32),
        "idx": np.zeros(T * K, np.uint32),
        "wt": np.zeros(T * K, np.float32),
        "slot": np.zeros(T * K, np.uint32),
        "count": np.zeros(E, np.uint32),
        "off": np.zeros(E, np.uint32),
    }
    keep = []

    def P(name):
        a = inp.get(name)
        if a is None:
            return None
        a = np.ascontiguousarray(a)
        keep.append(a)
        return _ptr(a)

    L = Layer()
    L.shape = Shape(T, d, E, K, s["inter"], s["shared"])
    L.tile, L.hp_scale, L.x_scale, L.threads = tile, hp_scale, x_scale, _nthreads(threads)
    L.x, L.w_router, L.bias = P("x"), P("w_router"), P("bias")
    L.x32 = P("x32")  # fp32 activations (then x may be None)
    L.w_gate_up, L.w_down = P("w_gate_up"), P("w_down")
    L.w_sh_gate_up, L.w_sh_down = P("w_sh_gate_up"), P("w_sh_down")
    L.rows_sel = _ptr(sel)
    L.n_sel = 0 if sel is None else sel.shape[0]
    for k in ["out", "proj", "idx", "wt", "slot", "count", "off"]:
        setattr(L, k, _ptr(res[k]))
    L.ye16 = 1 if ye16 else 0
    stage_ms = np.zeros(len(LAYER_STAGES), np.float64)
    L.stage_ms = _ptr(stage_ms)
    rc = lib().orc_moe_layer(_ref(L))
    res["stage_ms"] = dict(zip(LAYER_STAGES, stage_ms.tolist()))
    if rc != 0:
        raise ValueError("oracle layer rejected the shape %r" % (s,))
    return res


def ref_hash_lib():
    """The reference's own src/hash.c built by oracle/Makefile, or None."""
    if not os.path.exists(REF_HASH_PATH):
        return None
    L = ctypes.CDLL(REF_HASH_PATH)
    L.mda_hash_u64.restype = ctypes.c_uint64
    L.mda_hash_u64.argtypes = [ctypes.c_uint64] * 3
    L.mda_hash_mix.restype = ctypes.c_uint64
    L.mda_hash_mix.argtypes = [ctypes.c_uint64]
    return L


class RefSafetFile(ctypes.Structure):  # mda_safet_file_t, src/safet.h:24-30
    _fields_ = [("bytes", _p), ("header", _p), ("data", _p), ("size", ctypes.c_uint64), ("mapped", ctypes.c_uint64)]


class RefSafetTensor(ctypes.Structure):  # mda_safet_tensor_t, src/safet.h:32-38
    _fields_ = [("data", _p), ("rows", _u32), ("cols", _u32), ("dtype", _u32), ("ok", ctypes.c_bool)]


def ref_safet_lib():
    """The reference's own src/safet.c built by oracle/Makefile, or None."""
    if not os.path.exists(REF_SAFET_PATH):
        return None
    L = ctypes.CDLL(REF_SAFET_PATH)
    L.mda_safet_read.restype = RefSafetFile
    L.mda_safet_read.argtypes = [ctypes.c_char_p]
    L.mda_safet_free.argtypes = [ctypes.POINTER(RefSafetFile)]
    L.mda_safet_has.restype = ctypes.c_bool
    L.mda_safet_has.argtypes = [ctypes.POINTER(RefSafetFile), ctypes.c_char_p]
    L.mda_safet_tensor.restype = RefSafetTensor
    L.mda_safet_tensor.argtypes = [ctypes.POINTER(RefSafetFile), ctypes.c_char_p]
    return L


class RefSafetSet(ctypes.Structure):  # mda_safet_set_t, src/safet.h:40-43
    _fields_ = [("files", _p), ("n", _u32)]


def ref_safet_set_api(L):
    """Bind the reference's shard-set functions (src/safet.c:236-275)."""
    L.mda_safet_open_set.restype = RefSafetSet
    L.mda_safet_open_set.argtypes = [ctypes.c_char_p]
    L.mda_safet_free_set.argtypes = [ctypes.POINTER(RefSafetSet)]
    L.mda_safet_find.restype = RefSafetTensor
    L.mda_safet_find.argtypes = [ctypes.POINTER(RefSafetSet), ctypes.c_char_p]
    L.mda_safet_set_file.restype = _u32
    L.mda_safet_set_file.argtypes = [ctypes.POINTER(RefSafetSet), ctypes.c_char_p]
    return L
