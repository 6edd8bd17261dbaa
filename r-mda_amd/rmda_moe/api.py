"""Python mirror of the C ABI (include/rmda_moe.h) over torch device tensors.

Method names and argument order follow the reference's per-kernel recording
calls (mda_vkc_run with the push-constant struct and buffers in binding
order, src/qwen.c:770-907); torch only supplies device memory and the stream.
Every call goes through librmda_moe.so and raises MoeError on a non-zero
status, carrying the context's sticky message.
"""
import ctypes

import torch

from . import _lib
from ._lib import (NONE, NO_SLOT, Bf16PC, CombinePC, ElemPC, LayerArgs, MmPC, RoutePC, RouterPC,
                   ScanPC, ScatterPC, Shape, SlotPC, WsLayout)


class MoeError(RuntimeError):
    def __init__(self, code, message):
        super().__init__("%s (%d): %s" % (_lib.ERRORS.get(code, "?"), code, message))
        self.code = code
        self.message = message


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return t.data_ptr()


def _u32(t):
    """Reinterpret an int32 tensor as the uint32 buffers of the ABI (no copy)."""
    return t


def shape_struct(shape):
    return Shape(shape["rows"], shape["d"], shape["experts"], shape["topk"], shape["inter"], shape["shared"])


def workspace_bytes(shape):
    """rmda_moe_workspace_bytes; 0 means the shape is rejected.  Host-only."""
    s = shape_struct(shape)
    return _lib.lib().rmda_moe_workspace_bytes(ctypes.byref(s))


def workspace_bytes_x32(shape):
    """rmda_moe_workspace_bytes_x32 (the fp32-activation mode); 0 = rejected."""
    s = shape_struct(shape)
    return _lib.lib().rmda_moe_workspace_bytes_x32(ctypes.byref(s))


def packed_bytes(shape):
    """rmda_moe_packed_bytes; 0 means the shape is rejected.  Host-only."""
    s = shape_struct(shape)
    return _lib.lib().rmda_moe_packed_bytes(ctypes.byref(s))


def workspace_layout(shape):
    s = shape_struct(shape)
    lay = WsLayout()
    rc = _lib.lib().rmda_moe_workspace_layout(ctypes.byref(s), ctypes.byref(lay))
    if rc != 0:
        raise MoeError(rc, "workspace layout rejected the shape")
    return {k: getattr(lay, k) for k, _ in WsLayout._fields_}


class Context:
    """One rmda_moe_ctx_t bound to a device and a stream (torch's current one
    by default)."""

    def __init__(self, device=0, stream=None):
        self.L = _lib.lib()
        self.device = device
        h = ctypes.c_void_p()
        raw = self._raw_stream(stream)
        rc = self.L.rmda_moe_ctx_create(ctypes.byref(h), device, raw)
        if rc != 0:
            raise MoeError(rc, "rmda_moe_ctx_create failed")
        self.h = h

    @staticmethod
    def _raw_stream(stream):
        if stream is None:
            return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        if isinstance(stream, int):
            return ctypes.c_void_p(stream)
        return ctypes.c_void_p(stream.cuda_stream)

    def close(self):
        if getattr(self, "h", None) is not None:
            self.L.rmda_moe_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream):
        self._check(self.L.rmda_moe_set_stream(self.h, self._raw_stream(stream)))

    def set_hot_rows(self, rows):
        """rmda_moe_set_hot_rows: rows that make an expert hot (0 = never use
        the compute tile)."""
        self._check(self.L.rmda_moe_set_hot_rows(self.h, int(rows)))

    TILE_ADAPTIVE, TILE_AUTO, TILE_STREAM, TILE_HOT = 0, 1, 2, 3

    def set_tile_policy(self, policy):
        """rmda_moe_set_tile_policy (TILE_ADAPTIVE, TILE_AUTO, TILE_STREAM, TILE_HOT)."""
        self._check(self.L.rmda_moe_set_tile_policy(self.h, int(policy)))

    def set_route_in_rank(self, on):
        """rmda_moe_set_route_in_rank: the top-k inside the rank launch above
        one rank block (two launches before gate_up instead of three)."""
        self._check(self.L.rmda_moe_set_route_in_rank(self.h, 1 if on else 0))

    def set_fused_combine(self, on):
        """rmda_moe_set_fused_combine: fold the combine into the down GEMM."""
        self._check(self.L.rmda_moe_set_fused_combine(self.h, 1 if on else 0))

    def _check(self, rc):
        if rc != 0:
            msg = self.L.rmda_moe_ctx_message(self.h)
            raise MoeError(rc, msg.decode() if msg else "")

    def error(self):
        return self.L.rmda_moe_ctx_error(self.h)

    def message(self):
        msg = self.L.rmda_moe_ctx_message(self.h)
        return msg.decode() if msg else ""

    def clear_error(self):
        self.L.rmda_moe_ctx_clear_error(self.h)

    def sync(self):
        self._check(self.L.rmda_moe_sync(self.h))

    # ---- per-stage drop-ins ----

    def route(self, rows, experts, topk, stride, proj, idx, wt, count):
        pc = RoutePC(rows, experts, topk, stride)
        self._check(self.L.rmda_moe_route(self.h, ctypes.byref(pc), _ptr(proj), _ptr(idx), _ptr(wt),
                                          _ptr(count)))

    def scan(self, experts, tile, count, off, tiles, n_tiles):
        pc = ScanPC(experts, tile)
        self._check(self.L.rmda_moe_scan(self.h, ctypes.byref(pc), _ptr(count), _ptr(off), _ptr(tiles),
                                         n_tiles))

    def scatter_experts(self, experts):
        self._check(self.L.rmda_moe_scatter_experts(self.h, experts))

    def scatter(self, rows, topk, d8, idx, off, fill, x16, xp, slot):
        pc = ScatterPC(rows, topk, d8)
        self._check(self.L.rmda_moe_scatter(self.h, ctypes.byref(pc), _ptr(idx), _ptr(off), _ptr(fill),
                                            _ptr(x16), _ptr(xp), _ptr(slot)))

    def mm(self, m, n, k, sa, sb, a, b, c, amax, tiles):
        pc = MmPC(m, n, k, sa, sb)
        self._check(self.L.rmda_moe_mm(self.h, ctypes.byref(pc), _ptr(a), _ptr(b), _ptr(c), _ptr(amax),
                                       _ptr(tiles)))

    def combine(self, pc_fields, wt, slot, y, proj, sh, inj, h):
        pc = CombinePC(*pc_fields)
        self._check(self.L.rmda_moe_combine(self.h, ctypes.byref(pc), _ptr(wt), _ptr(slot), _ptr(y),
                                            _ptr(proj), _ptr(sh), _ptr(inj), _ptr(h)))

    def combine_plain(self, pc_fields, wt, slot, y, proj, sh, out):
        pc = CombinePC(*pc_fields)
        self._check(self.L.rmda_moe_combine_plain(self.h, ctypes.byref(pc), _ptr(wt), _ptr(slot), _ptr(y),
                                                  _ptr(proj), _ptr(sh), _ptr(out)))

    def qwen_elem(self, rows, n, astride, ao, bo, op, scale, a, y):
        pc = ElemPC(rows, n, astride, ao, bo, op, scale)
        self._check(self.L.rmda_qwen_elem(self.h, ctypes.byref(pc), _ptr(a), _ptr(y)))

    def absmax(self, n, slot, x, amax):
        pc = SlotPC(n, slot)
        self._check(self.L.rmda_absmax(self.h, ctypes.byref(pc), _ptr(x), _ptr(amax)))

    def cast_f16(self, n, slot, src, dst, amax):
        pc = SlotPC(n, slot)
        self._check(self.L.rmda_cast_f16(self.h, ctypes.byref(pc), _ptr(src), _ptr(dst), _ptr(amax)))

    def qwen_bf16(self, n, w):
        pc = Bf16PC(n)
        self._check(self.L.rmda_qwen_bf16(self.h, ctypes.byref(pc), _ptr(w)))

    def router(self, rows, d, cols, stride, nbias, x16, w, bias, proj, slot=None, amax=None):
        """rmda_moe_router; with `slot` (and the slot words `amax`) x16 is a
        slot-scaled cast and rmda_moe_router_slot divides the scale out."""
        pc = RouterPC(rows, d, cols, stride, nbias)
        if slot is None:
            self._check(self.L.rmda_moe_router(self.h, ctypes.byref(pc), _ptr(x16), _ptr(w), _ptr(bias),
                                               _ptr(proj)))
        else:
            self._check(self.L.rmda_moe_router_slot(self.h, ctypes.byref(pc), _ptr(x16), slot, _ptr(amax), _ptr(w),
                                                    _ptr(bias), _ptr(proj)))

    # ---- fused layer ----

    def layer(self, shape, x, w_router, bias, w_gate_up, w_down, w_sh_gate_up, w_sh_down, out, workspace,
              packed=None, h=None, inj=None, inj_stride=0, inj_off=0, hc=0, x32=None):
        """rmda_moe_layer; with `h` (rows x hc x d fp32) the output is injected into
        the hyper-connection streams (and `out` may be None); with `x32` (fp32
        activations, x then None) the reference's scale-slot protocol runs."""
        s = shape_struct(shape)
        args = LayerArgs(_ptr(x), _ptr(w_router), _ptr(bias), _ptr(w_gate_up), _ptr(w_down),
                         _ptr(w_sh_gate_up), _ptr(w_sh_down), _ptr(out), _ptr(workspace),
                         workspace.numel() * workspace.element_size(), _ptr(packed), _ptr(h), _ptr(inj),
                         inj_stride, inj_off, hc, _ptr(x32))
        self._check(self.L.rmda_moe_layer(self.h, ctypes.byref(s), ctypes.byref(args)))

    def layer_static(self, shape, x, w_router, bias, out, packed=None, w_gate_up=None, w_down=None,
                     w_sh_gate_up=None, w_sh_down=None, h=None, inj=None, inj_stride=0, inj_off=0, hc=0, x32=None):
        """rmda_moe_layer_static: the layer on the library's static scratch
        (no workspace argument, nothing allocated); x32 as in layer()."""
        s = shape_struct(shape)
        args = LayerArgs(_ptr(x), _ptr(w_router), _ptr(bias), _ptr(w_gate_up), _ptr(w_down),
                         _ptr(w_sh_gate_up), _ptr(w_sh_down), _ptr(out), None, 0, _ptr(packed), _ptr(h), _ptr(inj),
                         inj_stride, inj_off, hc, _ptr(x32))
        self._check(self.L.rmda_moe_layer_static(self.h, ctypes.byref(s), ctypes.byref(args)))

    def pack_weights(self, shape, w_router, w_gate_up, w_down, w_sh_gate_up=None, w_sh_down=None, bf16=False,
                     packed=None):
        """rmda_moe_pack_weights into `packed` (allocated when None); returns it."""
        if packed is None:
            n = packed_bytes(shape)
            if n == 0:
                raise ValueError("shape rejected by rmda_moe_packed_bytes: %r" % (shape,))
            packed = torch.empty(n // 2, dtype=torch.float16, device=w_gate_up.device)
        s = shape_struct(shape)
        self._check(self.L.rmda_moe_pack_weights(self.h, ctypes.byref(s), _ptr(w_router), _ptr(w_gate_up),
                                                 _ptr(w_down), _ptr(w_sh_gate_up), _ptr(w_sh_down),
                                                 1 if bf16 else 0, _ptr(packed)))
        return packed

    def upload_layer(self, st, prefix, shape, packed=None):
        """rmda_moe_upload_layer from a SafeTensors (rmda_moe.st) into `packed`
        (allocated when None); returns it.  Enqueued on the upload stream."""
        if packed is None:
            n = packed_bytes(shape)
            if n == 0:
                raise ValueError("shape rejected by rmda_moe_packed_bytes: %r" % (shape,))
            packed = torch.empty(n // 2, dtype=torch.float16, device="cuda")
        s = shape_struct(shape)
        self._check(self.L.rmda_moe_upload_layer(self.h, st.h, prefix.encode(), ctypes.byref(s), _ptr(packed)))
        return packed

    def upload_wait(self):
        """The compute stream waits for every upload enqueued so far."""
        self._check(self.L.rmda_moe_upload_wait(self.h))

    # ---- stage profiler ----

    def prof_begin(self):
        self._check(self.L.rmda_moe_prof_begin(self.h))

    def prof_end(self):
        """Stop profiling; returns ({stage: summed ms}, layer calls covered)."""
        ms = (ctypes.c_double * _lib.PROF_STAGES)()
        n = ctypes.c_uint32()
        self._check(self.L.rmda_moe_prof_end(self.h, ms, ctypes.byref(n)))
        names = [self.L.rmda_moe_prof_stage_name(i).decode() for i in range(_lib.PROF_STAGES)]
        return dict(zip(names, list(ms))), n.value

    def prof_empty_ms(self):
        """rmda_moe_prof_empty_ms: summed empty-interval time of the last profiled run."""
        ms = ctypes.c_double()
        self._check(self.L.rmda_moe_prof_empty_ms(self.h, ctypes.byref(ms)))
        return ms.value

    def fill_normal(self, t, stream, seed, std):
        if t.dtype == torch.float16:
            self._check(self.L.rmda_moe_fill_normal_f16(self.h, _ptr(t), t.numel(), stream, seed, std))
        elif t.dtype == torch.float32:
            self._check(self.L.rmda_moe_fill_normal_f32(self.h, _ptr(t), t.numel(), stream, seed, std))
        else:
            raise ValueError("fill_normal supports float16 and float32")


def ws_views(shape, workspace):
    """Typed views of the routing intermediates inside a layer workspace."""
    lay = workspace_layout(shape)
    T, K, E = shape["rows"], shape["topk"], shape["experts"]
    base = workspace

    def view(off, n, dtype):
        nbytes = n * torch.tensor([], dtype=dtype).element_size()
        return base[off:off + nbytes].view(dtype)

    return {
        "proj": view(lay["proj"], T * lay["proj_stride"], torch.float32).view(T, lay["proj_stride"]),
        "idx": view(lay["idx"], T * K, torch.int32),
        "wt": view(lay["wt"], T * K, torch.float32),
        "count": view(lay["count"], E, torch.int32),
        "off": view(lay["off"], E, torch.int32),
        "slot": view(lay["slot"], T * K, torch.int32),
        "n_items": view(lay["n_items"], 1, torch.int32),
        "n_items_hot": view(lay["n_items_hot"], 1, torch.int32),
    }


class QwenMoe:
    """rmda_qwen_moe_t: the qwen.c MoE recording (mda_qwen_moe_rec,
    mda_qwen_route_rec, mda_qwen_moe_mm; src/qwen.c:770-907) over the stage
    entry points, with its scratch allocated here once for max_rows."""

    def __init__(self, ctx, shape, w_router, w_gate_up, w_down, w_sh_gate_up=None, w_sh_down=None, max_rows=None,
                 hc=0, hc_rank=0, inj_stride=0):
        self.ctx = ctx
        q = _lib.QwenMoe()
        q.ctx = ctx.h
        q.d, q.experts, q.topk = shape["d"], shape["experts"], shape["topk"]
        q.inter, q.shared = shape["inter"], shape["shared"]
        q.hc, q.hc_rank, q.inj_stride = hc, hc_rank, inj_stride
        self._keep = [w_router, w_gate_up, w_down, w_sh_gate_up, w_sh_down]
        q.w_router, q.w_gate_up, q.w_down = _ptr(w_router), _ptr(w_gate_up), _ptr(w_down)
        q.w_sh_gate_up, q.w_sh_down = _ptr(w_sh_gate_up), _ptr(w_sh_down)
        q.max_rows = shape["rows"] if max_rows is None else max_rows
        n = _lib.lib().rmda_qwen_moe_scratch_bytes(ctypes.byref(q))
        if n == 0:
            raise ValueError("rmda_qwen_moe_scratch_bytes rejected the configuration %r" % (shape,))
        self.scratch = torch.empty(n, dtype=torch.uint8, device="cuda")
        q.scratch = self.scratch.data_ptr()
        q.scratch_bytes = n
        self.q = q
        lay = _lib.QwenLayout()
        rc = _lib.lib().rmda_qwen_moe_layout(ctypes.byref(q), ctypes.byref(lay))
        if rc != 0:
            raise MoeError(rc, "rmda_qwen_moe_layout rejected the configuration")
        self.layout = {k: getattr(lay, k) for k, _ in _lib.QwenLayout._fields_}

    def moe_rec(self, x, rows, inj=None, h=None, out=None):
        self.ctx._check(_lib.lib().rmda_qwen_moe_rec(ctypes.byref(self.q), _ptr(x), _ptr(inj), _ptr(h), _ptr(out),
                                                     rows))

    def views(self, rows):
        """Typed views of the chunk's routing intermediates in the scratch."""
        lay, q = self.layout, self.q
        K, E = q.topk, q.experts
        mrows = (rows * K + E * 127 + 127) // 128 * 128  # mda_qwen_moe_rows (src/qwen.c:68-70)

        def view(off, n, dtype):
            nbytes = n * torch.tensor([], dtype=dtype).element_size()
            return self.scratch[off:off + nbytes].view(dtype)

        return {
            "p": view(lay["p"], rows * lay["p_stride"], torch.float32).view(rows, lay["p_stride"]),
            "idx": view(lay["idx"], rows * K, torch.int32),
            "wt": view(lay["wt"], rows * K, torch.float32),
            "count": view(lay["count"], E, torch.int32),
            "off": view(lay["off"], E, torch.int32),
            "slot": view(lay["slot"], rows * K, torch.int32),
            "amax": view(lay["amax"], 16, torch.int32),
            "hp": view(lay["hp"], mrows * q.inter, torch.float32).view(mrows, q.inter),
            "hp16": view(lay["hp16"], mrows * q.inter, torch.float16).view(mrows, q.inter),
            "tiles": view(lay["tiles"], mrows // 128, torch.int32),
        }
