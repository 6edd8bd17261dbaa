"""CPU suite: the C-ABI library loads, exports every function the header
declares, and its host-only logic (shape checks, workspace sizing and
layout, device check, error codes) behaves as documented.  No kernel is
launched here."""
import ctypes
import os
import re
import subprocess

import pytest

from rmda_moe import _lib, configs

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_lib.LIB_PATH):
        subprocess.run(["make", "-s", "-j8", "-C", _lib.CSRC_DIR, "all"], check=True)
    return _lib.lib()


def test_exports_every_header_function(L):
    names = _lib.header_functions()
    assert len(names) >= 25
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (rmda_\w+)$", out, re.M))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    # and nothing C++-mangled leaks through the ABI
    assert not re.search(r" T _Z\w*rmda_moe_(route|layer)", out)


def test_python_binding_covers_the_header():
    assert sorted(_lib.SIGNATURES) == _lib.header_functions()


def test_struct_layouts_match_reference_push_constants():
    # src/pc.h:369-404: all-uint32 structs, so size = 4 * fields
    for cls, n in [(_lib.RoutePC, 4), (_lib.ScanPC, 2), (_lib.ScatterPC, 3), (_lib.MmPC, 5),
                   (_lib.CombinePC, 8), (_lib.ElemPC, 7), (_lib.SlotPC, 2), (_lib.Bf16PC, 1)]:
        assert ctypes.sizeof(cls) == 4 * n


def test_version_and_stage_names(L):
    assert b"gfx950" in L.rmda_moe_version()
    # the library was built against this header's binary interface
    want = int(re.search(r"#define RMDA_MOE_ABI_VERSION (\d+)", open(_lib.HEADER_PATH).read()).group(1))
    assert L.rmda_moe_abi_version() == want
    names = [L.rmda_moe_prof_stage_name(i).decode() for i in range(_lib.PROF_STAGES)]
    assert names == ["router", "route", "rank", "permute", "gate_up", "down", "combine"]
    assert L.rmda_moe_prof_stage_name(_lib.PROF_STAGES) is None


def test_no_device_is_reported(L):
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    h = ctypes.c_void_p()
    assert L.rmda_moe_ctx_create(ctypes.byref(h), 0, None) == -7  # RMDA_ERR_DEVICE
    assert h.value is None
    assert L.rmda_moe_ctx_create(None, 0, None) == -1
    # null contexts are rejected without touching a device
    assert L.rmda_moe_sync(None) == -1
    assert L.rmda_moe_ctx_error(None) == -1
    assert L.rmda_moe_layer(None, None, None) == -1


def shape(**kw):
    s = dict(rows=2048, d=2048, experts=128, topk=8, inter=768, shared=0)
    s.update(kw)
    return _lib.Shape(s["rows"], s["d"], s["experts"], s["topk"], s["inter"], s["shared"])


@pytest.mark.parametrize("cfg_id", [1, 2, 3, 4, 5])
def test_workspace_layout_for_every_config(L, cfg_id):
    cfg = configs.CONFIGS[cfg_id]
    s = _lib.Shape(*[cfg[k] for k in ("rows", "d", "experts", "topk", "inter", "shared")])
    total = L.rmda_moe_workspace_bytes(ctypes.byref(s))
    assert total > 0
    lay = _lib.WsLayout()
    assert L.rmda_moe_workspace_layout(ctypes.byref(s), ctypes.byref(lay)) == 0
    assert lay.total == total
    T, K, E = cfg["rows"], cfg["topk"], cfg["experts"]
    assert lay.proj_stride == E + (1 if cfg["shared"] else 0)
    spans = sorted([(lay.proj, T * lay.proj_stride * 4), (lay.idx, T * K * 4), (lay.wt, T * K * 4),
                    (lay.slot, T * K * 4), (lay.count, E * 4), (lay.off, E * 4)])
    for (a, n), (b, _) in zip(spans, spans[1:]):
        assert a % 256 == 0 and a + n <= b, "workspace regions overlap"
    assert spans[-1][0] + spans[-1][1] <= total
    # the workspace holds the fp16 intermediates of every routed pair (+ shared rows)
    rows = T * K + (T if cfg["shared"] else 0)
    assert total >= rows * (cfg["inter"] + cfg["d"]) * 2


@pytest.mark.parametrize("bad", [dict(d=100), dict(d=0), dict(d=384), dict(experts=0), dict(experts=513),
                                 dict(topk=0), dict(topk=17), dict(experts=4, topk=5), dict(inter=96),
                                 dict(inter=192), dict(shared=64), dict(rows=1 << 28)])
def test_workspace_rejects_bad_shapes(L, bad):
    s = shape(**bad)
    assert L.rmda_moe_workspace_bytes(ctypes.byref(s)) == 0
    lay = _lib.WsLayout()
    assert L.rmda_moe_workspace_layout(ctypes.byref(s), ctypes.byref(lay)) == -2


def test_zero_rows_is_a_valid_shape(L):
    s = shape(rows=0)
    assert L.rmda_moe_workspace_bytes(ctypes.byref(s)) > 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.lib()


def _qwen(cfg, max_rows=None):
    q = _lib.QwenMoe()
    q.d, q.experts, q.topk, q.inter, q.shared = cfg["d"], cfg["experts"], cfg["topk"], cfg["inter"], cfg["shared"]
    q.max_rows = cfg["rows"] if max_rows is None else max_rows
    return q


def test_qwen_shim_scratch_sizing(L):
    """rmda_qwen_moe_scratch_bytes / _layout: the reference's MoE scratch
    (mda_qwen_scratch, src/qwen.c:166-179) for mrows = round(T*k + E*127, 128)."""
    cfg = configs.CONFIGS[3]
    q = _qwen(cfg)
    n = L.rmda_qwen_moe_scratch_bytes(ctypes.byref(q))
    T, d, E, K, I = cfg["rows"], cfg["d"], cfg["experts"], cfg["topk"], cfg["inter"]
    mrows = (T * K + E * 127 + 127) // 128 * 128
    assert mrows == 32640  # config 3: 2048 * 8 + 128 * 127 rounded up to 128 (255 tiles)
    # xp, g, hp, hp16 and ye alone
    assert n >= mrows * d * 2 + mrows * 2 * I * 4 + mrows * I * 6 + mrows * d * 4
    lay = _lib.QwenLayout()
    assert L.rmda_qwen_moe_layout(ctypes.byref(q), ctypes.byref(lay)) == 0
    assert lay.total == n and lay.p_stride == E
    offs = [lay.p, lay.idx, lay.wt, lay.count, lay.off, lay.slot, lay.xp, lay.amax, lay.hp, lay.hp16, lay.tiles]
    assert all(o % 256 == 0 for o in offs) and len(set(offs)) == len(offs) and max(offs) < n
    # a shared expert adds the gate column to p
    q5 = _qwen(configs.CONFIGS[5], max_rows=512)
    assert L.rmda_qwen_moe_layout(ctypes.byref(q5), ctypes.byref(lay)) == 0 and lay.p_stride == 513
    # rejected configurations size to 0
    for field, bad in [("d", 100), ("topk", 0), ("inter", 96), ("experts", 600), ("max_rows", 0), ("shared", 64)]:
        qb = _qwen(cfg)
        setattr(qb, field, bad)
        assert L.rmda_qwen_moe_scratch_bytes(ctypes.byref(qb)) == 0, field
