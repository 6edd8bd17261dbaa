"""A seeded sweep of layer shapes drawn at random within the ABI's limits
(d a multiple of 256, inter a multiple of 128, 1..512 experts, top-k up to
min(16, experts), shared expert on or off, skewed or uniform routing,
1..699 tokens), each through the fused layer against the CPU oracle, the
way tests/test_gpu_layer.py checks the benchmark configurations:
- routing bit-exact;
- the output within max-abs 2e-3 and rel-L2 1e-3 on every row;
- packed weights bitwise equal to the HF layout.
On packed weights the compute tile (every expert hot), the streaming tile
and both enqueued (AUTO) must then give bitwise the same output.  Every
third shape also runs with fp32 activations of a random magnitude through
the slot-scaled mode, against the oracle's fp32-activation mode, and every
second one through the qwen.c recording (rmda_qwen_moe_rec) the same way.
"""
import numpy as np
import pytest
import torch

from gpu_util import u32
from oracle import oracle as orc
from rmda_moe import api, inputs
from test_gpu_layer import check_layer

pytestmark = pytest.mark.gpu

N_SHAPES = 24
SWEEP_SEED = 2026


def sweep_shapes(n, seed):
    rng = np.random.default_rng(seed)
    shapes = []
    for i in range(n):
        E = int(rng.choice([1, 2, 5, 8, 16, 33, 64, 128, 200, 512]))
        k = int(rng.integers(1, min(E, 16) + 1))
        inter = int(128 * rng.integers(1, 5))
        shapes.append(dict(name="sweep%02d" % i, rows=int(rng.integers(1, 700)), d=int(256 * rng.integers(1, 5)),
                           experts=E, topk=k, inter=inter, shared=inter if rng.random() < 0.3 else 0,
                           skew=bool(E >= 4 and rng.random() < 0.35)))
    return shapes


SHAPES = sweep_shapes(N_SHAPES, SWEEP_SEED)


@pytest.fixture(scope="module")
def ctx():
    torch.cuda.set_device(0)
    c = api.Context(0)
    yield c
    c.close()


def packed_out(ctx, inp, packed, policy, hot_rows):
    shape = inp["shape"]
    ctx.set_tile_policy(policy)
    ctx.set_hot_rows(hot_rows)
    ws = inputs.workspace_for(shape)
    ws.fill_(255)
    out = torch.full((shape["rows"], shape["d"]), float("nan"), dtype=torch.float16, device="cuda")
    ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, out, ws, packed=packed)
    ctx.sync()
    return out


@pytest.mark.parametrize("cfg", SHAPES, ids=lambda c: "%s_T%d_d%d_E%d_k%d_I%d%s%s" % (
    c["name"], c["rows"], c["d"], c["experts"], c["topk"], c["inter"], "_sh" if c["shared"] else "",
    "_skew" if c["skew"] else ""))
def test_sweep_layer(ctx, cfg):
    seed = int(cfg["name"][5:]) + 100
    out = check_layer(ctx, cfg, seed=seed)
    inp = inputs.make_inputs(ctx, cfg, seed=seed)
    packed = ctx.pack_weights(inp["shape"], inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                              inp["w_sh_down"])
    try:
        for policy, hot_rows in ((api.Context.TILE_HOT, 1), (api.Context.TILE_AUTO, 1), (api.Context.TILE_STREAM, 256)):
            got = packed_out(ctx, inp, packed, policy, hot_rows)
            assert torch.equal(got.view(torch.int16), out.view(torch.int16)), (policy, hot_rows)
    finally:
        ctx.set_tile_policy(api.Context.TILE_ADAPTIVE)
        ctx.set_hot_rows(256)


@pytest.mark.parametrize("cfg", SHAPES[::3], ids=lambda c: c["name"])
def test_sweep_fp32_activations(ctx, cfg):
    """The slot-scaled mode on the sweep's shapes: logits, routing and the
    permutation bit-exact against the oracle's fp32-activation mode, the
    output y (read from one hyper-connection stream, which starts at zero)
    within rel-L2 1e-3 and max-abs 1e-2 of its largest magnitude."""
    seed = int(cfg["name"][5:]) + 100
    mag = float(np.random.default_rng(seed).choice([1e-4, 1.0, 1e4]))
    print("x32 %s mag %g" % (cfg["name"], mag), flush=True)
    inp = inputs.make_inputs(ctx, cfg, seed=seed)
    shape = inp["shape"]
    T, d = shape["rows"], shape["d"]
    g = torch.Generator(device="cuda").manual_seed(seed)
    x32 = torch.randn(T, d, device="cuda", generator=g, dtype=torch.float32) * mag
    packed = ctx.pack_weights(shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                              inp["w_sh_down"])
    ws = torch.full((api.workspace_bytes_x32(shape),), 255, dtype=torch.uint8, device="cuda")
    h = torch.zeros(T, 1, d, dtype=torch.float32, device="cuda")
    inj = torch.zeros(T, 1, dtype=torch.float32, device="cuda")
    ctx.layer(shape, None, inp["w_router"], inp["bias"], None, None, None, None, None, ws, packed=packed, h=h, inj=inj,
              inj_stride=1, inj_off=0, hc=1, x32=x32)
    ctx.sync()
    host = inputs.to_host(inp)
    host["x"] = None
    host["x32"] = x32.cpu().numpy()
    ref = orc.layer(host, tile=16, x_scale=1, hp_scale=1, threads=16)
    views = api.ws_views(shape, ws)
    assert np.array_equal(views["proj"].cpu().numpy().view(np.uint32), ref["proj"].view(np.uint32)), "router logits"
    assert np.array_equal(u32(views["idx"]), ref["idx"]), "expert indices"
    assert np.array_equal(u32(views["count"]), ref["count"]), "per-expert counts"
    assert np.array_equal(u32(views["slot"]), ref["slot"]), "permutation"
    y = h[:, 0, :].cpu().numpy().astype(np.float64)
    want = ref["out"].astype(np.float64)
    assert np.isfinite(y).all()
    scale = np.abs(want).max()
    err = np.abs(y - want).max()
    rel = np.linalg.norm(y - want) / np.linalg.norm(want) if scale > 0 else 0.0
    print("  max|y| %.3g rel-L2 %.3g max-abs %.3g" % (scale, rel, err), flush=True)
    assert rel <= 1e-3 and err <= 1e-2 * scale, (rel, err)


@pytest.mark.parametrize("cfg", SHAPES[1::2], ids=lambda c: c["name"])
def test_sweep_recording(ctx, cfg):
    """The qwen.c recording (rmda_qwen_moe_rec: 128-row segments, slot-scaled
    fp16 casts, fp32 GEMM outputs) on every second sweep shape, from fp32
    activations of a random magnitude, into one hyper-connection stream
    (h += y * 2 * sigmoid(0) = y), against the oracle in the reference's
    mode: logits, routing, 128-row offsets and the permutation bit-exact, y
    within rel-L2 1e-3 and max-abs 1e-2 of its largest magnitude.  The
    recording takes no router bias, so skewed shapes route uniformly here."""
    seed = int(cfg["name"][5:]) + 200
    mag = float(np.random.default_rng(seed).choice([1e-4, 1.0, 1e4]))
    print("rec %s mag %g" % (cfg["name"], mag), flush=True)
    inp = inputs.make_inputs(ctx, cfg, seed=seed)
    shape = inp["shape"]
    T, d = shape["rows"], shape["d"]
    g = torch.Generator(device="cuda").manual_seed(seed)
    x32 = torch.randn(T, d, device="cuda", generator=g, dtype=torch.float32) * mag
    q = api.QwenMoe(ctx, shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                    inp["w_sh_down"], hc=1, hc_rank=0, inj_stride=1)
    q.scratch.fill_(255)
    h = torch.zeros(T, 1, d, dtype=torch.float32, device="cuda")
    inj = torch.zeros(T, 1, dtype=torch.float32, device="cuda")
    q.moe_rec(x32, T, inj=inj, h=h)
    ctx.sync()
    host = inputs.to_host(inp)
    host["x"] = None
    host["bias"] = None
    host["x32"] = x32.cpu().numpy()
    ref = orc.layer(host, tile=128, x_scale=1, hp_scale=1, threads=16)
    v = q.views(T)
    assert np.array_equal(v["p"].cpu().numpy().view(np.uint32), ref["proj"].view(np.uint32)), "router logits"
    assert np.array_equal(u32(v["idx"]), ref["idx"]), "expert indices"
    assert np.array_equal(u32(v["count"]), ref["count"]), "per-expert counts"
    assert np.array_equal(u32(v["off"]), ref["off"]), "128-row segment offsets"
    assert np.array_equal(u32(v["slot"]), ref["slot"]), "permutation"
    y = h[:, 0, :].cpu().numpy().astype(np.float64)
    want = ref["out"].astype(np.float64)
    assert np.isfinite(y).all()
    scale = np.abs(want).max()
    err = np.abs(y - want).max()
    rel = np.linalg.norm(y - want) / np.linalg.norm(want) if scale > 0 else 0.0
    print("  max|y| %.3g rel-L2 %.3g max-abs %.3g" % (scale, rel, err), flush=True)
    assert rel <= 1e-3 and err <= 1e-2 * scale, (rel, err)
