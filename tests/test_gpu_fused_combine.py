"""The combine folded into the down GEMM (rmda_moe_set_fused_combine).

Each down-GEMM wave that stores the last of a token's rows for 64 output
columns sums them there, with the combine kernel's own arithmetic, so the
folded layer must give bitwise the same fp16 output and hyper-connection
streams as the layer with the separate combine kernel, which
test_gpu_layer.py checks against the oracle.  Covered: every benchmark
configuration (config 4 runs the compute tile, where the combine kernel
still runs and the folded path must stand aside), the reference teacher's
shape, a shared expert with every token on one routed expert, tokens that
select nothing, and the arrival counters over repeated calls on a workspace
full of garbage.
"""
import numpy as np
import pytest
import torch

from gpu_util import MAX_ABS, REL_L2, oracle_layer, out_metrics, u32
from rmda_moe import api, configs, inputs

pytestmark = pytest.mark.gpu

TEACHER = dict(name="teacher", rows=256, d=2560, experts=512, topk=10, inter=640, shared=640, skew=False)

SHAPES = [
    configs.CONFIGS[1],
    configs.CONFIGS[2],
    configs.CONFIGS[3],
    configs.CONFIGS[4],
    configs.CONFIGS[5],
    TEACHER,
    # one expert, shared expert on: every token's rows in one routed group and the shared group
    dict(name="e1_shared", rows=37, d=256, experts=1, topk=1, inter=128, shared=128, skew=False),
    # 3081 pairs: a token's pairs straddle rank blocks (topk 3 does not divide 1024)
    dict(name="count_all_tail", rows=1027, d=256, experts=40, topk=3, inter=128, shared=0, skew=False),
    # skewed, shared expert: 61 of 64 experts empty, one with most tokens
    dict(name="skew_shared", rows=4096, d=512, experts=64, topk=2, inter=256, shared=256, skew=True),
]


@pytest.fixture(scope="module")
def ctx():
    torch.cuda.set_device(0)
    c = api.Context(0)
    yield c
    c.set_fused_combine(False)
    c.close()


def pack(ctx, inp):
    return ctx.pack_weights(inp["shape"], inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                            inp["w_sh_down"])


def layer(ctx, inp, packed, fused, ws=None, h=None, inj=None, inj_stride=0, inj_off=0, hc=0, with_out=True):
    shape = inp["shape"]
    ctx.set_fused_combine(fused)
    if ws is None:
        ws = inputs.workspace_for(shape)
        ws.fill_(255)  # garbage counters: the rank kernel presets them every call
    out = None
    if with_out:
        out = torch.full((shape["rows"], shape["d"]), float("nan"), dtype=torch.float16, device="cuda")
    ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, out, ws, packed=packed,
              h=h, inj=inj, inj_stride=inj_stride, inj_off=inj_off, hc=hc)
    ctx.sync()
    return out


ORACLE_SHAPES = [configs.CONFIGS[k] for k in (1, 2, 3, 4, 5)] + [TEACHER]


@pytest.mark.parametrize("cfg", ORACLE_SHAPES, ids=[c["name"] for c in ORACLE_SHAPES])
def test_fused_combine_vs_oracle(ctx, cfg):
    """The folded layer against the CPU oracle on every output row, with the
    hyper-connection streams and the fp16 output written by the same call
    (shader/moe_combine.comp:26-40, src/qwen.c:887-906): routing bit-exact,
    out within the layer tolerance, h within twice it.  Config 4 runs the
    compute tile, where combine16_kernel does the combine."""
    print("fused combine vs oracle %s" % cfg["name"], flush=True)
    seed = 0
    inp = inputs.make_inputs(ctx, cfg, seed=seed)
    packed = pack(ctx, inp)
    T, d = cfg["rows"], cfg["d"]
    hc, inj_stride, inj_off = (4, 384, 320) if cfg is TEACHER else (4, 11, 3)
    g = torch.Generator(device="cuda").manual_seed(9)
    h0 = torch.randn(T, hc, d, device="cuda", generator=g)
    inj = torch.randn(T, inj_stride, device="cuda", generator=g) * 3
    h = h0.clone()
    ws = inputs.workspace_for(inp["shape"])
    ws.fill_(255)
    out = layer(ctx, inp, packed, True, ws=ws, h=h, inj=inj, inj_stride=inj_stride, inj_off=inj_off, hc=hc)
    ref = oracle_layer(inp, cfg, seed, tile=16)
    views = api.ws_views(inp["shape"], ws)
    assert np.array_equal(u32(views["idx"]), ref["idx"]), "expert indices"
    assert np.array_equal(u32(views["count"]), ref["count"]), "per-expert counts"
    assert np.array_equal(u32(views["off"]), ref["off"]), "expert offsets"
    assert np.array_equal(u32(views["slot"]), ref["slot"]), "permutation"
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    max_abs, rel = out_metrics(got, ref["out"])
    print("  out max-abs %.3g rel-L2 %.3g" % (max_abs, rel), flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)
    gate = 2.0 / (1.0 + np.exp(-inj.cpu().numpy().astype(np.float64)[:, inj_off:inj_off + hc] / hc))
    want = h0.cpu().numpy().astype(np.float64) + ref["out"].astype(np.float64)[:, None, :] * gate[:, :, None]
    err = np.abs(h.cpu().numpy().astype(np.float64) - want).max()
    print("  hc max-abs %.3g" % err, flush=True)
    assert err <= 2 * MAX_ABS, err


@pytest.mark.parametrize("cfg", SHAPES, ids=[c["name"] for c in SHAPES])
def test_fused_combine_bitwise(ctx, cfg):
    print("fused combine %s" % cfg["name"], flush=True)
    inp = inputs.make_inputs(ctx, cfg, seed=11)
    packed = pack(ctx, inp)
    ref = layer(ctx, inp, packed, False)
    got = layer(ctx, inp, packed, True)
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), "folded combine differs from combine16"


@pytest.mark.parametrize("policy", [api.Context.TILE_AUTO, api.Context.TILE_ADAPTIVE, api.Context.TILE_STREAM])
def test_fused_combine_under_tile_policies(ctx, policy):
    """Config 4 (compute tile chosen on the device) and config 3 (streaming
    tile) in turn: whichever tile runs, the output is the unfolded layer's."""
    try:
        ctx.set_tile_policy(policy)
        ins = {k: inputs.make_inputs(ctx, configs.CONFIGS[k], seed=0) for k in (3, 4)}
        packs = {k: pack(ctx, ins[k]) for k in (3, 4)}
        refs = {k: layer(ctx, ins[k], packs[k], False) for k in (3, 4)}
        for k in (4, 4, 3, 3, 4):
            got = layer(ctx, ins[k], packs[k], True)
            assert torch.equal(got.view(torch.int16), refs[k].view(torch.int16)), "config %d" % k
    finally:
        ctx.set_tile_policy(api.Context.TILE_ADAPTIVE)


@pytest.mark.parametrize("cfg,hc,inj_stride,inj_off,with_out", [
    (configs.CONFIGS[5], 4, 11, 3, False),
    (TEACHER, 4, 384, 320, True),
], ids=["fine_shared", "teacher"])
def test_fused_combine_hyper_connection(ctx, cfg, hc, inj_stride, inj_off, with_out):
    """The hyper-connection streams (h += y * 2 * sigmoid(inj / hc)) from the
    folded combine, with and without the fp16 output beside them."""
    inp = inputs.make_inputs(ctx, cfg, seed=4)
    packed = pack(ctx, inp)
    T, d = cfg["rows"], cfg["d"]
    g = torch.Generator(device="cuda").manual_seed(9)
    h0 = torch.randn(T, hc, d, device="cuda", generator=g)
    inj = torch.randn(T, inj_stride, device="cuda", generator=g) * 3
    outs = []
    hs = []
    for fused in (False, True):
        h = h0.clone()
        outs.append(layer(ctx, inp, packed, fused, h=h, inj=inj, inj_stride=inj_stride, inj_off=inj_off, hc=hc,
                          with_out=with_out))
        hs.append(h)
    assert torch.equal(hs[1].view(torch.int32), hs[0].view(torch.int32)), "hyper-connection streams differ"
    if with_out:
        assert torch.equal(outs[1].view(torch.int16), outs[0].view(torch.int16))


def test_fused_combine_tokens_without_rows(ctx):
    """NaN tokens select no expert: no row of theirs reaches the down GEMM,
    so no wave combines them; the rank kernel writes their zero rows."""
    cfg = dict(name="nonfinite", rows=300, d=256, experts=16, topk=4, inter=128, shared=0, skew=False)
    inp = inputs.make_inputs(ctx, cfg, seed=13)
    inp["x"][5] = float("nan")
    inp["x"][177] = float("nan")
    packed = pack(ctx, inp)
    ref = layer(ctx, inp, packed, False)
    got = layer(ctx, inp, packed, True)
    assert bool((got[5] == 0).all()) and bool((got[177] == 0).all())
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_fused_combine_repeated_calls_one_workspace(ctx):
    """Back-to-back calls on one workspace, alternating inputs: the counters
    are preset by every call, whatever the previous call left."""
    cfg = configs.CONFIGS[3]
    ins = [inputs.make_inputs(ctx, cfg, seed=s) for s in (0, 1)]
    packs = [pack(ctx, i) for i in ins]
    refs = [layer(ctx, ins[i], packs[i], False) for i in range(2)]
    ws = inputs.workspace_for(ins[0]["shape"])
    ws.fill_(255)
    for rep in range(4):
        i = rep % 2
        got = layer(ctx, ins[i], packs[i], True, ws=ws)
        assert torch.equal(got.view(torch.int16), refs[i].view(torch.int16)), "call %d" % rep


def test_fused_combine_stage_profile(ctx):
    """With the combine folded in, no combine stage is recorded and the
    profiler still closes every call on its last recorded event."""
    cfg = configs.CONFIGS[2]
    inp = inputs.make_inputs(ctx, cfg, seed=0)
    packed = pack(ctx, inp)
    shape = inp["shape"]
    ws = inputs.workspace_for(shape)
    out = torch.empty(shape["rows"], shape["d"], dtype=torch.float16, device="cuda")
    ctx.set_fused_combine(True)
    ctx.prof_begin()
    for _ in range(5):
        ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, out, ws, packed=packed)
    stage_ms, n = ctx.prof_end()
    ctx.set_fused_combine(False)
    assert n == 5
    assert stage_ms["combine"] == 0.0 and stage_ms["down"] > 0.0 and stage_ms["gate_up"] > 0.0
