"""The qwen.c MoE recording (rmda_qwen_moe_rec, rmda_qwen_route_rec,
rmda_qwen_moe_mm; src/qwen.c:770-907) against the CPU oracle's layer in the
reference's own mode: 128-row segments (mda_qwen_moe_rows), activations and
SwiGLU outputs cast to fp16 with power-of-two slot scales (src/qwen.c:500-539,
absmax.comp + cast_f16.comp) that the next GEMM divides out.

Routing intermediates are bit-exact (logits, expert indices, counts, 128-row
offsets, slots); the output is within the layer's tolerance.  The scratch is
filled with NaN bytes first, so a stage that leaves its part of the chain
unwritten shows up."""
import numpy as np
import pytest
import torch

from gpu_util import MAX_ABS, REL_L2, oracle_layer, out_metrics, u32
from oracle import oracle as orc
from rmda_moe import api, configs, inputs

pytestmark = pytest.mark.gpu

SHAPES = [
    configs.CONFIGS[1],  # tiny: 8 experts, top-2
    configs.CONFIGS[2],  # decode: 128 experts, top-8, T = 128
    dict(name="shared_small", rows=200, d=256, experts=16, topk=4, inter=128, shared=128, skew=False),
    dict(name="ragged_k5", rows=77, d=512, experts=24, topk=5, inter=256, shared=0, skew=False),
    # the reference teacher's own MoE shape (src/qwen.c:11-37), a 256-row chunk
    dict(name="teacher", rows=256, d=2560, experts=512, topk=10, inter=640, shared=640, skew=False),
]


@pytest.fixture(scope="module")
def ctx():
    torch.cuda.set_device(0)
    c = api.Context(0)
    yield c
    c.close()


def make_shim(ctx, inp, **kw):
    return api.QwenMoe(ctx, inp["shape"], inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                       inp["w_sh_down"], **kw)


@pytest.mark.parametrize("cfg", SHAPES, ids=[c["name"] for c in SHAPES])
def test_moe_rec_matches_oracle_reference_mode(ctx, cfg):
    print("shim %s" % cfg["name"], flush=True)
    inp = inputs.make_inputs(ctx, cfg, seed=3)
    T, d = cfg["rows"], cfg["d"]
    q = make_shim(ctx, inp)
    q.scratch.fill_(255)
    out = torch.full((T, d), float("nan"), dtype=torch.float16, device="cuda")
    q.moe_rec(inp["x"].float(), T, out=out)
    ctx.sync()
    ref = orc.layer(inputs.to_host(inp), tile=128, hp_scale=1, x_scale=1, threads=16)
    v = q.views(T)
    assert np.array_equal(v["p"].cpu().numpy().view(np.uint32), ref["proj"].view(np.uint32)), "router logits"
    assert np.array_equal(u32(v["idx"]), ref["idx"]), "expert indices"
    assert np.array_equal(u32(v["count"]), ref["count"]), "per-expert counts"
    assert np.array_equal(u32(v["off"]), ref["off"]), "128-row segment offsets"
    assert np.array_equal(u32(v["slot"]), ref["slot"]), "permutation"
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    max_abs, rel = out_metrics(got, ref["out"])
    print("  max-abs %.3g rel-L2 %.3g" % (max_abs, rel), flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)
    # three fp16 scale slots were taken: x, hp and (with a shared expert) hs
    assert q.q.n_slots == (3 if cfg["shared"] else 2)


@pytest.mark.parametrize("cfg_id,n_sample", [(3, 512), (5, 640)])
def test_moe_rec_matches_oracle_at_bench_sizes(ctx, cfg_id, n_sample):
    """The recording at the sizes bench.py times it (config 3: mrows 32 640
    over 255 tiles, the live-row and fused-SwiGLU GEMMs and the 128-row hp
    cast; config 5: 828 tiles and the shared expert) in the reference's
    mode: routing bit-exact on every token, the output within tolerance on a
    sample of tokens that holds a row in every used 128-row tile (one token
    per tile, then random ones up to n_sample)."""
    cfg = configs.CONFIGS[cfg_id]
    print("shim %s" % cfg["name"], flush=True)
    seed = 3
    inp = inputs.make_inputs(ctx, cfg, seed=seed)
    T, d, K = cfg["rows"], cfg["d"], cfg["topk"]
    q = make_shim(ctx, inp)
    q.scratch.fill_(255)
    out = torch.full((T, d), float("nan"), dtype=torch.float16, device="cuda")
    q.moe_rec(inp["x"].float(), T, out=out)
    ctx.sync()
    v = q.views(T)
    slot = u32(v["slot"])
    tiles = u32(v["tiles"])
    used = np.flatnonzero(tiles != 0xFFFFFFFF)
    tile_of_pair = np.where(slot == 0xFFFFFFFF, -1, slot.astype(np.int64) // 128)
    first_pair = np.full(tiles.size, -1, np.int64)
    for p in range(slot.size - 1, -1, -1):
        if tile_of_pair[p] >= 0:
            first_pair[tile_of_pair[p]] = p
    assert np.all(first_pair[used] >= 0), "a used tile holds no routed row"
    must = np.unique(first_pair[used] // K)
    rest = np.setdiff1d(np.arange(T), must)
    extra = np.random.default_rng(cfg_id).choice(rest, max(0, n_sample - must.size), replace=False)
    sel = np.sort(np.concatenate([must, extra])).astype(np.uint32)
    ref = oracle_layer(inp, cfg, seed, tile=128, hp_scale=1, x_scale=1, rows_sel=sel)
    assert np.array_equal(v["p"].cpu().numpy().view(np.uint32), ref["proj"].view(np.uint32)), "router logits"
    assert np.array_equal(u32(v["idx"]), ref["idx"]), "expert indices"
    assert np.array_equal(u32(v["count"]), ref["count"]), "per-expert counts"
    assert np.array_equal(u32(v["off"]), ref["off"]), "128-row segment offsets"
    assert np.array_equal(slot, ref["slot"]), "permutation"
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    max_abs, rel = out_metrics(got[sel.astype(np.int64)], ref["out"])
    print("  %d used tiles, %d tokens checked; max-abs %.3g rel-L2 %.3g" % (used.size, sel.size, max_abs, rel),
          flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


@pytest.mark.parametrize("cfg,hc,stride,rank", [
    (dict(name="hc", rows=96, d=256, experts=12, topk=3, inter=128, shared=128, skew=False), 4, 10, 3),
    # the teacher: 4 streams, injection logits at hc_rank 320 of rows padded to
    # MDA_QWEN_HC_PAD 384 (src/qwen.c:13-28, src/qwen.h:20-21)
    (dict(name="teacher", rows=128, d=2560, experts=512, topk=10, inter=640, shared=640, skew=False), 4, 384, 320),
], ids=["small", "teacher"])
def test_moe_rec_hyper_connection_streams(ctx, cfg, hc, stride, rank):
    """h[r, s, c] += y[r, c] * 2 * sigmoid(inj[r, hc_rank + s] / hc), the
    reference's combine epilogue (shader/moe_combine.comp:36-38), against the
    oracle's y; the plain output of the same call is the y the streams got."""
    inp = inputs.make_inputs(ctx, cfg, seed=5)
    T, d = cfg["rows"], cfg["d"]
    q = make_shim(ctx, inp, hc=hc, hc_rank=rank, inj_stride=stride)
    g = torch.Generator(device="cuda").manual_seed(9)
    h0 = torch.randn(T, hc, d, device="cuda", generator=g)
    inj = torch.randn(T, stride, device="cuda", generator=g) * 3
    h = h0.clone()
    out = torch.empty(T, d, dtype=torch.float16, device="cuda")
    q.moe_rec(inp["x"].float(), T, inj=inj, h=h, out=out)
    ctx.sync()
    ref = orc.layer(inputs.to_host(inp), tile=128, hp_scale=1, x_scale=1, threads=16)
    gate = 2.0 / (1.0 + np.exp(-inj.cpu().numpy().astype(np.float64)[:, rank:rank + hc] / hc))
    want = h0.cpu().numpy().astype(np.float64) + ref["out"].astype(np.float64)[:, None, :] * gate[:, :, None]
    err = np.abs(h.cpu().numpy().astype(np.float64) - want).max()
    print("  hc max-abs %.3g" % err, flush=True)
    assert err <= 2 * MAX_ABS, err
    max_abs, rel = out_metrics(out.float().cpu().numpy(), ref["out"])
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


FUSED_SWIGLU = [configs.CONFIGS[2], configs.CONFIGS[3], SHAPES[3], SHAPES[4]]


@pytest.mark.parametrize("cfg", FUSED_SWIGLU, ids=[c["name"] for c in FUSED_SWIGLU])
def test_moe_rec_fused_swiglu_matches_mm_then_elem(ctx, cfg):
    """The recording's gate_up writes SwiGLU(g) and hp's absmax slot from its
    epilogue and skips the padding rows of each 128-row segment, and the hp
    cast runs over those rows only.  On every row that holds a routed pair,
    hp and hp16 must be bitwise the public drop-ins run as the reference runs
    them (rmda_moe_mm over the whole tiles, fp32 g, rmda_qwen_elem op 0, then
    rmda_cast_f16 with hp's slot), and the slot the absmax of those rows."""
    print("fused swiglu %s" % cfg["name"], flush=True)
    inp = inputs.make_inputs(ctx, cfg, seed=5)
    T, d, E, K, I = cfg["rows"], cfg["d"], cfg["experts"], cfg["topk"], cfg["inter"]
    q = make_shim(ctx, inp)
    q.scratch.fill_(255)
    out = torch.empty(T, d, dtype=torch.float16, device="cuda")
    q.moe_rec(inp["x"].float(), T, out=out)
    ctx.sync()
    v = q.views(T)
    mrows = v["hp"].shape[0]
    off, count = u32(v["off"]), u32(v["count"])
    live = np.zeros(mrows, dtype=bool)
    for e in range(E):
        live[off[e]:off[e] + count[e]] = True
    assert live.sum() == T * K
    hp = v["hp"].cpu().numpy()[live]
    hp16 = v["hp16"].cpu().numpy().view(np.uint16)[live]
    slots = v["amax"].clone()
    # the reference's sequence on the same xp and x slot (slot 0)
    lay = q.layout
    xp = q.scratch[lay["xp"]:lay["xp"] + mrows * d * 2].view(torch.float16).view(mrows, d)
    g32 = torch.empty(mrows, 2 * I, dtype=torch.float32, device="cuda")
    ctx.mm(mrows, 2 * I, d, 0, 0xFFFFFFFF, xp, inp["w_gate_up"], g32, slots, v["tiles"])
    hp_ref = torch.empty(mrows, I, dtype=torch.float32, device="cuda")
    ctx.qwen_elem(mrows, I, 2 * I, 0, I, 0, 1.0, g32, hp_ref)
    ctx.sync()
    ref = hp_ref.cpu().numpy()[live]
    assert np.isfinite(ref).all()
    bad = np.flatnonzero((hp.view(np.uint32) != ref.view(np.uint32)).any(axis=1))
    assert bad.size == 0, "rows differ: %s" % bad[:8]
    amax = np.float32(np.abs(ref).max())
    assert slots[1].item() == int(amax.view(np.int32)), (slots[1].item(), amax)
    hp16_ref = torch.empty(mrows, I, dtype=torch.float16, device="cuda")
    ctx.cast_f16(mrows * I, 1, hp_ref, hp16_ref, slots)
    ctx.sync()
    ref16 = hp16_ref.cpu().numpy().view(np.uint16)[live]
    bad = np.flatnonzero((hp16 != ref16).any(axis=1))
    assert bad.size == 0, "hp16 rows differ: %s" % bad[:8]


def run_documented_stages(ctx, inp, buf, xp_garbage=None, x32=None, h=None):
    """One chunk through the stage entry points in the order INTEGRATION.md
    documents for a qwen.c that keeps its own recording (src/qwen.c:838-907):
    slot words zeroed (:500-503), x cast with a slot, the fp32 router on that
    cast with the slot's scale divided out, route, scan, xp zero-filled
    (:798), scatter, gate_up, qwen_elem op 0, hp absmax + cast with a slot,
    down, combine.  x is the fp16 inputs' fp32 copy, or `x32`; with `h` the
    combine adds y into one hyper-connection stream instead of writing
    buf["out"].  `buf` holds every buffer and is reused across calls, as the
    reference's scratch is."""
    s = inp["shape"]
    T, d, E, K, I = s["rows"], s["d"], s["experts"], s["topk"], s["inter"]
    mrows = (T * K + E * 127 + 127) // 128 * 128
    x = inp["x"].float() if x32 is None else x32
    amax = buf["amax"]
    amax.zero_()
    ctx.absmax(T * d, 0, x, amax)
    ctx.cast_f16(T * d, 0, x, buf["a16"], amax)
    ctx.router(T, d, E, E, 0, buf["a16"], inp["w_router"], None, buf["p"], slot=0, amax=amax)
    ctx.route(T, E, K, E, buf["p"], buf["idx"], buf["wt"], buf["count"])
    ctx.scan(E, 128, buf["count"], buf["off"], buf["tiles"], mrows // 128)
    if xp_garbage is not None:
        buf["xp"].view(torch.int16).fill_(xp_garbage)
    buf["xp"].zero_()  # the reference's fill of xp before the scatter
    ctx.scatter(T, K, d // 8, buf["idx"], buf["off"], buf["fill"], buf["a16"], buf["xp"], buf["slot"])
    ctx.mm(mrows, 2 * I, d, 0, 0xFFFFFFFF, buf["xp"], inp["w_gate_up"], buf["g"], amax, buf["tiles"])
    ctx.qwen_elem(mrows, I, 2 * I, 0, I, 0, 1.0, buf["g"], buf["hp"])
    ctx.absmax(mrows * I, 1, buf["hp"], amax)
    ctx.cast_f16(mrows * I, 1, buf["hp"], buf["hp16"], amax)
    ctx.mm(mrows, d, I, 1, 0xFFFFFFFF, buf["hp16"], inp["w_down"], buf["ye"], amax, buf["tiles"])
    if h is None:
        ctx.combine_plain((T, d, K, E, E, 0, 0, 0), buf["wt"], buf["slot"], buf["ye"], buf["p"], None, buf["out"])
    else:
        inj = torch.zeros(T, 1, dtype=torch.float32, device="cuda")
        ctx.combine((T, d, K, E, E, 1, 0, 1), buf["wt"], buf["slot"], buf["ye"], buf["p"], None, inj, h)
    ctx.sync()


def stage_buffers(cfg):
    """The stage sequence's buffers: those the stages overwrite start as NaN /
    all-ones; g, hp, hp16 and ye start at zero, so their only stale rows are
    an earlier chunk's."""
    T, d, E, K, I = cfg["rows"], cfg["d"], cfg["experts"], cfg["topk"], cfg["inter"]
    mrows = (T * K + E * 127 + 127) // 128 * 128
    f32e = lambda *shp: torch.full(shp, float("nan"), dtype=torch.float32, device="cuda")
    u32e = lambda n: torch.full((n,), -1, dtype=torch.int32, device="cuda")
    f16e = lambda *shp: torch.full(shp, float("nan"), dtype=torch.float16, device="cuda")
    z32 = lambda *shp: torch.zeros(shp, dtype=torch.float32, device="cuda")
    return dict(amax=u32e(16), a16=f16e(T, d), p=f32e(T, E), idx=u32e(T * K), wt=f32e(T * K),
                count=u32e(E), off=u32e(E), tiles=u32e(mrows // 128), xp=f16e(mrows, d), fill=u32e(E),
                slot=u32e(T * K), g=z32(mrows, 2 * I), hp=z32(mrows, I),
                hp16=torch.zeros(mrows, I, dtype=torch.float16, device="cuda"), ye=z32(mrows, d), out=f16e(T, d))


def test_documented_stage_sequence_on_stale_scratch(ctx):
    """The stage-by-stage sequence a qwen.c keeps when it drives the drop-ins
    itself, on a scratch the way the reference reuses it: a first chunk
    leaves its g, hp and ye behind (rows of tiles the second chunk does not
    use stay stale and reach qwen_elem and the absmax, as in the reference),
    and xp holds large finite garbage (fp16 61 280) until the documented zero
    fill.  rmda_moe_mm computes every row of each named tile, so only that
    fill keeps the padding rows' garbage out of g and the hp scale slot.  The
    second chunk against the oracle in the reference's mode: routing
    bit-exact, output within tolerance."""
    cfg = dict(name="stages", rows=300, d=512, experts=16, topk=4, inter=256, shared=0, skew=False)
    buf = stage_buffers(cfg)
    prev = inputs.make_inputs(ctx, cfg, seed=8)
    run_documented_stages(ctx, prev, buf)
    inp = inputs.make_inputs(ctx, cfg, seed=9)
    run_documented_stages(ctx, inp, buf, xp_garbage=0x7B7B)
    ref = orc.layer(inputs.to_host(inp), tile=128, hp_scale=1, x_scale=1)
    assert np.array_equal(buf["p"].cpu().numpy().view(np.uint32), ref["proj"].view(np.uint32)), "router logits"
    assert np.array_equal(u32(buf["idx"]), ref["idx"]), "expert indices"
    assert np.array_equal(u32(buf["count"]), ref["count"]), "per-expert counts"
    assert np.array_equal(u32(buf["off"]), ref["off"]), "128-row segment offsets"
    assert np.array_equal(u32(buf["slot"]), ref["slot"]), "permutation"
    got = buf["out"].float().cpu().numpy()
    assert np.isfinite(got).all()
    max_abs, rel = out_metrics(got, ref["out"])
    print("  max-abs %.3g rel-L2 %.3g" % (max_abs, rel), flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


@pytest.mark.parametrize("mag", [1e-4, 1e4])
def test_documented_stage_sequence_fp32_activations(ctx, mag):
    """The same stage sequence from fp32 activations outside fp16's normal
    range (|x| around 1e-4, where fp16 is subnormal, or 1e4, where SwiGLU and
    down outputs pass 65504), into one hyper-connection stream
    (h += y * 2 * sigmoid(0) = y): routing bit-exact against the oracle's
    fp32-activation mode, y within rel-L2 1e-3 and max-abs 1e-2 of its
    largest magnitude."""
    cfg = dict(name="stages", rows=300, d=512, experts=16, topk=4, inter=256, shared=0, skew=False)
    T, d = cfg["rows"], cfg["d"]
    buf = stage_buffers(cfg)
    inp = inputs.make_inputs(ctx, cfg, seed=12)
    g = torch.Generator(device="cuda").manual_seed(12)
    x32 = torch.randn(T, d, device="cuda", generator=g, dtype=torch.float32) * mag
    h = torch.zeros(T, 1, d, dtype=torch.float32, device="cuda")
    run_documented_stages(ctx, inp, buf, x32=x32, h=h)
    host = inputs.to_host(inp)
    host["x"] = None
    host["x32"] = x32.cpu().numpy()
    ref = orc.layer(host, tile=128, hp_scale=1, x_scale=1, threads=16)
    assert np.array_equal(buf["p"].cpu().numpy().view(np.uint32), ref["proj"].view(np.uint32)), "router logits"
    assert np.array_equal(u32(buf["idx"]), ref["idx"]), "expert indices"
    assert np.array_equal(u32(buf["off"]), ref["off"]), "128-row segment offsets"
    assert np.array_equal(u32(buf["slot"]), ref["slot"]), "permutation"
    y = h[:, 0, :].cpu().numpy().astype(np.float64)
    want = ref["out"].astype(np.float64)
    assert np.isfinite(y).all()
    scale = np.abs(want).max()
    err = np.abs(y - want).max()
    rel = np.linalg.norm(y - want) / np.linalg.norm(want)
    print("  mag %g max|y| %.3g rel-L2 %.3g max-abs %.3g" % (mag, scale, rel, err), flush=True)
    assert rel <= 1e-3 and err <= 1e-2 * scale, (rel, err)


def test_moe_rec_runs_twice_bitwise_and_chunks(ctx):
    """Run-to-run determinism, and a smaller second chunk through the same
    scratch (laid out for max_rows) gives the oracle's answer for that chunk."""
    cfg = configs.CONFIGS[1]
    inp = inputs.make_inputs(ctx, cfg, seed=7)
    T, d = cfg["rows"], cfg["d"]
    q = make_shim(ctx, inp)
    outs = []
    for _ in range(2):
        out = torch.empty(T, d, dtype=torch.float16, device="cuda")
        q.moe_rec(inp["x"].float(), T, out=out)
        ctx.sync()
        outs.append(out)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    n = 100
    small = dict(cfg, rows=n)
    sub = {k: (v[:n] if k == "x" else v) for k, v in inp.items()}
    sub["shape"] = configs.shape_of(small)
    out = torch.empty(n, d, dtype=torch.float16, device="cuda")
    q.moe_rec(inp["x"][:n].float().contiguous(), n, out=out)
    ctx.sync()
    ref = orc.layer(inputs.to_host(sub), tile=128, hp_scale=1, x_scale=1)
    max_abs, rel = out_metrics(out.float().cpu().numpy(), ref["out"])
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


def test_moe_rec_rejects_bad_calls(ctx):
    cfg = configs.CONFIGS[1]
    inp = inputs.make_inputs(ctx, cfg, seed=1)
    q = make_shim(ctx, inp, max_rows=64)
    out = torch.empty(cfg["rows"], cfg["d"], dtype=torch.float16, device="cuda")
    with pytest.raises(api.MoeError):
        q.moe_rec(inp["x"].float(), cfg["rows"], out=out)  # more rows than the scratch holds
    ctx.clear_error()
    with pytest.raises(api.MoeError):
        q.moe_rec(inp["x"].float(), 64)  # neither out nor h
    ctx.clear_error()
