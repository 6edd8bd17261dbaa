"""Load buckets of the fused layer's grouped GEMMs: the compute tile for hot
experts (gemm_hot.hip) against the weight-streaming tile (gemm2.hip).

The rank kernel cuts the work list into 256-row items when experts with at
least `hot rows` rows hold half of the rows or more, else into 192-row items;
each GEMM launch reads its own count.  Both tiles run the same MFMA sequence
per output element, so the layer output must be bitwise identical whichever
tile runs; the streaming tile itself is checked against the oracle in
test_gpu_layer.py.
"""
import numpy as np
import pytest
import torch

from gpu_util import MAX_ABS, REL_L2, out_metrics, u32
from oracle import oracle as orc
from rmda_moe import api, configs, inputs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    """A context that lets the rank kernel choose the tile on every call
    (both tiles launch), so each call's lists show its own choice."""
    torch.cuda.set_device(0)
    c = api.Context(0)
    c.set_tile_policy(api.Context.TILE_AUTO)
    yield c
    c.set_hot_rows(256)
    c.close()


def packed_layer(ctx, inp, packed, hot_rows):
    """The packed layer; hot_rows None keeps the context's threshold (and its
    adaptive tile hint: setting the threshold resets it)."""
    shape = inp["shape"]
    if hot_rows is not None:
        ctx.set_hot_rows(hot_rows)
    ws = inputs.workspace_for(shape)
    ws.fill_(255)  # NaN activations wherever a task was skipped
    out = torch.full((shape["rows"], shape["d"]), float("nan"), dtype=torch.float16, device="cuda")
    ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, out, ws, packed=packed)
    ctx.sync()
    views = api.ws_views(shape, ws)
    n_stream = int(u32(views["n_items"])[0])
    n_hot = int(u32(views["n_items_hot"])[0])
    return out, views, n_stream, n_hot


def pack(ctx, inp):
    return ctx.pack_weights(inp["shape"], inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                            inp["w_sh_down"])


def test_bucket_choice(ctx):
    """Config 4 (ten experts hold 97% of the rows) takes the compute tile,
    config 3 (every expert 100-160 rows) the streaming tile; the list of the
    tile not taken is empty."""
    for cfg_id, want_hot in ((4, True), (3, False)):
        inp = inputs.make_inputs(ctx, configs.CONFIGS[cfg_id], seed=0)
        out, views, n_stream, n_hot = packed_layer(ctx, inp, pack(ctx, inp), 256)
        counts = u32(views["count"]).astype(np.int64)
        print("config %d: stream items %d, hot items %d" % (cfg_id, n_stream, n_hot), flush=True)
        if want_hot:
            assert n_stream == 0
            # every expert's rows in ceil(count / 256) items
            assert n_hot == int(((counts + 255) // 256).sum())
        else:
            assert n_hot == 0
            assert n_stream == int(((counts + 191) // 192).sum())
        assert torch.isfinite(out.float()).all()


SHAPES = [
    configs.CONFIGS[1],
    configs.CONFIGS[3],
    configs.CONFIGS[4],
    configs.CONFIGS[5],
    dict(name="e1_shared", rows=37, d=256, experts=1, topk=1, inter=128, shared=128, skew=False),
    dict(name="skew_k1", rows=900, d=512, experts=24, topk=1, inter=256, shared=256, skew=True),
    dict(name="ragged", rows=203, d=512, experts=8, topk=2, inter=1024, shared=0, skew=False),
    dict(name="e130_k7", rows=129, d=768, experts=130, topk=7, inter=384, shared=0, skew=False),
    # four hot experts hold ~35% of the rows, 124 cold ones the rest
    configs.MIXED,
]


@pytest.mark.parametrize("cfg", SHAPES, ids=[c["name"] for c in SHAPES])
def test_hot_tile_bitwise(ctx, cfg):
    """Compute tile forced (every expert with a row is hot) against the
    streaming tile forced (compute tile off): bitwise equal outputs, and each
    run used the list it was meant to."""
    print("hot tile %s" % cfg["name"], flush=True)
    inp = inputs.make_inputs(ctx, cfg, seed=2)
    packed = pack(ctx, inp)
    out_s, _, n_stream, n_hot0 = packed_layer(ctx, inp, packed, 0)
    assert n_hot0 == 0 and n_stream > 0
    out_h, _, n_stream1, n_hot = packed_layer(ctx, inp, packed, 1)
    assert n_stream1 == 0 and n_hot > 0
    assert torch.isfinite(out_h.float()).all()
    assert torch.equal(out_h.view(torch.int16), out_s.view(torch.int16)), "compute tile differs from streaming tile"


def test_mixed_load_bucket_and_oracle(ctx):
    """The mixed load: the hot bucket (four experts, ~35% of the rows) holds
    under half the rows, so the call runs the streaming tile; forced onto the
    compute tile it gives the same bits; and the output is within tolerance
    of the oracle on a sample of tokens."""
    cfg = configs.MIXED
    inp = inputs.make_inputs(ctx, cfg, seed=0)
    packed = pack(ctx, inp)
    out, views, n_stream, n_hot = packed_layer(ctx, inp, packed, 256)
    counts = u32(views["count"]).astype(np.int64)
    frac = counts[counts >= 256].sum() / counts.sum()
    print("mixed: hot experts %d, rows on them %.3f" % ((counts >= 256).sum(), frac), flush=True)
    assert (counts >= 256).sum() == len(configs.MIXED_HOT) and 0.25 < frac < 0.5
    assert n_hot == 0 and n_stream > 0
    out_h, _, n_stream1, n_hot1 = packed_layer(ctx, inp, packed, 1)
    assert n_stream1 == 0 and n_hot1 > 0
    assert torch.equal(out_h.view(torch.int16), out.view(torch.int16))
    ctx.set_hot_rows(256)
    sel = np.sort(np.random.default_rng(1).choice(cfg["rows"], 256, replace=False)).astype(np.uint32)
    ref = orc.layer(inputs.to_host(inp), tile=16, rows_sel=sel, threads=16)
    assert np.array_equal(u32(views["idx"]), ref["idx"])
    max_abs, rel = out_metrics(out.float().cpu().numpy()[sel.astype(np.int64)], ref["out"])
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


def test_hot_tile_against_oracle_config4(ctx):
    """The default (bucketed) layer at config 4 against the oracle on every
    output row: routing bit-exact, output within the acceptance tolerance."""
    cfg = configs.CONFIGS[4]
    inp = inputs.make_inputs(ctx, cfg, seed=0)
    out, views, n_stream, n_hot = packed_layer(ctx, inp, pack(ctx, inp), 256)
    assert n_hot > 0 and n_stream == 0
    ref = orc.layer(inputs.to_host(inp), tile=16, threads=16)
    assert np.array_equal(u32(views["idx"]), ref["idx"])
    assert np.array_equal(u32(views["slot"]), ref["slot"])
    got = out.float().cpu().numpy()
    max_abs, rel = out_metrics(got, ref["out"])
    print("  config 4 all rows: max-abs %.3g rel-L2 %.3g" % (max_abs, rel), flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


def test_adaptive_policy_follows_previous_call():
    """RMDA_TILE_ADAPTIVE (the default): the first call on a key (packed
    weights, rows) lets the rank kernel choose, later calls on that key launch
    only the tile its previous call chose and have the rank kernel cut its
    list for it, even when the new call's routing would choose the other
    tile; calls on another key neither read nor disturb that choice.  Every
    call's output is bitwise the streaming tile's."""
    torch.cuda.set_device(0)
    c = api.Context(0)
    try:
        ins = {k: inputs.make_inputs(c, configs.CONFIGS[k], seed=0) for k in (3, 4)}
        packs = {k: pack(c, ins[k]) for k in (3, 4)}
        # configs 3 and 4 share their weights (config 4 adds a router bias),
        # so either packed buffer serves either input
        assert torch.equal(packs[3].view(torch.int16), packs[4].view(torch.int16))
        # references: the streaming tile, on a context fixed to it
        ref = {}
        c.set_tile_policy(api.Context.TILE_STREAM)
        for k in (3, 4):
            ref[k], _, n_s, n_h = packed_layer(c, ins[k], packs[k], None)
            assert n_s > 0 and n_h == 0
        c.set_tile_policy(api.Context.TILE_ADAPTIVE)

        def call(k, key, want):
            out, _, n_s, n_h = packed_layer(c, ins[k], packs[key], None)
            got = "hot" if n_h > 0 else "stream"
            print("adaptive: config %d on weights %d used the %s tile" % (k, key, got), flush=True)
            assert got == want and (n_s == 0) == (n_h > 0)
            assert torch.equal(out.view(torch.int16), ref[k].view(torch.int16))

        # one key (packs[3]): the first call decides on the device; each
        # later call follows the one before it
        for k, want in [(4, "hot"), (4, "hot"), (3, "hot"), (3, "stream"), (4, "stream"), (4, "hot")]:
            call(k, 3, want)
        # a second key (packs[4]) keeps its own choice, interleaved with the first
        c.set_tile_policy(api.Context.TILE_ADAPTIVE)  # forget every key
        for k, key, want in [(4, 4, "hot"), (3, 3, "stream"), (4, 4, "hot"), (3, 3, "stream"), (4, 4, "hot")]:
            call(k, key, want)
    finally:
        c.close()
