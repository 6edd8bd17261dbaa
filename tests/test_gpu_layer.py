"""Fused MoE layer (rmda_moe_layer) against the CPU oracle on every
benchmark configuration.

Routing intermediates are bit-exact (router logits, expert indices, counts,
offsets, slots); the fp16 output is within max-abs 2e-3 and relative L2 1e-3
of the oracle's fp32 output, on every output row (the oracle's layer runs
multithreaded), so every (work item, 16-row group) of both GEMMs is covered.
"""
import numpy as np
import pytest
import torch

from gpu_util import MAX_ABS, REL_L2, oracle_layer, out_metrics, u32
from oracle import oracle as orc
from rmda_moe import api, configs, inputs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    torch.cuda.set_device(0)
    c = api.Context(0)
    yield c
    c.close()


def run_layer(ctx, inp, packed=None):
    shape = inp["shape"]
    ws = inputs.workspace_for(shape)
    # all-ones bytes are NaN as fp16: a GEMM task the schedule skipped would
    # leave NaN activations that reach the output, not stale values of an
    # earlier call
    ws.fill_(255)
    out = torch.full((shape["rows"], shape["d"]), float("nan"), dtype=torch.float16, device="cuda")
    if packed is None:
        ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], inp["w_gate_up"], inp["w_down"],
                  inp["w_sh_gate_up"], inp["w_sh_down"], out, ws)
    else:
        # packed weights only: the HF-layout pointers are not passed
        ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, out, ws, packed=packed)
    ctx.sync()
    return out, api.ws_views(shape, ws)


def check_layer(ctx, cfg, seed, n_sample=None):
    print("layer %s seed %d" % (cfg["name"], seed), flush=True)
    inp = inputs.make_inputs(ctx, cfg, seed=seed)
    out, views = run_layer(ctx, inp)
    T = cfg["rows"]
    sel = None
    if n_sample is not None and n_sample < T:
        sel = np.sort(np.random.default_rng(seed).choice(T, n_sample, replace=False)).astype(np.uint32)
    ref = oracle_layer(inp, cfg, seed, tile=16, rows_sel=sel)
    assert np.array_equal(views["proj"].cpu().numpy().view(np.uint32), ref["proj"].view(np.uint32)), "router logits"
    assert np.array_equal(u32(views["idx"]), ref["idx"]), "expert indices"
    assert np.array_equal(u32(views["count"]), ref["count"]), "per-expert counts"
    assert np.array_equal(u32(views["off"]), ref["off"]), "expert offsets"
    assert np.array_equal(u32(views["slot"]), ref["slot"]), "permutation"
    np.testing.assert_allclose(views["wt"].cpu().numpy(), ref["wt"], rtol=2e-6, atol=1e-7)
    got = out.float().cpu().numpy()
    if sel is not None:
        got = got[sel]
    assert np.isfinite(got).all()
    max_abs, rel = out_metrics(got, ref["out"])
    print("  max-abs %.3g rel-L2 %.3g" % (max_abs, rel), flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)
    # packed weights feed the MFMAs the same LDS images: bitwise the same output
    proj = views["proj"].clone()
    packed = ctx.pack_weights(inp["shape"], inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                              inp["w_sh_down"])
    out_p, views_p = run_layer(ctx, inp, packed=packed)
    assert torch.equal(views_p["proj"].view(torch.int32), proj.view(torch.int32)), "packed-router logits differ"
    assert torch.equal(out_p.view(torch.int16), out.view(torch.int16)), "packed-weight output differs"
    return out


@pytest.mark.parametrize("cfg_id", [1, 2])
def test_layer_full(ctx, cfg_id):
    check_layer(ctx, configs.CONFIGS[cfg_id], seed=0)


@pytest.mark.parametrize("cfg_id", [3, 4, 5])
def test_layer_all_rows(ctx, cfg_id):
    check_layer(ctx, configs.CONFIGS[cfg_id], seed=0)


# The reference teacher's own MoE shape (src/qwen.c:11-37, src/qwen.h:20-21):
# hidden 2560, 512 experts, top-10, expert and shared width 640, at a row
# chunk of 256 tokens
TEACHER = dict(name="teacher", rows=256, d=2560, experts=512, topk=10, inter=640, shared=640, skew=False)


@pytest.mark.parametrize("cfg", [
    # one expert, shared expert on: every token in one group plus the dense group
    dict(name="e1_shared", rows=37, d=256, experts=1, topk=1, inter=128, shared=128, skew=False),
    # few experts, inter 128: gate_up N = 256 (one tile), down K = 128 (4 K steps)
    dict(name="e6_i128", rows=77, d=256, experts=6, topk=2, inter=128, shared=0, skew=False),
    # 130 columns: the router's fifth 32-column block holds 2 columns; top-k over 3 values per lane
    dict(name="e130_k7", rows=129, d=768, experts=130, topk=7, inter=384, shared=0, skew=False),
    # skewed routing at topk 1: hot experts get several 192-row work items
    dict(name="skew_k1", rows=900, d=512, experts=24, topk=1, inter=256, shared=256, skew=True),
    # maximum top-k, 512 experts, d not a multiple of 512 (1280 = 5 x 256: 10 sub-tiles per router chunk)
    dict(name="e512_k16", rows=33, d=1280, experts=512, topk=16, inter=128, shared=0, skew=False),
    # 3081 pairs: several rank blocks that all count every pair (count_all), a
    # partial last block and npairs % 4 = 1 pairs past the 16-byte words
    dict(name="count_all_tail", rows=1027, d=256, experts=40, topk=3, inter=128, shared=0, skew=False),
    # the wide router tile (64 tokens x 128 columns per workgroup, 49 x 4 of
    # them, the last token block ragged), the shared gate's column 512 by the
    # 32 x 32 tile in a second launch
    dict(name="wide_router_shared", rows=3100, d=256, experts=512, topk=4, inter=128, shared=128, skew=False),
    # 65 x 3 wide workgroups, no remainder columns, 6 k steps per router chunk
    dict(name="wide_router_e384", rows=4100, d=768, experts=384, topk=6, inter=128, shared=0, skew=False),
    # 32-token wide workgroups (64-token ones would be 32 x 4 < 192): 63 x 4,
    # the last token block ragged, the shared gate's column by the small tile
    dict(name="wide32_router_shared", rows=1999, d=512, experts=512, topk=4, inter=128, shared=128, skew=False),
    TEACHER,
], ids=lambda c: c["name"])
def test_layer_more_shapes(ctx, cfg):
    """Shapes away from the benchmark configurations, through both weight
    layouts, against the oracle: routing bit-exact, output within tolerance,
    packed bitwise equal to HF layout."""
    check_layer(ctx, cfg, seed=3)


@pytest.mark.parametrize("cfg", [
    # 524 288 pairs: 512 rank blocks hand their counts to the last one, and
    # about 2 800 work items of up to 192 rows are dealt over the persistent grid
    dict(name="large_uniform", rows=65536, d=256, experts=128, topk=8, inter=128, shared=0, skew=False),
    # skewed: 61 of 64 experts empty, one expert with all 32 768 tokens (171
    # items), plus a 32 768-row shared-expert group
    dict(name="large_skew_shared", rows=32768, d=512, experts=64, topk=2, inter=256, shared=256, skew=True),
])
def test_layer_large(ctx, cfg):
    """Sizes far above the benchmark configurations: routing bit-exact and
    output within tolerance on every token."""
    check_layer(ctx, cfg, seed=7)


def test_layer_teacher_chunk_2048(ctx):
    """The teacher's shape at a 2048-token chunk: with packed weights the
    router's wide tile (32-token workgroups) takes the 512 experts' columns
    and the route kernel the shared gate's; every logit bit-exact against the
    oracle and bitwise equal to the HF-layout call (whose router computes the
    gate itself), routing bit-exact, output within tolerance on sampled
    rows."""
    check_layer(ctx, dict(TEACHER, rows=2048, name="teacher_2048"), seed=5, n_sample=192)


def test_layer_other_seed_and_ragged(ctx):
    cfg = dict(configs.CONFIGS[1], rows=203, name="ragged")
    check_layer(ctx, cfg, seed=5)
    cfg = dict(configs.CONFIGS[3], rows=1, name="one_token")
    check_layer(ctx, cfg, seed=1)


@pytest.mark.parametrize("cfg,n_sample,hc,inj_stride,inj_off", [
    (configs.CONFIGS[1], None, 4, 11, 3),
    (configs.CONFIGS[5], 16, 4, 11, 3),
    # the teacher's streams: 4 of them, injection logits at hc_rank 320 of a
    # row padded to MDA_QWEN_HC_PAD 384 (src/qwen.h:20-21)
    (TEACHER, None, 4, 384, 320),
], ids=["tiny", "fine_shared", "teacher"])
def test_layer_hyper_connection_epilogue(ctx, cfg, n_sample, hc, inj_stride, inj_off):
    """h[r][s][c] += y[r][c] * 2 * sigmoid(inj[r*stride + off + s] / hc)
    (shader/moe_combine.comp:36-38), with y the fp32 layer output: checked
    against the oracle's fp32 output in float64; `out` may be omitted."""
    inp = inputs.make_inputs(ctx, cfg, seed=4)
    shape = inp["shape"]
    T, d = shape["rows"], shape["d"]
    g = torch.Generator(device="cuda").manual_seed(9)
    h0 = torch.randn(T, hc, d, device="cuda", generator=g)
    inj = torch.randn(T, inj_stride, device="cuda", generator=g) * 3
    h = h0.clone()
    ws = inputs.workspace_for(shape)
    ws.fill_(255)  # NaN as fp16: nothing unwritten may reach h
    ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], inp["w_gate_up"], inp["w_down"],
              inp["w_sh_gate_up"], inp["w_sh_down"], None, ws, h=h, inj=inj, inj_stride=inj_stride,
              inj_off=inj_off, hc=hc)
    ctx.sync()
    host = inputs.to_host(inp)
    sel = None
    if n_sample:
        sel = np.sort(np.random.default_rng(2).choice(T, n_sample, replace=False)).astype(np.uint32)
    ref = orc.layer(host, tile=16, rows_sel=sel, threads=16)
    rows = np.arange(T) if sel is None else sel.astype(np.int64)
    gate = 2.0 / (1.0 + np.exp(-inj.cpu().numpy().astype(np.float64)[rows, inj_off:inj_off + hc] / hc))
    want = h0.cpu().numpy()[rows].astype(np.float64) + ref["out"].astype(np.float64)[:, None, :] * gate[:, :, None]
    got = h.cpu().numpy()[rows].astype(np.float64)
    err = np.abs(got - want).max()
    print("  hc max-abs %.3g" % err, flush=True)
    assert err <= 2 * MAX_ABS, err
    assert torch.isfinite(h).all()


def test_layer_zero_rows_is_a_no_op(ctx):
    """rows = 0 (an empty chunk) enqueues nothing harmful and returns OK."""
    cfg = dict(configs.CONFIGS[3], rows=0, name="empty")
    inp = inputs.make_inputs(ctx, dict(configs.CONFIGS[3], rows=8), seed=0)
    shape = configs.shape_of(cfg)
    ws = inputs.workspace_for(shape)
    out = torch.full((1, shape["d"]), 3.0, dtype=torch.float16, device="cuda")  # pointers stay non-null
    ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], inp["w_gate_up"], inp["w_down"], None, None, out, ws)
    ctx.sync()
    assert bool((out == 3.0).all()), "nothing may be written for rows = 0"


def test_layer_deterministic(ctx):
    cfg = configs.CONFIGS[4]
    inp = inputs.make_inputs(ctx, cfg, seed=2)
    a, _ = run_layer(ctx, inp)
    b, _ = run_layer(ctx, inp)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_layer_skew_has_empty_experts(ctx):
    cfg = configs.CONFIGS[4]
    inp = inputs.make_inputs(ctx, cfg, seed=0)
    _, views = run_layer(ctx, inp)
    cnt = u32(views["count"])
    assert (cnt == 0).sum() > 0, "config 4 is meant to leave some experts empty"
    assert cnt.sum() == cfg["rows"] * cfg["topk"]


def test_pack_bf16_input_equals_fp16_of_converted(ctx):
    """bf16 packing converts like qwen_bf16 (round to nearest even), then packs."""
    cfg = dict(configs.CONFIGS[1], rows=64, name="bf16")
    shape = configs.shape_of(cfg)
    E, d, I = shape["experts"], shape["d"], shape["inter"]
    g = torch.Generator(device="cuda").manual_seed(3)
    gu = (torch.randn(E, 2 * I, d, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    dn = (torch.randn(E, d, I, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    wr = torch.randn(E, d, device="cuda", generator=g, dtype=torch.float32)
    p_bf = ctx.pack_weights(shape, wr, gu.view(torch.float16), dn.view(torch.float16), bf16=True)
    # reference conversion through the oracle's qwen_bf16 restatement
    gu16 = orc.qwen_bf16(gu.view(torch.int32).cpu().numpy().view(np.uint32))
    dn16 = orc.qwen_bf16(dn.view(torch.int32).cpu().numpy().view(np.uint32))
    gu_h = torch.from_numpy(gu16.view(np.int16)).cuda().view(torch.float16).view(E, 2 * I, d)
    dn_h = torch.from_numpy(dn16.view(np.int16)).cuda().view(torch.float16).view(E, d, I)
    p_h = ctx.pack_weights(shape, wr, gu_h, dn_h)
    ctx.sync()
    assert torch.equal(p_bf.view(torch.int16), p_h.view(torch.int16))
    # expert-weight packing is a permutation of the elements
    n_exp = E * 2 * I * d + E * d * I
    a = np.sort(p_h.view(torch.int16).cpu().numpy()[:n_exp])
    b = np.sort(np.concatenate([gu16.view(np.int16).ravel(), dn16.view(np.int16).ravel()]))
    assert np.array_equal(a, b)
    # the router matrix follows as [d/16][cols rounded up to 64][4][4] fp32, zero padded, bits
    # unchanged: element (k, c) at ((k/16)*cpad + c)*16 + (k%4)*4 + (k%16)/4
    cpad = (E + 63) // 64 * 64
    rt = p_h[n_exp:n_exp + 2 * d * cpad].view(torch.float32).cpu().numpy()
    assert rt.size == d * cpad
    # then 256 bytes: the down weights' largest row sum of |w|, then zeros
    tail = p_h[n_exp + 2 * d * cpad:].view(torch.float32).cpu().numpy()
    assert tail.size == 64 and np.all(tail[1:] == 0)
    rowsum = np.abs(orc.h2f(dn16.view(np.uint16)).astype(np.float64)).reshape(E, d, I).sum(axis=2).max()
    assert abs(tail[0] - rowsum) <= 1e-5 * rowsum, (tail[0], rowsum)
    want = np.zeros((d // 16, cpad, 4, 4), np.float32)
    # w[c][16g + 4s + kk] -> want[g][c][kk][s]
    want[:, :E] = wr.cpu().numpy().reshape(E, d // 16, 4, 4).transpose(1, 0, 3, 2)
    assert np.array_equal(rt.view(np.uint32), want.reshape(-1).view(np.uint32))
    k, c = 37, 5  # one element by the formula
    assert rt[((k // 16) * cpad + c) * 16 + (k % 4) * 4 + (k % 16) // 4] == wr[c, k].item()


@pytest.mark.parametrize("rows,experts", [(64, 16), (100, 64), (300, 64)],
                         ids=["router_topk", "rank_topk", "route_kernel"])
def test_layer_nonfinite_tokens(ctx, rows, experts):
    """A token whose activations are NaN has NaN logits, so no expert is
    selectable: its pairs carry RMDA_NONE through rank (not counted), the
    permutation (slot NONE), the work list and the combine (skipped), and its
    output row is 0 (no shared expert).  A token with one +inf activation has
    +inf or NaN logits.  Every other token's routing is bit-exact and its
    output within tolerance.  The three cases route in the router (16
    columns), in the rank kernel (one rank block) and in route_kernel (two
    rank blocks)."""
    cfg = dict(name="nonfinite", rows=rows, d=256, experts=experts, topk=4, inter=128, shared=0, skew=False)
    inp = inputs.make_inputs(ctx, cfg, seed=13)
    inp["x"][5] = float("nan")
    inp["x"][9, 3] = float("inf")
    out, views = run_layer(ctx, inp)
    ref = orc.layer(inputs.to_host(inp), tile=16)
    idx = u32(views["idx"])
    assert np.array_equal(idx, ref["idx"]), "expert indices (with RMDA_NONE)"
    assert np.all(idx.reshape(rows, 4)[5] == 0xFFFFFFFF), "a NaN token selects nothing"
    assert np.array_equal(u32(views["count"]), ref["count"]), "counts exclude unselected pairs"
    assert np.array_equal(u32(views["off"]), ref["off"])
    assert np.array_equal(u32(views["slot"]), ref["slot"])
    got = out.float().cpu().numpy()
    assert np.all(got[5] == 0.0), "no selected expert: zero output"
    ok = np.ones(rows, bool)
    ok[[5, 9]] = False
    assert np.isfinite(got[ok]).all()
    max_abs, rel = out_metrics(got[ok], ref["out"][ok])
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


def test_layer_rejects_misaligned_pointers():
    """x one fp16 element past 16-byte alignment: RMDA_ERR_ARG (-1) before
    anything is enqueued (the kernels read 16-byte chunks of x rows)."""
    c = api.Context(0)
    inp = inputs.make_inputs(c, configs.CONFIGS[1], seed=0)
    shape = inp["shape"]
    x = inp["x"]
    xbuf = torch.empty(x.numel() + 8, dtype=torch.float16, device="cuda")
    xm = xbuf[1:1 + x.numel()].view_as(x)
    assert xm.data_ptr() % 16 != 0
    out = torch.empty(shape["rows"], shape["d"], dtype=torch.float16, device="cuda")
    with pytest.raises(api.MoeError) as e:
        c.layer(shape, xm, inp["w_router"], inp["bias"], inp["w_gate_up"], inp["w_down"], None, None, out,
                inputs.workspace_for(shape))
    assert e.value.code == -1
    c.close()


@pytest.mark.parametrize("cfg", [
    configs.CONFIGS[3],
    configs.CONFIGS[4],
    configs.CONFIGS[5],
    # 3081 pairs: 4 rank blocks, a partial last one, a token's pairs straddling two
    dict(name="count_all_tail", rows=1027, d=256, experts=40, topk=3, inter=128, shared=0, skew=False),
    # 65 536 pairs, the largest call that routes in the rank launch (64 rank blocks)
    dict(name="rank_all_max", rows=8192, d=256, experts=64, topk=8, inter=128, shared=128, skew=False),
], ids=lambda c: c["name"])
def test_layer_route_in_rank(ctx, cfg):
    """rmda_moe_set_route_in_rank: the top-k selected inside the rank launch
    (one workgroup per 8 tokens, the last ones to finish ranking after the
    ticket) gives bitwise the routing, permutation and output of the separate
    route launch, which test_layer_all_rows checks against the oracle; two
    calls in a row, so the ticket the router clears is reused."""
    print("route in rank %s" % cfg["name"], flush=True)
    inp = inputs.make_inputs(ctx, cfg, seed=6)
    packed = ctx.pack_weights(inp["shape"], inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                              inp["w_sh_down"])
    ref, vref = run_layer(ctx, inp, packed=packed)
    ctx.set_route_in_rank(True)
    try:
        for _ in range(2):
            out, v = run_layer(ctx, inp, packed=packed)
            for k in ("idx", "wt", "count", "off", "slot"):
                assert torch.equal(v[k].view(torch.int32), vref[k].view(torch.int32)), k
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    finally:
        ctx.set_route_in_rank(False)


@pytest.mark.parametrize("cfg,mag,n_sample", [
    (configs.CONFIGS[1], 1.0, None),
    (configs.CONFIGS[1], 1e6, None),
    (configs.CONFIGS[1], 1e-6, None),
    (dict(name="shared_small", rows=300, d=512, experts=16, topk=4, inter=256, shared=256, skew=False), 1e6, None),
    (configs.CONFIGS[3], 1e6, 256),
    (configs.CONFIGS[4], 1e-6, 256),
    # 512 experts + shared gate at 4096 tokens: the router's wide tile takes the
    # experts' columns and the route kernel the shared gate's
    (configs.CONFIGS[5], 1e-3, 128),
], ids=["tiny_1", "tiny_1e6", "tiny_1e-6", "shared_1e6", "prefill_1e6", "skewed_1e-6", "fine_shared_1e-3"])
def test_layer_fp32_activations(ctx, cfg, mag, n_sample):
    """rmda_moe_layer_args_t::x32: fp32 activations of magnitude 1e-6 .. 1e6
    (x32 = mag * N(0, 1), values not representable in fp16), through the
    reference's slot protocol: x cast with a slot (router and gate_up divide
    it out), hp cast with a slot (down divides it out), fp32 expert rows.
    Against the oracle's fp32-activation mode: logits, routing and
    permutation bit-exact; the layer output y, read from one
    hyper-connection stream (h += y * 2 * sigmoid(0), so h = y exactly from
    h = 0) because y itself leaves fp16's range, within relative L2 1e-3 and
    max-abs 1e-2 of the largest output.  The fp16 output of the same call
    equals fp16(y) where y fits.  The compute tile runs at config 4."""
    print("x32 %s mag %g" % (cfg["name"], mag), flush=True)
    inp = inputs.make_inputs(ctx, cfg, seed=12)
    shape = inp["shape"]
    T, d = shape["rows"], shape["d"]
    g = torch.Generator(device="cuda").manual_seed(12)
    x32 = torch.randn(T, d, device="cuda", generator=g, dtype=torch.float32) * mag
    packed = ctx.pack_weights(shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                              inp["w_sh_down"])
    ws = torch.empty(api.workspace_bytes_x32(shape), dtype=torch.uint8, device="cuda")
    ws.fill_(255)
    h = torch.zeros(T, 1, d, dtype=torch.float32, device="cuda")
    inj = torch.zeros(T, 1, dtype=torch.float32, device="cuda")
    out = torch.full((T, d), float("nan"), dtype=torch.float16, device="cuda")
    ctx.layer(shape, None, inp["w_router"], inp["bias"], None, None, None, None, out, ws, packed=packed, h=h, inj=inj,
              inj_stride=1, inj_off=0, hc=1, x32=x32)
    ctx.sync()
    host = inputs.to_host(inp)
    host["x"] = None
    host["x32"] = x32.cpu().numpy()
    sel = None
    if n_sample is not None:
        sel = np.sort(np.random.default_rng(12).choice(T, n_sample, replace=False)).astype(np.uint32)
    ref = orc.layer(host, tile=16, x_scale=1, hp_scale=1, rows_sel=sel, threads=16)
    views = api.ws_views(shape, ws)
    assert np.array_equal(views["proj"].cpu().numpy().view(np.uint32), ref["proj"].view(np.uint32)), "router logits"
    assert np.array_equal(u32(views["idx"]), ref["idx"]), "expert indices"
    assert np.array_equal(u32(views["count"]), ref["count"]), "per-expert counts"
    assert np.array_equal(u32(views["slot"]), ref["slot"]), "permutation"
    y = h[:, 0, :].cpu().numpy().astype(np.float64)
    if sel is not None:
        y = y[sel.astype(np.int64)]
    want = ref["out"].astype(np.float64)
    assert np.isfinite(y).all()
    err = np.abs(y - want).max()
    rel = np.linalg.norm(y - want) / np.linalg.norm(want)
    print("  max|y| %.3g rel-L2 %.3g max-abs %.3g" % (np.abs(want).max(), rel, err), flush=True)
    assert rel <= 1e-3 and err <= 1e-2 * np.abs(want).max(), (rel, err)
    # the fp16 output is the same y rounded, where it fits
    o = out.float().cpu().numpy().astype(np.float64)
    if sel is not None:
        o = o[sel.astype(np.int64)]
    y32 = h[:, 0, :].cpu().numpy()
    if sel is not None:
        y32 = y32[sel.astype(np.int64)]
    fits = np.abs(y32) < 65504
    assert np.array_equal(o[fits], y32[fits].astype(np.float16).astype(np.float64))


def test_layer_fp32_activations_of_fp16_values(ctx):
    """x32 holding fp32 copies of the fp16 activations: the slot scale is a
    power of two, exact on these values, so the logits and the routing are
    bitwise the fp16-input layer's, and the output differs only by keeping
    hp's and the expert rows' extra precision (within the layer tolerance)."""
    cfg = configs.CONFIGS[3]
    inp = inputs.make_inputs(ctx, cfg, seed=0)
    shape = inp["shape"]
    ref, vref = run_layer(ctx, inp)
    ws = torch.empty(api.workspace_bytes_x32(shape), dtype=torch.uint8, device="cuda")
    ws.fill_(255)
    out = torch.full((shape["rows"], shape["d"]), float("nan"), dtype=torch.float16, device="cuda")
    ctx.layer(shape, None, inp["w_router"], inp["bias"], inp["w_gate_up"], inp["w_down"], None, None, out, ws,
              x32=inp["x"].float())
    ctx.sync()
    v = api.ws_views(shape, ws)
    for k in ("proj", "idx", "wt", "count", "off", "slot"):
        assert torch.equal(v[k].view(torch.int32), vref[k].view(torch.int32)), k
    max_abs, rel = out_metrics(out.float().cpu().numpy(), ref.float().cpu().numpy())
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


def test_layer_fp32_activations_reused_workspace_and_tiles(ctx):
    """The slot-scaled mode keeps no state between calls: a call with
    activations of 1e-6 on a workspace that a 1e6 call used first (its hp
    absmax words then hold 1e6-scale values) is bitwise the same call on a
    fresh workspace; and the compute tile (every expert hot), the streaming
    tile and both launched (AUTO) give bitwise the same outputs."""
    cfg = dict(name="x32_reuse", rows=600, d=512, experts=16, topk=4, inter=256, shared=256, skew=True)
    inp = inputs.make_inputs(ctx, cfg, seed=21)
    shape = inp["shape"]
    T, d = shape["rows"], shape["d"]
    g = torch.Generator(device="cuda").manual_seed(21)
    x_big = torch.randn(T, d, device="cuda", generator=g, dtype=torch.float32) * 1e6
    x_small = torch.randn(T, d, device="cuda", generator=g, dtype=torch.float32) * 1e-6
    packed = ctx.pack_weights(shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                              inp["w_sh_down"])
    nbytes = api.workspace_bytes_x32(shape)

    def run(x32, ws, policy, hot_rows):
        ctx.set_tile_policy(policy)
        ctx.set_hot_rows(hot_rows)
        h = torch.zeros(T, 1, d, dtype=torch.float32, device="cuda")
        inj = torch.zeros(T, 1, dtype=torch.float32, device="cuda")
        out = torch.full((T, d), float("nan"), dtype=torch.float16, device="cuda")
        ctx.layer(shape, None, inp["w_router"], inp["bias"], None, None, None, None, out, ws, packed=packed, h=h,
                  inj=inj, inj_stride=1, inj_off=0, hc=1, x32=x32)
        ctx.sync()
        return h, out

    try:
        fresh = torch.full((nbytes,), 255, dtype=torch.uint8, device="cuda")
        ref_h, ref_out = run(x_small, fresh, api.Context.TILE_STREAM, 256)
        assert torch.isfinite(ref_h).all() and ref_h.abs().max() > 0
        ws = torch.full((nbytes,), 255, dtype=torch.uint8, device="cuda")
        big_h, _ = run(x_big, ws, api.Context.TILE_STREAM, 256)
        assert big_h.abs().max() > 1e3 * ref_h.abs().max()
        for policy, hot_rows in ((api.Context.TILE_STREAM, 256), (api.Context.TILE_HOT, 1),
                                 (api.Context.TILE_AUTO, 1), (api.Context.TILE_AUTO, 0)):
            h, out = run(x_small, ws, policy, hot_rows)
            print("x32 reuse: policy %d hot rows %d" % (policy, hot_rows), flush=True)
            assert torch.equal(h.view(torch.int32), ref_h.view(torch.int32)), (policy, hot_rows)
            assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), (policy, hot_rows)
    finally:
        ctx.set_tile_policy(api.Context.TILE_ADAPTIVE)
        ctx.set_hot_rows(256)


@pytest.mark.parametrize("mag", [1e4, 1e-4])
def test_layer_fp32_activations_large_down_rows(ctx, mag):
    """With packed weights the slot-scaled mode keeps the expert rows in fp16,
    multiplied by 2^-c where 2^c exceeds the down weights' largest row sum of
    |w|, a bound the packing writes into the packed buffer's last 256 bytes
    (checked here against numpy's float64 sums).  One expert's down row set
    to 4.0 throughout (row sum 1024, where the others sum to about 4) must
    not overflow: the output against the oracle's fp32-row mode, within the
    slot-scaled tolerance, and the same call on HF-layout weights (fp32
    rows) within it too."""
    cfg = dict(name="big_row", rows=300, d=512, experts=16, topk=4, inter=256, shared=256, skew=False)
    inp = inputs.make_inputs(ctx, cfg, seed=31)
    shape = inp["shape"]
    T, d = shape["rows"], shape["d"]
    inp["w_down"][3, 7, :] = 4.0
    packed = ctx.pack_weights(shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                              inp["w_sh_down"])
    ctx.sync()
    bound = packed.view(torch.uint8)[-256:-252].cpu().numpy().view(np.float32)[0]
    wd = np.abs(inp["w_down"].float().cpu().numpy().astype(np.float64)).sum(axis=2).max()
    ws_ = np.abs(inp["w_sh_down"].float().cpu().numpy().astype(np.float64)).sum(axis=1).max()
    want_bound = max(wd, ws_)
    assert want_bound == 1024.0
    assert abs(float(bound) - want_bound) <= 1e-5 * want_bound, (bound, want_bound)
    g = torch.Generator(device="cuda").manual_seed(31)
    x32 = torch.randn(T, d, device="cuda", generator=g, dtype=torch.float32) * mag
    host = inputs.to_host(inp)
    host["x"] = None
    host["x32"] = x32.cpu().numpy()
    ref = orc.layer(host, tile=16, x_scale=1, hp_scale=1, threads=16)
    want = ref["out"].astype(np.float64)
    idx = ref["idx"].reshape(T, -1)
    assert (idx == 3).any(), "expert 3 must be routed"
    for layout in ("packed", "hf"):
        ws = torch.full((api.workspace_bytes_x32(shape),), 255, dtype=torch.uint8, device="cuda")
        h = torch.zeros(T, 1, d, dtype=torch.float32, device="cuda")
        inj = torch.zeros(T, 1, dtype=torch.float32, device="cuda")
        if layout == "packed":
            ctx.layer(shape, None, inp["w_router"], inp["bias"], None, None, None, None, None, ws, packed=packed,
                      h=h, inj=inj, inj_stride=1, inj_off=0, hc=1, x32=x32)
        else:
            ctx.layer(shape, None, inp["w_router"], inp["bias"], inp["w_gate_up"], inp["w_down"],
                      inp["w_sh_gate_up"], inp["w_sh_down"], None, ws, h=h, inj=inj, inj_stride=1, inj_off=0, hc=1,
                      x32=x32)
        ctx.sync()
        y = h[:, 0, :].cpu().numpy().astype(np.float64)
        assert np.isfinite(y).all(), layout
        err = np.abs(y - want).max()
        rel = np.linalg.norm(y - want) / np.linalg.norm(want)
        print("  %s max|y| %.3g rel-L2 %.3g max-abs %.3g" % (layout, np.abs(want).max(), rel, err), flush=True)
        assert rel <= 1e-3 and err <= 1e-2 * np.abs(want).max(), (layout, rel, err)


def test_layer_fp32_activations_rejections(ctx):
    """x and x32 together, and a workspace sized for the fp16 mode, are
    rejected before anything is enqueued."""
    cfg = configs.CONFIGS[1]
    inp = inputs.make_inputs(ctx, cfg, seed=0)
    shape = inp["shape"]
    x32 = inp["x"].float()
    out = torch.empty(shape["rows"], shape["d"], dtype=torch.float16, device="cuda")
    assert api.workspace_bytes_x32(shape) > api.workspace_bytes(shape)
    for x, ws, code in [(inp["x"], inputs.workspace_for(shape), -1), (None, inputs.workspace_for(shape), -6)]:
        with pytest.raises(api.MoeError) as e:
            ctx.layer(shape, x, inp["w_router"], None, inp["w_gate_up"], inp["w_down"], None, None, out, ws, x32=x32)
        assert e.value.code == code
        ctx.clear_error()
