"""A seeded sweep of the reference-shaped stage entry points (route, scan,
scatter, rmda_moe_mm, combine, router) over shapes drawn at random within
each one's documented limits, against the CPU oracle, the way
tests/test_gpu_stages.py checks hand-picked shapes: integer and index
outputs bit-exact, router logits bit-exact, floating-point outputs within
the tolerances written in each test.
"""
import numpy as np
import pytest
import torch

from gpu_util import dev, empty_u32, u16, u32
from oracle import oracle as orc
from rmda_moe import api
from test_gpu_stages import NONE, planted_logits

pytestmark = pytest.mark.gpu

N_CASES = 24
SEED = 4099


@pytest.fixture(scope="module")
def ctx():
    torch.cuda.set_device(0)
    c = api.Context(0)
    yield c
    c.close()


def draw(i):
    """Case i: a routing shape (rows, experts, topk) and the seed its data
    come from."""
    r = np.random.default_rng(SEED + i)
    experts = int(r.choice([1, 2, 3, 8, 31, 64, 100, 128, 257, 512]))
    topk = int(r.integers(1, min(16, experts) + 1))
    rows = int(r.integers(1, 6000))
    return r, rows, experts, topk


@pytest.mark.parametrize("i", range(N_CASES))
def test_sweep_route_scan_scatter(ctx, i):
    """route -> scan -> scatter on logits with planted ties, NaN, -inf and
    unselectable values, a random padded stride, a random segment tile and a
    random row width: idx, count, off, tiles, slot, fill and xp bit-exact, wt
    within 2e-6 relative."""
    r, rows, experts, topk = draw(i)
    stride = experts + int(r.integers(0, 8))
    tile = int(r.choice([1, 7, 16, 128]))
    d = 8 * int(r.integers(1, 65))
    print("case %d: rows %d experts %d topk %d stride %d tile %d d %d" % (i, rows, experts, topk, stride, tile, d),
          flush=True)
    p = planted_logits(rows, experts, stride, seed=SEED + i)
    idx_r, wt_r, cnt_r = orc.route(p, experts, topk)
    idx = empty_u32(rows * topk)
    wt = torch.empty(rows * topk, dtype=torch.float32, device="cuda")
    cnt = empty_u32(experts, fill=99)
    ctx.route(rows, experts, topk, stride, dev(p), idx, wt, cnt)
    n_tiles = int((rows * topk + experts * (tile - 1)) // tile + int(r.integers(0, 4)))
    off_r, tiles_r = orc.scan(cnt_r, tile, n_tiles)
    off = empty_u32(experts)
    tiles = empty_u32(n_tiles, fill=0x5A5A5A5A)
    ctx.scan(experts, tile, cnt, off, tiles, n_tiles)
    mrows = max(n_tiles * tile, 1)
    x = orc.fill_normal_f16(rows * d, 7, SEED + i, 1.0).reshape(rows, d)
    xp_r, slot_r, fill_r = orc.scatter(idx_r, off_r, x, topk, mrows)
    ctx.scatter_experts(experts)
    fill = empty_u32(experts, fill=777)
    slot = empty_u32(rows * topk)
    xp = torch.zeros(mrows, d, dtype=torch.float16, device="cuda")
    ctx.scatter(rows, topk, d // 8, idx, off, fill, dev(x), xp, slot)
    ctx.sync()
    assert np.array_equal(u32(idx), idx_r), "idx"
    assert np.array_equal(u32(cnt), cnt_r), "count"
    np.testing.assert_allclose(wt.cpu().numpy(), wt_r, rtol=2e-6, atol=1e-7)
    assert np.array_equal(u32(off), off_r), "off"
    assert np.array_equal(u32(tiles), tiles_r), "tiles"
    assert np.array_equal(u32(slot), slot_r), "slot"
    assert np.array_equal(u32(fill), fill_r), "fill"
    assert np.array_equal(u16(xp), xp_r), "xp"


@pytest.mark.parametrize("i", range(N_CASES))
def test_sweep_moe_mm(ctx, i):
    """rmda_moe_mm on a random tile map (unused tiles included), n a multiple
    of 128, k of 32, with or without scale slots (a zero slot word included):
    used rows within 1e-5 of max|C| of the oracle, unused rows untouched."""
    r = np.random.default_rng(SEED + 100 + i)
    E = int(r.integers(1, 40))
    ntile = int(r.integers(1, 25))
    n = 128 * int(r.integers(1, 9))
    k = 32 * int(r.integers(1, 33))
    m = 128 * ntile
    scaled = bool(r.random() < 0.5)
    print("case %d: E %d m %d n %d k %d scaled %d" % (i, E, m, n, k, scaled), flush=True)
    tiles = r.integers(0, E, ntile).astype(np.uint32)
    tiles[r.random(ntile) < 0.2] = NONE
    a = orc.fill_normal_f16(m * k, 11, SEED + i, 1.0).reshape(m, k)
    b = orc.fill_normal_f16(E * n * k, 12, SEED + i, 0.02).reshape(E, n, k)
    amax = np.zeros(4, np.uint32)
    sa = sb = NONE
    if scaled:
        amax[1] = np.float32(r.uniform(1e-3, 1e3)).view(np.uint32)
        amax[2] = np.float32(r.choice([0.0, 5.5])).view(np.uint32)
        sa, sb = 1, 2
    ref = orc.moe_mm(a, b, tiles, n, k, sa=sa, sb=sb, amax=amax, c_init=np.full((m, n), 1e30, np.float32))
    c = torch.full((m, n), 1e30, dtype=torch.float32, device="cuda")
    ctx.mm(m, n, k, sa, sb, dev(a), dev(b), c, dev(amax), dev(tiles))
    ctx.sync()
    got = c.cpu().numpy()
    skip = np.repeat(tiles == NONE, 128)
    assert np.all(got[skip] == 1e30), "rows of unused tiles must stay untouched"
    live = ~skip
    if live.any():
        err = np.abs(got[live] - ref[live]).max()
        assert err <= 1e-5 * max(1.0, np.abs(ref[live]).max()), err


@pytest.mark.parametrize("i", range(N_CASES))
def test_sweep_combine(ctx, i):
    """rmda_moe_combine (hc streams) and rmda_moe_combine_plain on a random
    routing, some pairs unrouted, with or without the shared expert, any
    width d (odd ones take the per-element kernel): the streams within 1e-5
    of the oracle, the fp16 output within 2e-3 of the oracle's rounded."""
    r, rows, experts, topk = draw(i)
    rows = min(rows, 3000)
    d = int(r.choice([4, 8, 64, 258, 1024, 2560, 7 * int(r.integers(1, 40))]))
    hc = int(r.integers(1, 5))
    shared = bool(r.random() < 0.5)
    pstride = experts + 1 + int(r.integers(0, 4))
    inj_stride = hc + int(r.integers(0, 6))
    inj_off = int(r.integers(0, inj_stride - hc + 1))
    print("case %d: rows %d experts %d topk %d d %d hc %d shared %d" % (i, rows, experts, topk, d, hc, shared),
          flush=True)
    p = r.standard_normal((rows, pstride)).astype(np.float32)
    idx, wt, _ = orc.route(p, experts, topk)
    nrows = rows * topk + int(r.integers(0, 50))
    slot = r.permutation(nrows)[: rows * topk].astype(np.uint32)
    slot[r.random(rows * topk) < 0.1] = NONE
    y = r.standard_normal((nrows, d)).astype(np.float32)
    sh = r.standard_normal((rows, d)).astype(np.float32) if shared else None
    inj = (r.standard_normal((rows, inj_stride)) * 3).astype(np.float32)
    fields = (rows, d, topk, pstride, experts, inj_stride, inj_off, hc)
    h0 = r.standard_normal((rows, hc, d)).astype(np.float32)
    ref = orc.combine(fields, wt, slot, y, p, sh, inj, h0)
    h = dev(h0)
    ctx.combine(fields, dev(wt), dev(slot), dev(y), dev(p), None if sh is None else dev(sh), dev(inj), h)
    ref_plain = orc.combine_plain(fields, wt, slot, y, p, sh)
    out = torch.empty(rows, d, dtype=torch.float16, device="cuda")
    ctx.combine_plain(fields, dev(wt), dev(slot), dev(y), dev(p), None if sh is None else dev(sh), out)
    ctx.sync()
    np.testing.assert_allclose(h.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(out.float().cpu().numpy(), orc.h2f(orc.f2h(ref_plain)), rtol=0, atol=2e-3)


@pytest.mark.parametrize("i", range(N_CASES))
def test_sweep_router(ctx, i):
    """rmda_moe_router on random rows, d a multiple of 128, columns and
    stride, with or without a bias on the first nbias columns: logits
    bit-exact against the oracle's canonical order, columns past cols
    untouched."""
    r = np.random.default_rng(SEED + 200 + i)
    rows = int(r.integers(1, 3000))
    d = 128 * int(r.integers(1, 24))
    cols = int(r.integers(1, 700))
    stride = cols + int(r.integers(0, 5))
    nbias = int(r.integers(0, cols + 1)) if r.random() < 0.5 else 0
    print("case %d: rows %d d %d cols %d stride %d nbias %d" % (i, rows, d, cols, stride, nbias), flush=True)
    x = orc.fill_normal_f16(rows * d, 1, SEED + i, 1.0).reshape(rows, d)
    w = orc.fill_normal_f32(cols * d, 2, SEED + i, 0.02).reshape(cols, d)
    b = r.standard_normal(cols).astype(np.float32) if nbias else None
    ref = orc.router(x, w, b, nbias=nbias, stride=stride)
    proj = torch.full((rows, stride), 7.0, dtype=torch.float32, device="cuda")
    ctx.router(rows, d, cols, stride, nbias, dev(x), dev(w), None if b is None else dev(b), proj)
    ctx.sync()
    got = proj.cpu().numpy()
    assert np.array_equal(got[:, :cols].view(np.uint32), ref[:, :cols].view(np.uint32))
    assert np.all(got[:, cols:] == 7.0), "columns beyond cols must stay untouched"
