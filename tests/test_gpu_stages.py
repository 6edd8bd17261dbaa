"""Per-stage parity of the HIP drop-ins against the CPU oracle, through the C ABI.

Integer/index outputs (idx, count, off, tiles, slot, fill, permuted rows,
router logits) must be bit-exact; floating-point outputs are held to the
tolerances written in each test.
"""
import numpy as np
import pytest
import torch

from gpu_util import dev, empty_u32, f32, u16, u32
from oracle import oracle as orc
from rmda_moe import api, configs

pytestmark = pytest.mark.gpu

NONE = 0xFFFFFFFF


@pytest.fixture(scope="module")
def ctx():
    torch.cuda.set_device(0)
    c = api.Context(0)
    yield c
    c.close()


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- generator

@pytest.mark.parametrize("n,stream,seed,std", [(100003, 3, 0, 0.02), (4096, 1, 7, 1.0)])
def test_fill_matches_oracle_bitwise(ctx, n, stream, seed, std):
    t16 = torch.empty(n, dtype=torch.float16, device="cuda")
    t32 = torch.empty(n, dtype=torch.float32, device="cuda")
    ctx.fill_normal(t16, stream, seed, std)
    ctx.fill_normal(t32, stream, seed, std)
    ctx.sync()
    assert np.array_equal(u16(t16), orc.fill_normal_f16(n, stream, seed, std))
    assert np.array_equal(t32.cpu().numpy().view(np.uint32), orc.fill_normal_f32(n, stream, seed, std).view(np.uint32))


# ---------------------------------------------------------------- router (A0)

@pytest.mark.parametrize("rows,d,cols,stride,bias", [
    (256, 512, 8, 8, False),       # config 1 (16 x 16 workgroup tile: few 32 x 32 workgroups)
    (128, 2048, 128, 128, False),   # config 2, decode (16 x 16 tile)
    (2048, 2048, 128, 128, False),  # config 3 (32 x 32 tile)
    (2048, 2048, 128, 130, True),   # config 4 (skew bias), padded stride
    (512, 2048, 513, 513, False),   # config 5 row subset: 512 experts + shared gate
    (37, 256, 70, 72, True),        # ragged tile edges
    (37, 2048, 70, 72, True),       # d = 2048 kernel: shifted last token tile, partial column group
    (23, 2048, 513, 513, True),     # d = 2048 kernel, one column in the last group
    (5, 2048, 128, 128, False),     # fewer rows than one token tile
    (37, 384, 70, 72, True),        # 3 sub-tiles of 16 k per chunk: the 4-slot ring's tail step
    (64, 128, 40, 40, False),       # one sub-tile per chunk
    (100, 1152, 33, 33, True),      # 9 sub-tiles per chunk; 33 columns: a second column block of one
])
def test_router_bitexact(ctx, rows, d, cols, stride, bias):
    x = orc.fill_normal_f16(rows * d, configs.STREAM_X, 1, 1.0).reshape(rows, d)
    w = orc.fill_normal_f32(cols * d, configs.STREAM_W_ROUTER, 1, 0.02).reshape(cols, d)
    b = configs.skew_bias(cols, 1) if bias else None
    nbias = cols if bias else 0
    ref = orc.router(x, w, b, nbias=nbias, stride=stride)
    proj = torch.full((rows, stride), 7.0, dtype=torch.float32, device="cuda")
    ctx.router(rows, d, cols, stride, nbias, dev(x), dev(w), None if b is None else dev(b), proj)
    ctx.sync()
    got = proj.cpu().numpy()
    assert np.array_equal(got[:, :cols].view(np.uint32), ref[:, :cols].view(np.uint32))
    assert np.all(got[:, cols:] == 7.0), "columns beyond cols must stay untouched"


@pytest.mark.parametrize("mag,bias", [(1.0, True), (1e-5, False), (1e5, True)])
def test_router_slot_bitexact(ctx, mag, bias):
    """rmda_moe_router_slot on x cast with a slot (absmax + cast on the GPU)
    against the oracle's scaled router with 1/scale, fp32 activations of
    magnitude 1, 1e-5 (below fp16's normal range unscaled) and 1e5 (above
    65504); for fp16-exact activations it equals rmda_moe_router on the
    unscaled cast bit for bit."""
    rows, d, cols = 77, 1024, 40
    x32 = orc.fill_normal_f32(rows * d, configs.STREAM_X, 2, mag).reshape(rows, d)
    w = orc.fill_normal_f32(cols * d, configs.STREAM_W_ROUTER, 2, 0.02).reshape(cols, d)
    b = configs.skew_bias(cols, 2) if bias else None
    nbias = cols if bias else 0
    amax_h = orc.absmax(x32, np.zeros(16, np.uint32), 3)
    xs = orc.cast_f16(x32, amax_h, 3).reshape(rows, d)
    ref = orc.router(xs, w, b, nbias=nbias, post=1.0 / orc.slot_scale(amax_h, 3))
    amax = torch.zeros(16, dtype=torch.int32, device="cuda")
    a16 = torch.empty(rows, d, dtype=torch.float16, device="cuda")
    xd, wd, bd = dev(x32), dev(w), None if b is None else dev(b)
    ctx.absmax(rows * d, 3, xd, amax)
    ctx.cast_f16(rows * d, 3, xd, a16, amax)
    proj = torch.full((rows, cols), 7.0, dtype=torch.float32, device="cuda")
    ctx.router(rows, d, cols, cols, nbias, a16, wd, bd, proj, slot=3, amax=amax)
    ctx.sync()
    assert np.array_equal(u16(a16), xs), "slot-scaled cast"
    assert np.array_equal(proj.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    # fp16-exact activations: the same logits as the unscaled router
    x16 = orc.f2h(x32 / np.float32(mag))
    xe = dev(orc.h2f(x16))
    amax.zero_()
    ctx.absmax(rows * d, 3, xe, amax)
    ctx.cast_f16(rows * d, 3, xe, a16, amax)
    ctx.router(rows, d, cols, cols, nbias, a16, wd, bd, proj, slot=3, amax=amax)
    plain = torch.full((rows, cols), 7.0, dtype=torch.float32, device="cuda")
    ctx.router(rows, d, cols, cols, nbias, dev(x16), wd, bd, plain)
    ctx.sync()
    assert torch.equal(proj.view(torch.int32), plain.view(torch.int32))
    assert np.array_equal(plain.cpu().numpy().view(np.uint32),
                          orc.router(x16.reshape(rows, d), w, b, nbias=nbias).view(np.uint32))


def test_router_special_values_bitexact(ctx):
    """The matrix-core router against fmaf on the values where an MFMA could
    differ from IEEE fused multiply-adds: subnormal products and partial sums
    (tiny activations x tiny weights, subnormal weights), exact cancellation
    to signed zeros, overflow to infinity, and infinities / NaN inputs.
    Non-NaN logits must match bitwise; NaN must appear exactly where the
    oracle has NaN (its payload is not compared)."""
    rows, d, cols = 48, 2048, 40
    r = rng(11)
    x = r.standard_normal((rows, d)).astype(np.float16)
    w = (r.standard_normal((cols, d)) * 0.02).astype(np.float32)
    x[0:8] = (r.standard_normal((8, d)) * 3e-5).astype(np.float16)  # includes fp16 subnormals
    w[0:8] = (r.standard_normal((8, d)) * 1e-34).astype(np.float32)  # tiny x tiny -> subnormal products
    w[8:12] = (r.standard_normal((4, d)) * 1e-39).astype(np.float32)  # subnormal weights
    # cancellation: each chunk's second half repeats the first half negated -> exact zeros, sign per rounding
    L = d // 8
    for c in range(12, 16):
        for q in range(8):
            half = w[c, q * L:q * L + L // 2].copy()
            w[c, q * L + L // 2:(q + 1) * L] = -half
            x[16:24, q * L + L // 2:(q + 1) * L] = x[16:24, q * L:q * L + L // 2]
    x[24:28, :] = np.float16(-0.0)  # all-negative-zero activations
    x[40, 5] = np.float16(np.inf)
    x[41, 7] = np.float16(-np.inf)
    w[20, 5] = 0.0                   # inf * 0 -> NaN in column 20 of row 40
    x[42, :] = np.float16(60000.0)
    w[21, :] = 1e35                  # overflow to +inf
    w[22, :] = -1e35                 # overflow to -inf
    x[43, 9] = np.float16(np.nan)
    ref = orc.router(x.view(np.uint16), w, None, nbias=0, stride=cols)
    proj = torch.full((rows, cols), 7.0, dtype=torch.float32, device="cuda")
    ctx.router(rows, d, cols, cols, 0, dev(x.view(np.uint16)), dev(w), None, proj)
    ctx.sync()
    got = proj.cpu().numpy()
    nan = np.isnan(ref)
    assert nan.any() and np.isinf(ref).any() and (ref == 0).any(), "the planted cases must occur"
    sub = (ref != 0) & (np.abs(ref) < np.finfo(np.float32).tiny)
    assert sub.any(), "some logits must be subnormal"
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


# ---------------------------------------------------------------- route (A1)

def planted_logits(rows, experts, stride, seed):
    r = rng(seed)
    p = r.standard_normal((rows, stride)).astype(np.float32)
    p[:, experts:] = 1e30  # padding columns must never be read
    # exact ties: copy a value to several columns
    for i in range(0, rows, 7):
        cols = r.choice(experts, size=min(4, experts), replace=False)
        p[i, cols] = p[i, cols[0]]
    # NaN / -inf / <= -3e38 are never selectable
    for i in range(3, rows, 11):
        p[i, r.integers(experts)] = np.nan
        p[i, r.integers(experts)] = -np.inf
        p[i, r.integers(experts)] = -3.0e38
        p[i, r.integers(experts)] = -3.3e38
    # +0 / -0 tie
    if rows > 5 and experts > 3:
        p[5, :experts] = -1.0
        p[5, 1] = -0.0
        p[5, 3] = 0.0
    # whole row of equal values: order must be 0, 1, 2, ...
    p[0, :experts] = 0.25
    return p


@pytest.mark.parametrize("rows,experts,topk,stride", [
    (256, 8, 2, 8), (333, 128, 8, 160), (64, 512, 10, 513), (50, 512, 16, 512),
    (40, 16, 16, 16), (77, 100, 1, 100), (9, 64, 3, 64),
])
def test_route_bitexact(ctx, rows, experts, topk, stride):
    p = planted_logits(rows, experts, stride, seed=rows + experts)
    idx_r, wt_r, cnt_r = orc.route(p, experts, topk)
    idx = empty_u32(rows * topk)
    wt = torch.empty(rows * topk, dtype=torch.float32, device="cuda")
    cnt = empty_u32(experts, fill=12345)  # must be overwritten, not added to
    ctx.route(rows, experts, topk, stride, dev(p), idx, wt, cnt)
    ctx.sync()
    assert np.array_equal(u32(idx), idx_r)
    assert np.array_equal(u32(cnt), cnt_r)
    np.testing.assert_allclose(wt.cpu().numpy(), wt_r, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("rows,experts,topk,shift,hot", [
    (9000, 128, 8, 0, 0),   # 72 000 pairs: above the one-workgroup count, counted by the rank kernel
    (5001, 64, 4, 1, 0),    # idx one word past 16-byte alignment: the count kernel's scalar-load variant
    # every token's top-k is mostly experts 0..7 (whole waves add to one counter), one-workgroup count
    (2051, 128, 8, 0, 8),
    (9001, 512, 10, 0, 6),  # the same above the one-workgroup count
])
def test_route_counts_both_paths(ctx, rows, experts, topk, shift, hot):
    p = planted_logits(rows, experts, experts, seed=rows)
    if hot:
        p[:, :hot] += 50.0  # finite rows of planted_logits stay finite; -inf and NaN columns stay unselectable
    idx_r, wt_r, cnt_r = orc.route(p, experts, topk)
    buf = empty_u32(rows * topk + shift)
    idx = buf[shift:]
    assert (idx.data_ptr() % 16 == 0) == (shift == 0)
    wt = torch.empty(rows * topk, dtype=torch.float32, device="cuda")
    cnt = empty_u32(experts, fill=777)
    ctx.route(rows, experts, topk, experts, dev(p), idx, wt, cnt)
    ctx.sync()
    assert np.array_equal(u32(idx), idx_r)
    assert np.array_equal(u32(cnt), cnt_r)
    assert int(u32(cnt).sum()) == rows * topk


def test_route_unselectable_rows(ctx):
    # fewer selectable columns than topk: the remaining picks are RMDA_NONE
    rows, experts, topk = 4, 8, 4
    p = np.full((rows, experts), np.nan, np.float32)
    p[0, 2] = 1.0
    p[1, :] = -np.inf
    p[2, 5] = 3.0
    p[2, 6] = 3.0
    p[3, :] = -3.0e38
    idx_r, wt_r, cnt_r = orc.route(p, experts, topk)
    idx = empty_u32(rows * topk)
    wt = torch.empty(rows * topk, dtype=torch.float32, device="cuda")
    cnt = empty_u32(experts)
    ctx.route(rows, experts, topk, experts, dev(p), idx, wt, cnt)
    ctx.sync()
    assert np.array_equal(u32(idx), idx_r)
    assert np.array_equal(u32(cnt), cnt_r)
    assert u32(idx)[0] == 2 and u32(idx)[1] == NONE
    np.testing.assert_allclose(wt.cpu().numpy(), wt_r, rtol=2e-6, atol=1e-7, equal_nan=True)


# ---------------------------------------------------------------- scan (A2)

@pytest.mark.parametrize("experts,tile", [(8, 128), (128, 128), (128, 1), (512, 128), (512, 16), (300, 7)])
def test_scan_bitexact(ctx, experts, tile):
    r = rng(experts * 31 + tile)
    cnt = r.integers(0, 400, experts).astype(np.uint32)
    cnt[r.choice(experts, experts // 5, replace=False)] = 0  # empty experts
    n_tiles = int((cnt.sum() + experts * (tile - 1)) // tile + 3)
    off_r, tiles_r = orc.scan(cnt, tile, n_tiles)
    off = empty_u32(experts)
    tiles = empty_u32(n_tiles, fill=0x5A5A5A5A)
    ctx.scan(experts, tile, dev(cnt), off, tiles, n_tiles)
    ctx.sync()
    assert np.array_equal(u32(off), off_r)
    assert np.array_equal(u32(tiles), tiles_r)


# ---------------------------------------------------------------- scatter (A3)

@pytest.mark.parametrize("rows,experts,topk,d,mode", [
    (2048, 128, 8, 2048, "route"),   # config-3 sized
    (256, 8, 2, 512, "route"),       # config 1
    (1001, 64, 4, 256, "random"),    # arbitrary idx with repeats and NONE; a ragged last block of tokens
    (4096, 512, 10, 128, "route"),   # several rank blocks, 512 experts
    (777, 32, 3, 128, "unaligned"),  # idx not 16-byte aligned: the one-launch path's scalar-load variant
    (9000, 128, 8, 64, "route"),     # 72 000 pairs: above the one-launch bound, rank then permute
])
def test_scatter_bitexact(ctx, rows, experts, topk, d, mode):
    """Both scatter paths (one launch up to RMDA_SCATTER1_MAX_PAIRS pairs,
    rank + permute above) against the oracle's sequential scatter."""
    r = rng(rows + d)
    if mode == "route":
        p = r.standard_normal((rows, experts)).astype(np.float32)
        idx_r, _, cnt_r = orc.route(p, experts, topk)
    else:
        idx_r = r.integers(0, experts, rows * topk).astype(np.uint32)
        idx_r[r.choice(rows * topk, rows // 3, replace=False)] = NONE
        cnt_r = np.bincount(idx_r[idx_r != NONE], minlength=experts).astype(np.uint32)
    tile = 128
    mrows = int(((rows * topk + experts * (tile - 1)) + tile - 1) // tile * tile)
    off_r, _ = orc.scan(cnt_r, tile, mrows // tile)
    x = orc.fill_normal_f16(rows * d, 1, 5, 1.0).reshape(rows, d)
    xp_r, slot_r, fill_r = orc.scatter(idx_r, off_r, x, topk, mrows)
    ctx.scatter_experts(experts)
    fill = empty_u32(experts, fill=777)
    slot = empty_u32(rows * topk)
    xp = torch.zeros(mrows, d, dtype=torch.float16, device="cuda")
    idx_d = dev(idx_r)
    if mode == "unaligned":
        buf = torch.empty(idx_r.size + 1, dtype=idx_d.dtype, device="cuda")
        buf[1:] = idx_d
        idx_d = buf[1:]
        assert idx_d.data_ptr() % 16 != 0
    ctx.scatter(rows, topk, d // 8, idx_d, dev(off_r), fill, dev(x), xp, slot)
    ctx.sync()
    assert np.array_equal(u32(slot), slot_r)
    assert np.array_equal(u32(fill), fill_r)
    assert np.array_equal(u16(xp), xp_r)
    # the permutation is the stable counting sort of idx
    valid = idx_r != NONE
    order = np.argsort(idx_r[valid], kind="stable")
    pos = np.empty(order.size, np.int64)
    pos[order] = np.arange(order.size)
    e = idx_r[valid].astype(np.int64)
    start = np.concatenate([[0], np.cumsum(cnt_r)])[:-1]
    assert np.array_equal(u32(slot)[valid] - off_r[e], pos - start[e])


def test_scatter_twice_deterministic(ctx):
    rows, experts, topk, d = 3000, 128, 8, 64
    p = rng(3).standard_normal((rows, experts)).astype(np.float32)
    idx_r, _, cnt_r = orc.route(p, experts, topk)
    off_r, _ = orc.scan(cnt_r, 1, 0)
    ctx.scatter_experts(experts)
    outs = []
    for _ in range(2):
        slot = empty_u32(rows * topk)
        fill = empty_u32(experts)
        xp = torch.zeros(rows * topk, d, dtype=torch.float16, device="cuda")
        x = torch.randn(rows, d, device="cuda", generator=torch.Generator("cuda").manual_seed(1)).half()
        ctx.scatter(rows, topk, d // 8, dev(idx_r), dev(off_r), fill, x, xp, slot)
        ctx.sync()
        outs.append((u32(slot), u16(xp)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


# ---------------------------------------------------------------- grouped GEMM (A4/A7, drop-in)

@pytest.mark.parametrize("m,n,k,E,scaled", [(512, 256, 512, 3, False), (640, 1536, 2048, 5, True),
                                           # 600 row tiles: the valid-tile list is compacted in two passes
                                           (76800, 256, 64, 7, False),
                                           (4096, 512, 768, 9, True),
                                           # n % 256 != 0, k % 64 != 0: the register-staged kernel
                                           (256, 128, 32, 2, False)])
def test_moe_mm_vs_oracle(ctx, m, n, k, E, scaled):
    r = rng(m + n + k)
    ntile = m // 128
    tiles = r.integers(0, E, ntile).astype(np.uint32)
    tiles[r.choice(ntile, max(1, ntile // 4), replace=False)] = NONE
    a = orc.fill_normal_f16(m * k, 11, m, 1.0).reshape(m, k)
    b = orc.fill_normal_f16(E * n * k, 12, n, 0.02).reshape(E, n, k)
    amax = np.zeros(4, np.uint32)
    sa = sb = 0xFFFFFFFF
    if scaled:
        amax[1] = np.float32(3.7).view(np.uint32)
        amax[2] = np.float32(0.0).view(np.uint32)  # zero amax -> scale 1
        sa, sb = 1, 2
    ref = orc.moe_mm(a, b, tiles, n, k, sa=sa, sb=sb, amax=amax, c_init=np.full((m, n), 1e30, np.float32))
    c = torch.full((m, n), 1e30, dtype=torch.float32, device="cuda")
    ctx.mm(m, n, k, sa, sb, dev(a), dev(b), c, dev(amax), dev(tiles))
    ctx.sync()
    got = c.cpu().numpy()
    skip = np.repeat(tiles == NONE, 128)
    assert np.all(got[skip] == 1e30), "rows of unused tiles must stay untouched"
    live = ~skip
    err = np.abs(got[live] - ref[live]).max()
    assert err <= 1e-5 * max(1.0, np.abs(ref[live]).max()), err


@pytest.mark.parametrize("n,k", [(1536, 2048), (2048, 768)], ids=["gate_up", "down"])
def test_moe_mm_vs_oracle_bench_size(ctx, n, k):
    """rmda_moe_mm at the size bench.py times it: config 3's tile map (128
    experts over mrows = 32 640, i.e. 255 tiles of 128 rows, from a scan of
    16 384 pairs) and its K.  The GPU runs every tile; the oracle computes
    every fifth used tile (the rest marked unused in its copy of the map),
    whose rows are compared; unused tiles stay untouched."""
    E, T, K = 128, 2048, 8
    r = rng(n + k)
    count = np.bincount(r.integers(0, E, T * K), minlength=E).astype(np.uint32)
    mrows = (T * K + E * 127 + 127) // 128 * 128
    ntile = mrows // 128
    assert ntile == 255
    _, tiles = orc.scan(count, 128, ntile)
    used = np.flatnonzero(tiles != NONE)
    check = used[::5]
    tiles_ref = np.full(ntile, NONE, np.uint32)
    tiles_ref[check] = tiles[check]
    a = orc.fill_normal_f16(mrows * k, 11, 5, 1.0).reshape(mrows, k)
    b = orc.fill_normal_f16(E * n * k, 12, 6, 0.02).reshape(E, n, k)
    amax = np.zeros(4, np.uint32)
    amax[0] = np.float32(4.1).view(np.uint32)
    ref = orc.moe_mm(a, b, tiles_ref, n, k, sa=0, amax=amax, threads=16)
    c = torch.full((mrows, n), 1e30, dtype=torch.float32, device="cuda")
    ctx.mm(mrows, n, k, 0, 0xFFFFFFFF, dev(a), dev(b), c, dev(amax), dev(tiles))
    ctx.sync()
    got = c.cpu().numpy()
    skip = np.repeat(tiles == NONE, 128)
    assert np.all(got[skip] == 1e30), "rows of unused tiles must stay untouched"
    rows = np.repeat(tiles_ref != NONE, 128)
    err = np.abs(got[rows] - ref[rows]).max()
    print("  %d used tiles, %d compared; max-abs %.3g" % (used.size, check.size, err), flush=True)
    assert err <= 1e-5 * max(1.0, np.abs(ref[rows]).max()), err


# ---------------------------------------------------------------- combine (A9) and helpers

@pytest.mark.parametrize("d", [256, 2048, 258])  # 258: d % 4 != 0 takes the per-element kernel
@pytest.mark.parametrize("shared,hc", [(False, 4), (True, 4), (True, 0)])
def test_combine_vs_oracle(ctx, shared, hc, d):
    r = rng(17)
    rows, topk, E = 300, 8, 64
    nrows = rows * topk + 50
    p = r.standard_normal((rows, E + 3)).astype(np.float32)
    idx, wt, cnt = orc.route(p, E, topk)
    slot = r.permutation(nrows)[: rows * topk].astype(np.uint32)
    slot[5] = NONE
    y = r.standard_normal((nrows, d)).astype(np.float32)
    sh = r.standard_normal((rows, d)).astype(np.float32) if shared else None
    inj = r.standard_normal((rows, 10)).astype(np.float32)
    fields = (rows, d, topk, E + 3, E, 10, 3, hc)
    if hc:
        h0 = r.standard_normal((rows, hc, d)).astype(np.float32)
        ref = orc.combine(fields, wt, slot, y, p, sh, inj, h0)
        h = dev(h0)
        ctx.combine(fields, dev(wt), dev(slot), dev(y), dev(p), None if sh is None else dev(sh), dev(inj), h)
        ctx.sync()
        np.testing.assert_allclose(h.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    else:
        ref = orc.combine_plain(fields, wt, slot, y, p, sh)
        out = torch.empty(rows, d, dtype=torch.float16, device="cuda")
        ctx.combine_plain(fields, dev(wt), dev(slot), dev(y), dev(p), None if sh is None else dev(sh), out)
        ctx.sync()
        np.testing.assert_allclose(f32(out), orc.h2f(orc.f2h(ref)), rtol=0, atol=2e-3)


def test_elem_absmax_cast_bf16(ctx):
    r = rng(23)
    rows, n = 97, 640
    a = (r.standard_normal((rows, 2 * n + 5)) * 3).astype(np.float32)
    for op, scale in [(0, 1.0), (1, 0.5)]:
        ref = orc.qwen_elem(a, rows, n, 2 * n + 5, 2, n + 3, op, scale)
        y = torch.empty(rows * n, dtype=torch.float32, device="cuda")
        ctx.qwen_elem(rows, n, 2 * n + 5, 2, n + 3, op, scale, dev(a), y)
        ctx.sync()
        np.testing.assert_allclose(y.cpu().numpy(), ref, rtol=2e-6, atol=1e-6)
    x = (r.standard_normal(100000) * 5).astype(np.float32)
    amax0 = np.array([0, np.float32(1.0).view(np.uint32), 0], np.uint32)
    ref_amax = orc.absmax(x, amax0, 2)
    amax = dev(amax0)
    ctx.absmax(x.size, 2, dev(x), amax)
    ctx.sync()
    assert np.array_equal(u32(amax), ref_amax)
    for slot in [2, 0xFFFFFFFF]:
        ref16 = orc.cast_f16(x, ref_amax, slot)
        dst = torch.empty(x.size, dtype=torch.float16, device="cuda")
        ctx.cast_f16(x.size, slot, dev(x), dst, dev(ref_amax))
        ctx.sync()
        assert np.array_equal(u16(dst), ref16)
    w = r.integers(0, 2 ** 32, 5000, dtype=np.uint64).astype(np.uint32)
    w &= ~np.uint32(0x7F807F80)  # keep exponents small enough for fp16 range tests...
    w |= np.uint32(0x3C003C00)   # ...and in the normal fp16 range
    refw = orc.qwen_bf16(w)
    wd = dev(w)
    ctx.qwen_bf16(w.size, wd)
    ctx.sync()
    assert np.array_equal(u32(wd), refw)


def test_elem_absmax_cast_both_paths(ctx):
    """Rows of whole float4s (n, astride, ao, bo multiples of 4, aligned
    buffers) take the 16-byte kernels, others the per-element ones: both
    against the oracle, bitwise for absmax and the cast."""
    r = rng(29)
    rows, n = 131, 768
    a = (r.standard_normal((rows, 2 * n)) * 3).astype(np.float32)
    for op, scale in [(0, 1.0), (1, 0.5)]:
        ref = orc.qwen_elem(a, rows, n, 2 * n, 0, n, op, scale)
        y = torch.empty(rows * n, dtype=torch.float32, device="cuda")
        ctx.qwen_elem(rows, n, 2 * n, 0, n, op, scale, dev(a), y)
        ctx.sync()
        np.testing.assert_allclose(y.cpu().numpy(), ref, rtol=2e-6, atol=1e-6)
    x = (r.standard_normal(100003) * 5).astype(np.float32)
    x[77] = 1e4  # the maximum, in the scalar tail of neither path
    for m in (100000, 100003, 99999):
        xs = np.ascontiguousarray(x[:m])
        amax0 = np.array([0, np.float32(1.0).view(np.uint32), 0], np.uint32)
        ref_amax = orc.absmax(xs, amax0, 2)
        amax = dev(amax0)
        ctx.absmax(m, 2, dev(xs), amax)
        ctx.sync()
        assert np.array_equal(u32(amax), ref_amax), m
        ref16 = orc.cast_f16(xs, ref_amax, 2)
        dst = torch.empty(m, dtype=torch.float16, device="cuda")
        ctx.cast_f16(m, 2, dev(xs), dst, dev(ref_amax))
        ctx.sync()
        assert np.array_equal(u16(dst), ref16), m


def test_qwen_bf16_every_bit_pattern(ctx):
    """qwen_bf16 over all 65536 bf16 values in both halves of the word:
    overflow to inf, fp16 subnormals, values that flush to zero, both zeros,
    infinities and NaNs.  Every non-NaN result is bitwise the oracle's; a NaN
    stays a NaN of the same sign."""
    lo = np.arange(65536, dtype=np.uint32)
    hi = rng(29).permutation(lo)
    w = (hi << np.uint32(16)) | lo
    refw = orc.qwen_bf16(w)
    wd = dev(w)
    ctx.qwen_bf16(w.size, wd)
    ctx.sync()
    got = u32(wd)
    for shift in (0, 16):
        g = ((got >> np.uint32(shift)) & np.uint32(0xFFFF)).astype(np.uint16)
        e = ((refw >> np.uint32(shift)) & np.uint32(0xFFFF)).astype(np.uint16)
        nan = ((e & 0x7C00) == 0x7C00) & ((e & 0x03FF) != 0)
        assert np.array_equal(g[~nan], e[~nan]), "non-NaN bf16 -> fp16 differs"
        gnan = ((g & 0x7C00) == 0x7C00) & ((g & 0x03FF) != 0)
        assert gnan[nan].all() and np.array_equal(g[nan] >> 15, e[nan] >> 15), "NaN not kept"
        print("  half %d: %d NaN payloads equal of %d" % (shift // 16, int((g[nan] == e[nan]).sum()), int(nan.sum())))


# ---------------------------------------------------------------- error behaviour

def test_errors_are_sticky_and_reported(ctx):
    c = api.Context(0)
    idx = empty_u32(8)
    wt = torch.empty(8, dtype=torch.float32, device="cuda")
    cnt = empty_u32(600)
    p = torch.zeros(4, 600, device="cuda")
    with pytest.raises(api.MoeError) as e:
        c.route(4, 600, 2, 600, p, idx, wt, cnt)  # experts > 512
    assert e.value.code == -2
    with pytest.raises(api.MoeError) as e:
        c.route(4, 8, 2, 8, p, idx, wt, cnt)  # valid call after a failure: sticky
    assert e.value.code == -5
    c.clear_error()
    c.route(4, 8, 2, 600, p, idx, wt, cnt)
    c.sync()
    with pytest.raises(api.MoeError) as e:
        c.mm(100, 128, 32, 0xFFFFFFFF, 0xFFFFFFFF, p, p, p, None, idx)  # m % 128 != 0
    assert e.value.code == -2
    c.close()


def test_misaligned_pointers(ctx):
    """Entry points whose kernels need 16-byte rows reject other alignments
    with RMDA_ERR_ARG (-1) and enqueue nothing; the drop-in combine falls
    back to its per-element kernel and gives the same bits."""
    c = api.Context(0)
    raw = torch.zeros(4096 + 8, dtype=torch.float16, device="cuda")
    with pytest.raises(api.MoeError) as e:
        c.scatter_experts(8)
        c.scatter(4, 2, 8, empty_u32(8), empty_u32(8), empty_u32(8), raw[1:513], raw[1:], empty_u32(8))
    assert e.value.code == -1
    c.clear_error()
    with pytest.raises(api.MoeError) as e:
        c.mm(128, 128, 32, 0xFFFFFFFF, 0xFFFFFFFF, raw[1:], raw[1:], torch.zeros(128 * 128 + 4, device="cuda")[1:],
             None, empty_u32(1))
    assert e.value.code == -1
    c.clear_error()
    c.close()
    # combine: fp32 expert rows one float past 16-byte alignment take the
    # per-element kernel; the output is checked against the oracle either way
    r = rng(11)
    rows, d, topk, E = 33, 256, 4, 16
    p = r.standard_normal((rows, E)).astype(np.float32)
    _, wt, _ = orc.route(p, E, topk)
    slot = r.permutation(rows * topk).astype(np.uint32)
    y = r.standard_normal((rows * topk, d)).astype(np.float32)
    fields = (rows, d, topk, E, E, 8, 0, 0)
    ref = orc.combine_plain(fields, wt, slot, y, p, None)
    ybuf = torch.empty(rows * topk * d + 1, dtype=torch.float32, device="cuda")
    for shift in (0, 1):
        yd = ybuf[shift:shift + rows * topk * d]
        yd.copy_(torch.from_numpy(y.reshape(-1)))
        assert (yd.data_ptr() % 16 == 0) == (shift == 0)
        out = torch.empty(rows, d, dtype=torch.float16, device="cuda")
        ctx.combine_plain(fields, dev(wt), dev(slot), yd, dev(p), None, out)
        ctx.sync()
        np.testing.assert_allclose(f32(out), orc.h2f(orc.f2h(ref)), rtol=0, atol=2e-3)
