"""CPU suite: pins the CPU oracle (oracle/moe_oracle.c) without a GPU.

Every oracle function is checked against something other than itself:
  - the reference's own counter hash (src/hash.c) through the committed known
    answers in tests/golden/ref_hash.json (and the live build in oracle/_ref
    when the reference tree is present);
  - closed forms, brute force and textbook routines in numpy (stable sorts,
    cumulative sums, float64 GEMMs, numpy's IEEE fp16 conversion);
  - special cases that reduce to a known answer (k=1 is argmax, k=E a full
    stable sort, padding 1 a plain exclusive scan, identity weights exact).
Planted mistakes (a dropped term, a wrong index, a transposed operand) fail
at least one of them.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as orc
from rmda_moe import configs

HERE = os.path.dirname(os.path.abspath(__file__))
NONE = 0xFFFFFFFF


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- fp16 conversion

def test_h2f_exhaustive_matches_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.h2f(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f2h_matches_numpy_rne():
    r = rng(1)
    # every fp16 boundary region: exact halves, midpoints, +-1 ulp of fp32,
    # subnormals, overflow threshold, zeros, infinities
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    nxt = np.append(f[1:], np.float32(65520.0))
    mid = ((f.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    cases = [f, mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0)),
             r.standard_normal(200000).astype(np.float32) * np.float32(1e3),
             r.standard_normal(200000).astype(np.float32) * np.float32(1e-6),
             np.array([0.0, 65504.0, 65519.99, 65520.0, 1e6, np.inf, 2.0 ** -25, 2.0 ** -24 * 1.5,
                       2.0 ** -26], np.float32)]
    x = np.concatenate(cases)
    x = np.concatenate([x, -x])
    got = orc.f2h(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    # NaN stays NaN
    assert np.isnan(orc.f2h(np.array([np.nan], np.float32)).view(np.float16)[0])


# ---------------------------------------------------------------- counter hash (reference KATs)

def test_hash_matches_reference_known_answers():
    kat = json.load(open(os.path.join(HERE, "golden", "ref_hash.json")))
    for s, k, i, h in kat["u64"]:
        assert orc.hash_u64(s, k, i) == h
        assert configs.hash_u64(s, k, i) == h
    assert len(kat["u64"]) >= 300 and len(kat["mix"]) >= 8


def test_hash_matches_live_reference_build():
    ref = orc.ref_hash_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference tree absent on this host)")
    r = rng(2)
    for s, k, i in r.integers(0, 2 ** 63, (200, 3), dtype=np.uint64).tolist():
        assert orc.hash_u64(s, k, i) == ref.mda_hash_u64(s, k, i)


def test_normal_generator_properties():
    n = 1 << 20
    z = orc.fill_normal_f32(n, 9, 0, 1.0).astype(np.float64)
    # standardised Irwin-Hall(4): mean 0, variance 1, support +-2*sqrt(3),
    # excess kurtosis -6/(5*4) = -0.3
    assert abs(z.mean()) < 5e-3
    assert abs(z.var() - 1.0) < 5e-3
    assert np.abs(z).max() <= 2 * np.sqrt(3) + 1e-6
    kurt = ((z - z.mean()) ** 4).mean() / z.var() ** 2 - 3.0
    assert abs(kurt + 0.3) < 0.02
    # the value at index i depends only on (stream, seed, i)
    a = orc.fill_normal_f32(1000, 9, 0, 1.0)
    assert np.array_equal(a, z[:1000].astype(np.float32))
    b = orc.fill_normal_f32(1000, 9, 1, 1.0)
    assert not np.array_equal(a, b)
    # fp16 fill is the RNE fp16 of the fp32 fill; std scales exactly
    h = orc.fill_normal_f16(1000, 9, 0, 0.02)
    assert np.array_equal(h, (a * np.float32(0.02)).astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------- router projection (A0)

@pytest.mark.parametrize("rows,d,cols,bias", [(33, 256, 8, False), (64, 2048, 129, True), (5, 128, 1, True)])
def test_router_matches_float64(rows, d, cols, bias):
    x = orc.fill_normal_f16(rows * d, 1, 3, 1.0).reshape(rows, d)
    w = orc.fill_normal_f32(cols * d, 2, 3, 0.02).reshape(cols, d)
    b = configs.skew_bias(cols, 3) if bias else None
    got = orc.router(x, w, b, stride=cols + 3)
    xf = x.view(np.float16).astype(np.float64)
    ref = xf @ w.astype(np.float64).T
    if b is not None:
        ref += b
    bound = 2e-6 * (np.abs(xf) @ np.abs(w.astype(np.float64)).T) + 1e-6 * (np.abs(b) if b is not None else 0)
    assert np.all(np.abs(got[:, :cols] - ref) <= bound + 1e-12)
    assert np.all(got[:, cols:] == 0)
    # a transposed operand or a dropped chunk is far outside the bound
    assert not np.allclose(got[:, :cols], ref - xf[:, : d // 8] @ w[:, : d // 8].T.astype(np.float64),
                           atol=1e-6)


def test_router_thread_count_does_not_change_bits():
    x = orc.fill_normal_f16(97 * 512, 1, 4, 1.0).reshape(97, 512)
    w = orc.fill_normal_f32(40 * 512, 2, 4, 0.02).reshape(40, 512)
    a = orc.router(x, w, threads=1)
    b = orc.router(x, w, threads=7)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_router_scaled_equals_unscaled_for_fp16_inputs():
    """orc_router_scaled on x cast with a power-of-two slot scale, with
    1/scale as `post`: scaling every product of a chain by a power of two
    commutes with fp32 rounding (no subnormal or overflow here), so the logits
    equal the unscaled router's bit for bit; a post that is not the inverse,
    or one applied to the bias as well, is not."""
    x = orc.fill_normal_f16(61 * 768, 1, 5, 1.0).reshape(61, 768)
    w = orc.fill_normal_f32(24 * 768, 2, 5, 0.02).reshape(24, 768)
    b = configs.skew_bias(24, 5)
    xf = orc.h2f(x)
    amax = orc.absmax(xf, np.zeros(16, np.uint32), 0)
    xs = orc.cast_f16(xf, amax, 0).reshape(x.shape)
    sc = orc.slot_scale(amax, 0)
    assert sc != 1.0 and not np.array_equal(xs, x)
    want = orc.router(x, w, b)
    got = orc.router(xs, w, b, post=1.0 / sc)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert not np.array_equal(orc.router(xs, w, b, post=2.0 / sc).view(np.uint32), want.view(np.uint32))
    assert not np.allclose(orc.router(xs, w, b * np.float32(sc), post=1.0 / sc), want, rtol=1e-3)


# ---------------------------------------------------------------- route (A1)

def np_route(p, experts, topk):
    """Brute force: stable sort by (value descending, index ascending) over
    the selectable columns (not NaN, > -3e38), softmax renormalised over the
    picks in float64."""
    rows = p.shape[0]
    idx = np.full((rows, topk), NONE, np.uint32)
    sv = np.full((rows, topk), -3.0e38, np.float64)
    for r in range(rows):
        v = p[r, :experts]
        cols = np.nonzero(~np.isnan(v) & (v > np.float32(-3.0e38)))[0]
        order = cols[np.lexsort((cols, -v[cols].astype(np.float64)))][:topk]
        idx[r, : order.size] = order
        sv[r, : order.size] = v[order]
    sv = np.where(idx == NONE, np.float64(np.float32(-3.0e38)), sv)
    e = np.exp(sv - sv[:, :1])
    wt = e / e.sum(axis=1, keepdims=True)
    sel = idx[idx != NONE]
    count = np.bincount(sel, minlength=experts).astype(np.uint32)
    return idx.reshape(-1), wt.reshape(-1), count


def planted(rows, experts, stride, seed):
    r = rng(seed)
    p = r.standard_normal((rows, stride)).astype(np.float32)
    p[:, experts:] = 1e30  # columns beyond experts must never be read
    for i in range(0, rows, 5):
        cols = r.choice(experts, size=min(5, experts), replace=False)
        p[i, cols] = p[i, cols[0]]
    for i in range(2, rows, 9):
        p[i, r.integers(experts)] = np.nan
        p[i, r.integers(experts)] = -np.inf
        p[i, r.integers(experts)] = -3.0e38
    p[0, :experts] = 0.5
    if experts > 3 and rows > 1:
        p[1, :experts] = -2.0
        p[1, 3] = 0.0
        p[1, 1] = -0.0
    return p


@pytest.mark.parametrize("rows,experts,topk,stride", [(60, 8, 2, 8), (50, 128, 8, 140), (20, 512, 10, 513),
                                                      (30, 16, 16, 16), (25, 64, 1, 64)])
def test_route_matches_brute_force(rows, experts, topk, stride):
    p = planted(rows, experts, stride, seed=experts + topk)
    idx, wt, cnt = orc.route(p, experts, topk)
    idx_r, wt_r, cnt_r = np_route(p, experts, topk)
    assert np.array_equal(idx, idx_r)
    assert np.array_equal(cnt, cnt_r)
    np.testing.assert_allclose(wt, wt_r, rtol=2e-6, atol=1e-9)
    assert cnt.sum() == (idx != NONE).sum()
    full = (idx.reshape(rows, topk) != NONE).all(axis=1)
    np.testing.assert_allclose(wt.reshape(rows, topk)[full].sum(axis=1), 1.0, rtol=0, atol=topk * 1.2e-7)


def test_route_special_cases():
    r = rng(7)
    p = r.standard_normal((40, 32)).astype(np.float32)
    idx, _, _ = orc.route(p, 32, 1)
    assert np.array_equal(idx, np.argmax(p, axis=1).astype(np.uint32))  # k=1: argmax
    idx, wt, _ = orc.route(p, 32, 16)
    full = orc.route(p[:, :16], 16, 16)[0].reshape(40, 16)
    assert np.array_equal(np.sort(full, axis=1), np.tile(np.arange(16, dtype=np.uint32), (40, 1)))
    order = np.argsort(-p, axis=1, kind="stable")[:, :16].astype(np.uint32)
    assert np.array_equal(idx.reshape(40, 16), order)  # k=E-prefix of a full stable sort
    # all-equal row: 0, 1, 2, ...; weights uniform
    q = np.full((1, 8), 3.0, np.float32)
    idx, wt, _ = orc.route(q, 8, 4)
    assert list(idx) == [0, 1, 2, 3]
    np.testing.assert_allclose(wt, 0.25, rtol=0, atol=1e-7)
    # nothing selectable: NONE, not counted
    q = np.full((1, 8), np.nan, np.float32)
    q[0, 6] = 1.0
    idx, wt, cnt = orc.route(q, 8, 3)
    assert list(idx) == [6, NONE, NONE]
    assert cnt.sum() == 1 and wt[0] == 1.0


# ---------------------------------------------------------------- scan (A2)

@pytest.mark.parametrize("experts,tile", [(8, 128), (128, 128), (512, 1), (300, 7)])
def test_scan_closed_form(experts, tile):
    r = rng(experts + tile)
    cnt = r.integers(0, 500, experts).astype(np.uint32)
    cnt[r.choice(experts, experts // 4, replace=False)] = 0
    width = (cnt.astype(np.int64) + tile - 1) // tile * tile
    n_tiles = int(width.sum() // tile + 2)
    off, tiles = orc.scan(cnt, tile, n_tiles)
    assert np.array_equal(off, (np.cumsum(width) - width).astype(np.uint32))
    owner = np.repeat(np.arange(experts, dtype=np.uint32), width // tile)
    assert np.array_equal(tiles[: owner.size], owner)
    assert np.all(tiles[owner.size:] == NONE)
    if tile == 1:
        assert np.array_equal(off, np.concatenate([[0], np.cumsum(cnt)[:-1]]).astype(np.uint32))


# ---------------------------------------------------------------- scatter (A3)

def test_scatter_is_stable_counting_sort():
    r = rng(11)
    rows, experts, topk, d = 300, 16, 4, 64
    p = r.standard_normal((rows, experts)).astype(np.float32)
    idx, _, cnt = orc.route(p, experts, topk)
    idx = idx.copy()
    idx[r.choice(idx.size, 20, replace=False)] = NONE
    cnt = np.bincount(idx[idx != NONE], minlength=experts).astype(np.uint32)
    off, _ = orc.scan(cnt, 128, 0)
    x = orc.fill_normal_f16(rows * d, 1, 11, 1.0).reshape(rows, d)
    mrows = int(off[-1] + (cnt[-1] + 127) // 128 * 128)
    xp, slot, fill = orc.scatter(idx, off, x, topk, mrows)
    assert np.array_equal(fill, cnt)
    valid = idx != NONE
    assert np.all(slot[~valid] == NONE)
    pr = np.nonzero(valid)[0]
    e = idx[pr].astype(np.int64)
    order = np.lexsort((pr, e))           # stable by expert, then by pair index
    rank = np.empty(pr.size, np.int64)
    start = np.concatenate([[0], np.cumsum(np.bincount(e, minlength=experts))[:-1]])
    rank[order] = np.arange(pr.size) - start[e[order]]
    assert np.array_equal(slot[pr], (off[e] + rank).astype(np.uint32))
    assert np.array_equal(xp[slot[pr]], x[pr // topk])  # bitwise row copies
    untouched = np.ones(mrows, bool)
    untouched[slot[pr]] = False
    assert np.all(xp[untouched] == 0)


# ---------------------------------------------------------------- grouped GEMM (A4/A7)

def test_moe_mm_matches_float64_per_expert():
    r = rng(13)
    m, n, k, E = 512, 256, 256, 3
    tiles = np.array([2, NONE, 0, 1], np.uint32)
    a = orc.fill_normal_f16(m * k, 11, 1, 1.0).reshape(m, k)
    b = orc.fill_normal_f16(E * n * k, 12, 1, 0.02).reshape(E, n, k)
    amax = np.array([0, np.float32(3.7).view(np.uint32), np.float32(0.2).view(np.uint32)], np.uint32)
    got = orc.moe_mm(a, b, tiles, n, k, sa=1, sb=2, amax=amax, c_init=np.full((m, n), 7.0, np.float32))
    s = orc.slot_scale(amax, 1) * orc.slot_scale(amax, 2)
    assert s == 2.0 ** 13 * 2.0 ** 17  # 3.7: 2^(141-128); 0.2: 2^(141-124)
    af = a.view(np.float16).astype(np.float64)
    bf = b.view(np.float16).astype(np.float64)
    for t, e in enumerate(tiles):
        rs = slice(128 * t, 128 * (t + 1))
        if e == NONE:
            assert np.all(got[rs] == 7.0)
            continue
        ref = af[rs] @ bf[e].T / s
        bound = 2e-6 * (np.abs(af[rs]) @ np.abs(bf[e]).T) / s
        assert np.all(np.abs(got[rs] - ref) <= bound + 1e-30)
    del r


def test_moe_mm_identity_weights_exact():
    m, k = 256, 128
    a = orc.fill_normal_f16(m * k, 11, 2, 1.0).reshape(m, k)
    eye = np.eye(k, dtype=np.float32).astype(np.float16).view(np.uint16).reshape(1, k, k)
    got = orc.moe_mm(a, eye, np.array([0, 0], np.uint32), k, k)
    assert np.array_equal(got, a.view(np.float16).astype(np.float32))


def test_slot_scale_closed_form():
    for v in [1.0, 3.7, 0.2, 65504.0, 1e-20, 1e30]:
        bits = np.float32(v).view(np.uint32)
        assert orc.slot_scale(np.array([bits], np.uint32), 0) == 2.0 ** (141 - ((int(bits) >> 23) & 0xFF))
    for v in [0.0, np.inf, np.nan]:
        assert orc.slot_scale(np.array([np.float32(v).view(np.uint32)], np.uint32), 0) == 1.0
    assert orc.slot_scale(None, 0xFFFFFFFF) == 1.0


# ---------------------------------------------------------------- combine (A9)

@pytest.mark.parametrize("shared,hc", [(False, 4), (True, 4), (True, 0), (False, 0)])
def test_combine_closed_form(shared, hc):
    r = rng(17 + hc)
    rows, d, topk, E = 40, 64, 4, 16
    nrows = rows * topk + 10
    p = r.standard_normal((rows, E + 3)).astype(np.float32)
    _, wt, _ = orc.route(p, E, topk)
    slot = r.permutation(nrows)[: rows * topk].astype(np.uint32)
    slot[3] = NONE
    y = r.standard_normal((nrows, d)).astype(np.float32)
    sh = r.standard_normal((rows, d)).astype(np.float32) if shared else None
    inj = r.standard_normal((rows, 10)).astype(np.float32)
    fields = (rows, d, topk, E + 3, E, 10, 3, hc)
    w64 = np.where(slot == NONE, 0.0, wt.astype(np.float64)).reshape(rows, topk)
    ysel = y.astype(np.float64)[np.where(slot == NONE, 0, slot).reshape(rows, topk)]
    acc = (w64[:, :, None] * ysel).sum(axis=1)
    if shared:
        acc += (1 / (1 + np.exp(-p[:, E].astype(np.float64))))[:, None] * sh
    if hc:
        h0 = r.standard_normal((rows, hc, d)).astype(np.float32)
        got = orc.combine(fields, wt, slot, y, p, sh, inj, h0)
        g = 1 / (1 + np.exp(-inj[:, 3:3 + hc].astype(np.float64) / hc))
        ref = h0 + acc[:, None, :] * 2 * g[:, :, None]
        np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)
    else:
        got = orc.combine_plain(fields, wt, slot, y, p, sh)
        np.testing.assert_allclose(got, acc, rtol=2e-6, atol=2e-6)


# ---------------------------------------------------------------- helpers

def test_elem_absmax_cast_bf16_closed_forms():
    r = rng(23)
    rows, n = 30, 96
    a = (r.standard_normal((rows, 2 * n + 5)) * 4).astype(np.float32)
    g = a[:, 2:2 + n].astype(np.float64)
    u = a[:, n + 3:2 * n + 3].astype(np.float64)
    got = orc.qwen_elem(a, rows, n, 2 * n + 5, 2, n + 3, 0).reshape(rows, n)
    np.testing.assert_allclose(got, g / (1 + np.exp(-g)) * u, rtol=2e-6, atol=1e-7)
    got = orc.qwen_elem(a, rows, n, 2 * n + 5, 2, n + 3, 1, 0.5).reshape(rows, n)
    np.testing.assert_allclose(got, g * 0.5 / (1 + np.exp(-g * 0.5)), rtol=2e-6, atol=1e-7)

    x = (r.standard_normal(5000) * 7).astype(np.float32)
    amax = orc.absmax(x, np.array([0, np.float32(100.0).view(np.uint32)], np.uint32), 0)
    assert amax[0] == np.abs(x).max().view(np.uint32)
    assert orc.absmax(x, np.array([0, np.float32(100.0).view(np.uint32)], np.uint32), 1)[1] == \
        np.float32(100.0).view(np.uint32)
    s = orc.slot_scale(amax, 0)
    assert np.array_equal(orc.cast_f16(x, amax, 0), (x * np.float32(s)).astype(np.float16).view(np.uint16))
    assert np.array_equal(orc.cast_f16(x, None, 0xFFFFFFFF), x.astype(np.float16).view(np.uint16))
    # the scaled cast puts the largest |x| in [16384, 32768)
    top = np.abs(orc.h2f(orc.cast_f16(x, amax, 0))).max()
    assert 16384 <= top < 32768

    w = r.integers(0, 2 ** 32, 4000, dtype=np.uint64).astype(np.uint32)
    got = orc.qwen_bf16(w)
    lo = (w << np.uint32(16)).view(np.float32).astype(np.float16).view(np.uint16).astype(np.uint32)
    hi = (w & np.uint32(0xFFFF0000)).view(np.float32).astype(np.float16).view(np.uint16).astype(np.uint32)
    ref = lo | (hi << np.uint32(16))
    nan = np.isnan((w << np.uint32(16)).view(np.float32)) | np.isnan((w & np.uint32(0xFFFF0000)).view(np.float32))
    assert np.array_equal(got[~nan], ref[~nan])


# ---------------------------------------------------------------- whole layer

def slot_round(v):
    """numpy restatement of absmax.comp + cast_f16.comp and the consuming
    GEMM's division: v * 2^(141 - biased exponent(max|v|)) rounded to fp16
    (numpy's RNE), then divided by the same power of two, in float64."""
    v32 = np.asarray(v, np.float32)
    amax = np.float32(np.abs(v32).max())
    if not (amax > 0) or not np.isfinite(amax):
        return v32.astype(np.float16).astype(np.float64)
    e = int((amax.view(np.uint32) >> np.uint32(23)) & np.uint32(0xFF))
    sc = np.ldexp(np.float32(1.0), 141 - e).astype(np.float32)
    return (v32 * sc).astype(np.float16).astype(np.float64) / np.float64(sc)


def np_layer(host, res, hp_fp16=True, x64=None, hp_slot=False):
    """float64 restatement of the MoE layer from the oracle's routing (which
    the route tests pin) and the raw weights: each pair's SwiGLU FFN with the
    intermediate rounded to fp16 (with hp_slot: through one slot scale for
    the routed pairs and one for the shared expert, as src/qwen.c:858-886
    does), combined in float64.  x64 replaces the fp16 x."""
    s = host["shape"]
    T, d, E, K, I, S = s["rows"], s["d"], s["experts"], s["topk"], s["inter"], s["shared"]
    x = host["x"].view(np.float16).astype(np.float64) if x64 is None else x64
    wgu = host["w_gate_up"].view(np.float16).astype(np.float64)
    wd = host["w_down"].view(np.float16).astype(np.float64)
    idx = res["idx"].reshape(T, K)
    wt = res["wt"].reshape(T, K).astype(np.float64)
    out = np.zeros((T, d))
    hs = {}
    for e in range(E):
        rr, jj = np.nonzero(idx == e)
        if rr.size == 0:
            continue
        g = x[rr] @ wgu[e].T
        hs[e] = (rr, jj, g[:, :I] / (1 + np.exp(-g[:, :I])) * g[:, I:])
    if hp_slot and hs:
        flat = slot_round(np.concatenate([h.astype(np.float32).ravel() for _, _, h in hs.values()]))
        o = 0
        for e, (rr, jj, h) in hs.items():
            hs[e] = (rr, jj, flat[o:o + h.size].reshape(h.shape))
            o += h.size
    for e, (rr, jj, h) in hs.items():
        if hp_fp16 and not hp_slot:
            h = h.astype(np.float16).astype(np.float64)
        np.add.at(out, rr, wt[rr, jj][:, None] * (h @ wd[e].T))
    if S:
        g = x @ host["w_sh_gate_up"].view(np.float16).astype(np.float64).T
        h = g[:, :S] / (1 + np.exp(-g[:, :S])) * g[:, S:]
        h = slot_round(h) if hp_slot else h.astype(np.float16).astype(np.float64)
        gate = 1 / (1 + np.exp(-res["proj"][:, E].astype(np.float64)))
        out += gate[:, None] * (h @ host["w_sh_down"].view(np.float16).astype(np.float64).T)
    return out


def host_inputs(cfg, seed):
    host = {"shape": configs.shape_of(cfg), "bias": None, "w_sh_gate_up": None, "w_sh_down": None}
    for name, shp, dt, stream, std in configs.tensor_specs(cfg):
        f = orc.fill_normal_f16 if dt == "f16" else orc.fill_normal_f32
        host[name] = f(int(np.prod(shp)), stream, seed, std).reshape(shp)
    if cfg.get("skew"):
        host["bias"] = configs.skew_bias(cfg["experts"], seed)
    return host


SMALL = [
    dict(name="small", rows=96, d=256, experts=8, topk=2, inter=128, shared=0, skew=False),
    dict(name="small_shared", rows=64, d=256, experts=16, topk=4, inter=64, shared=64, skew=False),
    dict(name="small_skew", rows=80, d=128, experts=32, topk=3, inter=64, shared=0, skew=True),
]


@pytest.mark.parametrize("cfg", SMALL, ids=lambda c: c["name"])
def test_layer_matches_float64(cfg):
    host = host_inputs(cfg, seed=4)
    res = orc.layer(host, tile=1)
    ref = np_layer(host, res)
    err = np.abs(res["out"] - ref)
    rel = np.linalg.norm(res["out"] - ref) / np.linalg.norm(ref)
    assert err.max() <= 2e-3 and rel <= 1e-3, (err.max(), rel)
    # routing: counts sum to T*k, offsets are the exclusive scan of counts
    T, K = cfg["rows"], cfg["topk"]
    assert res["count"].sum() == T * K
    assert np.array_equal(res["off"], np.concatenate([[0], np.cumsum(res["count"])[:-1]]).astype(np.uint32))
    # dropping the shared gate, or the SwiGLU up half, is caught
    if cfg["shared"]:
        host2 = dict(host)
        host2["w_sh_gate_up"] = np.zeros_like(host["w_sh_gate_up"])
        assert np.abs(orc.layer(host2, tile=1)["out"] - ref).max() > 1e-2


def test_layer_sampled_rows_equal_full_rows():
    cfg = SMALL[1]
    host = host_inputs(cfg, seed=5)
    full = orc.layer(host, tile=1)
    sel = np.array([0, 7, 8, 63], np.uint32)
    part = orc.layer(host, tile=1, rows_sel=sel)
    assert np.array_equal(part["out"], full["out"][sel])
    assert np.array_equal(part["idx"], full["idx"]) and np.array_equal(part["slot"], full["slot"])
    thr = orc.layer(host, tile=1, threads=1)
    assert np.array_equal(thr["out"], full["out"])


def test_layer_padding_and_scale_modes_agree():
    cfg = SMALL[0]
    host = host_inputs(cfg, seed=6)
    a = orc.layer(host, tile=1)
    b = orc.layer(host, tile=128, hp_scale=0, x_scale=0)
    # padding changes offsets only; power-of-two scaling of hp is exact except
    # where unscaled hp falls into fp16's subnormal range (|h| < 2^-14), so the
    # two modes agree to far inside the acceptance tolerance
    assert np.array_equal(a["idx"], b["idx"])
    assert np.abs(a["out"] - b["out"]).max() <= 2e-5
    width = (b["count"].astype(np.int64) + 127) // 128 * 128
    assert np.array_equal(b["off"], (np.cumsum(width) - width).astype(np.uint32))


def test_layer_x32_of_fp16_values_equals_fp16_input():
    """The fp32-activation mode on fp32 copies of fp16 values: the slot cast
    multiplies by a power of two (exact for these values, normal or not),
    the router divides it out before the bias and the GEMMs after the
    product, so logits, routing and output are bitwise those of the fp16
    input in the same (slot-scaled) mode."""
    for cfg in SMALL:
        host = host_inputs(cfg, seed=8)
        a = orc.layer(host, tile=1, x_scale=1, hp_scale=1)
        h32 = dict(host, x32=orc.h2f(host["x"]), x=None)
        b = orc.layer(h32, tile=1, x_scale=1, hp_scale=1)
        for k in ("proj", "idx", "wt", "count", "off", "slot", "out"):
            assert np.array_equal(a[k].view(np.uint32), b[k].view(np.uint32)), (cfg["name"], k)


@pytest.mark.parametrize("mag", [1e-6, 1.0, 1e6], ids=["1e-6", "1", "1e6"])
def test_layer_x32_extreme_magnitudes_match_float64(mag):
    """Activations far outside fp16's range: x32 = mag * N(0, 1) in fp32
    (values not representable in fp16).  The oracle casts x with a slot, and
    hp with a slot, where fp16 without them would flush to zero (1e-6) or
    overflow (1e6, where hp is ~1e12).  Against a float64 layer on the same
    routing whose only fp16 roundings are numpy's slot casts of x and hp:
    relative L2 1e-3 and max-abs 1e-2 of the largest output."""
    cfg = SMALL[1]
    host = host_inputs(cfg, seed=9)
    T, d = cfg["rows"], cfg["d"]
    x32 = (orc.fill_normal_f32(T * d, configs.STREAM_X, 9, 1.0).reshape(T, d) * np.float32(mag)).astype(np.float32)
    h32 = dict(host, x32=x32, x=None)
    res = orc.layer(h32, tile=1, x_scale=1, hp_scale=1)
    assert np.isfinite(res["out"]).all() and np.isfinite(res["proj"]).all()
    # logits: float64 GEMM of the slot-cast x (the cast pinned above), scale divided out
    xs = slot_round(x32)
    w = host["w_router"].astype(np.float64)
    proj64 = xs @ w.T
    bound = 2e-6 * (np.abs(xs) @ np.abs(w).T)
    assert np.all(np.abs(res["proj"] - proj64) <= bound)
    ref = np_layer(h32, res, x64=xs, hp_slot=True)
    err = np.abs(res["out"] - ref).max()
    rel = np.linalg.norm(res["out"] - ref) / np.linalg.norm(ref)
    assert rel <= 1e-3 and err <= 1e-2 * np.abs(ref).max(), (rel, err, np.abs(ref).max())
    assert np.abs(ref).max() > (1e10 if mag > 1 else 0) and np.abs(ref).max() < (1e-8 if mag < 1 else np.inf)
    # a mistake in the scale handling is caught: without hp's slot the fp16
    # intermediate overflows (1e6) or flushes (1e-6)
    if mag != 1.0:
        with np.errstate(all="ignore"):
            bad = np_layer(h32, res, x64=xs, hp_slot=False)
        assert not (np.isfinite(bad).all() and np.linalg.norm(res["out"] - bad) / np.linalg.norm(ref) <= 1e-3)


def test_skew_config_leaves_experts_empty():
    cfg = configs.CONFIGS[4]
    T, d, E = cfg["rows"], cfg["d"], cfg["experts"]
    x = orc.fill_normal_f16(T * d, configs.STREAM_X, 0, 1.0).reshape(T, d)
    w = orc.fill_normal_f32(E * d, configs.STREAM_W_ROUTER, 0, 0.02).reshape(E, d)
    b = configs.skew_bias(E, 0)
    assert sorted(np.round(np.exp(-b / 3.6)).astype(int).tolist()) == list(range(1, E + 1))
    proj = orc.router(x, w, b)
    _, _, cnt = orc.route(proj, E, cfg["topk"])
    assert cnt.sum() == T * cfg["topk"]
    assert (cnt == 0).sum() > 0
    assert np.sort(cnt)[-20:].sum() > 0.5 * cnt.sum()


def test_fp16_ye_error_share():
    """The fused layer keeps the expert output rows (ye) in fp16 where the
    reference keeps fp32 (src/qwen.c:878).  The oracle's ye16 switch rounds
    ye to fp16 and changes nothing else: routing is identical, and at
    BASELINE config 3 (every 8th token) the output moves by a relative L2 of
    about 2e-4, a fifth of the 1e-3 acceptance bound; with the fp16 output
    rounding as well about 3e-4."""
    cfg = configs.CONFIGS[3]
    host = host_inputs(cfg, seed=0)
    sel = np.arange(0, cfg["rows"], 8, dtype=np.uint32)
    a = orc.layer(host, tile=16, rows_sel=sel, threads=8)
    b = orc.layer(host, tile=16, rows_sel=sel, threads=8, ye16=True)
    assert np.array_equal(a["idx"], b["idx"]) and np.array_equal(a["slot"], b["slot"])

    def rel(x, y):
        return np.linalg.norm(x - y) / np.linalg.norm(y)

    r_ye = rel(b["out"], a["out"])
    r_both = rel(orc.h2f(orc.f2h(b["out"])), a["out"])
    assert 5e-5 < r_ye < 4e-4, r_ye
    assert r_ye < r_both < 6e-4, r_both
