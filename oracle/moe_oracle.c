/*
 * moe_oracle.c - CPU oracle and CPU baseline of the MoE feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg, as the checker or the timed CPU baseline.
 * The product library never links it.
 *
 * Each function restates one reference shader (file:line cited at the
 * function).  Arithmetic is fixed-order and single-precision where the
 * reference stores fp32, so a multithreaded run gives the same bits as a
 * single-threaded one (threads only split independent outputs).
 * Build: oracle/Makefile (-ffp-contract=off: every fused multiply-add here is
 * an explicit fmaf).
 */
#include "moe_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------ */
/* fp16 conversion                                                     */
/* ------------------------------------------------------------------ */

static uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float orc_h2f(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in fp32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return u2f(f2u(v) | s);
    } else if (e == 31) {
        return u2f(s | 0x7f800000u | (m << 13) | (m ? 0x400000u : 0u));
    }
    return u2f(s | ((e + 112u) << 23) | (m << 13));
}

uint16_t orc_f2h(float v) {
    uint32_t x = f2u(v);
    uint32_t s = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) {
        return (uint16_t)(s | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) {
        /* >= 65520 (including inf) rounds to infinity */
        return (uint16_t)(s | 0x7c00u);
    }
    if (ax >= 0x38800000u) {
        /* normal fp16 range: rebias the exponent, round 23 -> 10 mantissa bits */
        uint32_t r = ax - 0x38000000u;
        r += 0xfffu + ((r >> 13) & 1u);
        return (uint16_t)(s | (r >> 13));
    }
    uint32_t e = ax >> 23;
    if (e < 102u) {
        /* below half of the smallest subnormal (2^-25): rounds to zero */
        return (uint16_t)s;
    }
    /* fp16 subnormal: round (mant * 2^(e-150)) * 2^24 to an integer, ties to even */
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e;
    uint32_t m = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (m & 1u))) {
        m += 1u;
    }
    return (uint16_t)(s | m);
}

void orc_h2f_n(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i += 1) {
        dst[i] = orc_h2f(src[i]);
    }
}

void orc_f2h_n(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i += 1) {
        dst[i] = orc_f2h(src[i]);
    }
}

/* ------------------------------------------------------------------ */
/* counter hash + generator                                            */
/* ------------------------------------------------------------------ */

/* SplitMix64 finaliser (Steele, Lea, Flood 2014), applied three times to
 * (stream, key, index) as the reference's counter hash does
 * (src/hash.c:5-13). */
static uint64_t orc_mix(uint64_t x) {
    uint64_t a = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    uint64_t b = (a ^ (a >> 27)) * 0x94d049bb133111ebull;
    return b ^ (b >> 31);
}

uint64_t orc_hash_u64(uint64_t stream, uint64_t key, uint64_t i) {
    return orc_mix(orc_mix(orc_mix(stream + 0x9e3779b97f4a7c15ull) ^ key) ^ i);
}

/* Standardised Irwin-Hall(4): the four 16-bit fields of one hash are four
 * uniforms on (0,1) at odd multiples of 2^-17; their sum minus 2 is exact in
 * fp32, times sqrt(3) (unit variance) is one rounding, times std another.
 * No libm, so every IEEE host gives the same bits. */
float orc_normal(uint64_t stream, uint64_t key, uint64_t i, float std) {
    uint64_t h = orc_hash_u64(stream, key, i);
    int32_t s = 0;
    for (int q = 0; q < 4; q += 1) {
        s += 2 * (int32_t)((h >> (16 * q)) & 0xffffu) + 1;
    }
    float z = (float)(s - 262144) * 7.62939453125e-06f; /* (sum - 2^18) * 2^-17 */
    float v = z * 1.7320508075688772f;
    return v * std;
}

void orc_fill_normal_f16(uint16_t *dst, size_t n, uint64_t stream, uint64_t seed, float std) {
    for (size_t i = 0; i < n; i += 1) {
        dst[i] = orc_f2h(orc_normal(stream, seed, i, std));
    }
}

void orc_fill_normal_f32(float *dst, size_t n, uint64_t stream, uint64_t seed, float std) {
    for (size_t i = 0; i < n; i += 1) {
        dst[i] = orc_normal(stream, seed, i, std);
    }
}

/* ------------------------------------------------------------------ */
/* a tiny deterministic parallel-for (outputs are disjoint per item)    */
/* ------------------------------------------------------------------ */

typedef void (*orc_item_fn)(void *ctx, uint64_t item);

typedef struct {
    orc_item_fn fn;
    void *ctx;
    uint64_t n;
    atomic_uint_fast64_t next;
} orc_pool_t;

static void *orc_worker(void *arg) {
    orc_pool_t *p = arg;
    for (;;) {
        uint64_t i = atomic_fetch_add(&p->next, 1);
        if (i >= p->n) {
            break;
        }
        p->fn(p->ctx, i);
    }
    return NULL;
}

static void orc_parallel(uint64_t n, orc_item_fn fn, void *ctx, int threads) {
    if (threads <= 1 || n <= 1) {
        for (uint64_t i = 0; i < n; i += 1) {
            fn(ctx, i);
        }
        return;
    }
    if (threads > 256) {
        threads = 256;
    }
    orc_pool_t p = {.fn = fn, .ctx = ctx, .n = n};
    atomic_init(&p.next, 0);
    pthread_t tid[256];
    int started = 0;
    for (int t = 1; t < threads; t += 1) {
        if (pthread_create(&tid[started], NULL, orc_worker, &p) == 0) {
            started += 1;
        }
    }
    orc_worker(&p);
    for (int t = 0; t < started; t += 1) {
        pthread_join(tid[t], NULL);
    }
}

/* ------------------------------------------------------------------ */
/* fixed-order dot product used for every GEMM output                   */
/* ------------------------------------------------------------------ */

/* 16 interleaved fmaf chains (chain j takes i = j mod 16, increasing i), then
 * a fixed pairwise fold 8, 4, 2, 1.  n % 16 == 0. */
static float orc_dot16(const float *a, const float *b, uint32_t n) {
    float p[16];
    for (int j = 0; j < 16; j += 1) {
        p[j] = 0.0f;
    }
    for (uint32_t i = 0; i < n; i += 16) {
        for (int j = 0; j < 16; j += 1) {
            p[j] = fmaf(a[i + j], b[i + j], p[j]);
        }
    }
    for (int w = 8; w >= 1; w >>= 1) {
        for (int j = 0; j < w; j += 1) {
            p[j] = p[j] + p[j + w];
        }
    }
    return p[0];
}

/* ------------------------------------------------------------------ */
/* router projection: the library's canonical fp32 order                */
/* ------------------------------------------------------------------ */

typedef struct {
    const rmda_moe_router_t *pc;
    const uint16_t *x16;
    const float *wt; /* [cols][L][8] interleaved chunks */
    const float *bias;
    float post;      /* applied to the chunk sum before the bias (1/slot scale) */
    float *proj;
} orc_router_job_t;

static void orc_router_row(void *vctx, uint64_t r) {
    orc_router_job_t *j = vctx;
    uint32_t d = j->pc->d;
    uint32_t L = d / 8;
    float *xt = malloc(sizeof(float) * d);
    /* xt[i*8 + q] = x[q*L + i] */
    for (uint32_t q = 0; q < 8; q += 1) {
        for (uint32_t i = 0; i < L; i += 1) {
            xt[i * 8 + q] = orc_h2f(j->x16[r * d + q * L + i]);
        }
    }
    for (uint32_t c = 0; c < j->pc->cols; c += 1) {
        const float *w = j->wt + (size_t)c * d;
        float p[8];
        for (int q = 0; q < 8; q += 1) {
            p[q] = 0.0f;
        }
        for (uint32_t i = 0; i < L; i += 1) {
            for (int q = 0; q < 8; q += 1) {
                p[q] = fmaf(xt[i * 8 + q], w[i * 8 + q], p[q]);
            }
        }
        float s = p[0];
        for (int q = 1; q < 8; q += 1) {
            s = s + p[q];
        }
        s = s * j->post;
        if (j->bias != NULL && c < j->pc->nbias) {
            s = s + j->bias[c];
        }
        j->proj[r * j->pc->stride + c] = s;
    }
    free(xt);
}

void orc_router(const rmda_moe_router_t *pc, const uint16_t *x16, const float *w,
                const float *bias, float *proj, int threads) {
    orc_router_scaled(pc, x16, w, bias, 1.0f, proj, threads);
}

/* The same with every chunk sum multiplied by `post` before the bias: the
 * router on a slot-scaled x16 with 1/scale as post (the reference divides
 * the scale out in the GEMM's epilogue, shader/matmul_f16.comp's scale). */
void orc_router_scaled(const rmda_moe_router_t *pc, const uint16_t *x16, const float *w,
                       const float *bias, float post, float *proj, int threads) {
    uint32_t d = pc->d;
    uint32_t L = d / 8;
    float *wt = malloc(sizeof(float) * (size_t)pc->cols * d);
    for (uint32_t c = 0; c < pc->cols; c += 1) {
        for (uint32_t q = 0; q < 8; q += 1) {
            for (uint32_t i = 0; i < L; i += 1) {
                wt[(size_t)c * d + i * 8 + q] = w[(size_t)c * d + q * L + i];
            }
        }
    }
    orc_router_job_t j = {.pc = pc, .x16 = x16, .wt = wt, .bias = bias, .post = post, .proj = proj};
    orc_parallel(pc->rows, orc_router_row, &j, threads);
    free(wt);
}

/* ------------------------------------------------------------------ */
/* moe_route                                                           */
/* ------------------------------------------------------------------ */

/* shader/moe_route.comp:20-61.  Per round, the best untaken column by strict
 * '>' from -3.0e38 (so the lowest index wins ties, NaN and values <= -3e38
 * are never taken: :33-38, the subgroupMax/subgroupMin pair :39-44 picks the
 * lowest index among equal maxima).  wt = exp(l_k - l_0)/z with z summed in
 * selection order (:51-58).  Generalised: only columns < experts are read
 * (the shader reads 512 regardless, :24-26).  A round with nothing left emits
 * RMDA_NONE with value -3.0e38 and is not counted. */
void orc_moe_route(const rmda_pc_moe_route_t *pc, const float *proj, uint32_t *idx,
                   float *wt, uint32_t *count) {
    uint32_t E = pc->experts;
    uint32_t K = pc->topk;
    for (uint32_t e = 0; e < E; e += 1) {
        count[e] = 0;
    }
    uint8_t *taken = malloc(E > 0 ? E : 1);
    for (uint32_t r = 0; r < pc->rows; r += 1) {
        const float *l = proj + (size_t)r * pc->stride;
        memset(taken, 0, E > 0 ? E : 1);
        uint32_t sel[RMDA_MAX_TOPK];
        float sv[RMDA_MAX_TOPK];
        for (uint32_t k = 0; k < K; k += 1) {
            float lb = -3.0e38f;
            uint32_t li = RMDA_NONE;
            for (uint32_t j = 0; j < E; j += 1) {
                if (taken[j] == 0 && l[j] > lb) {
                    lb = l[j];
                    li = j;
                }
            }
            if (li != RMDA_NONE) {
                taken[li] = 1;
            }
            sel[k] = li;
            sv[k] = lb;
        }
        float z = 0.0f;
        for (uint32_t k = 0; k < K; k += 1) {
            z = z + expf(sv[k] - sv[0]);
        }
        for (uint32_t k = 0; k < K; k += 1) {
            idx[(size_t)r * K + k] = sel[k];
            wt[(size_t)r * K + k] = expf(sv[k] - sv[0]) / z;
            if (sel[k] != RMDA_NONE) {
                count[sel[k]] += 1;
            }
        }
    }
    free(taken);
}

/* ------------------------------------------------------------------ */
/* moe_scan                                                            */
/* ------------------------------------------------------------------ */

/* shader/moe_scan.comp:14-37: padded width p_e = ceil(c_e/tile)*tile,
 * off = exclusive prefix, tiles[t] = e over e's tiles.  Tiles the shader
 * does not write keep the host's 0xffffffff fill (src/qwen.c:796); here they
 * are written as RMDA_NONE. */
void orc_moe_scan(const rmda_pc_moe_scan_t *pc, const uint32_t *count, uint32_t *off,
                  uint32_t *tiles, uint32_t n_tiles) {
    uint32_t tile = pc->tile;
    for (uint32_t t = 0; t < n_tiles; t += 1) {
        tiles[t] = RMDA_NONE;
    }
    uint32_t lo = 0;
    for (uint32_t e = 0; e < pc->experts; e += 1) {
        uint32_t p = (count[e] + tile - 1u) / tile * tile;
        off[e] = lo;
        for (uint32_t t = lo / tile; t < (lo + p) / tile; t += 1) {
            if (t < n_tiles) {
                tiles[t] = e;
            }
        }
        lo += p;
    }
}

/* ------------------------------------------------------------------ */
/* moe_scatter                                                         */
/* ------------------------------------------------------------------ */

/* shader/moe_scatter.comp:18-33 executed one workgroup at a time in pr
 * order: p = off[e] + fill[e]++, slot[pr] = p, row pr/topk copied to row p. */
void orc_moe_scatter(const rmda_pc_moe_scatter_t *pc, const uint32_t *idx,
                     const uint32_t *off, uint32_t *fill, const uint16_t *x16,
                     uint16_t *xp, uint32_t *slot) {
    uint32_t d = pc->d8 * 8u;
    uint64_t n = (uint64_t)pc->rows * pc->topk;
    for (uint64_t pr = 0; pr < n; pr += 1) {
        uint32_t e = idx[pr];
        if (e == RMDA_NONE) {
            slot[pr] = RMDA_NONE;
            continue;
        }
        uint32_t p = off[e] + fill[e];
        fill[e] += 1;
        slot[pr] = p;
        if (xp != NULL && x16 != NULL) {
            memcpy(xp + (size_t)p * d, x16 + (size_t)(pr / pc->topk) * d, sizeof(uint16_t) * d);
        }
    }
}

/* ------------------------------------------------------------------ */
/* fp16 scale slots                                                    */
/* ------------------------------------------------------------------ */

/* shader/matmul_f16_moe.comp:60-68 and shader/cast_f16.comp:20-28 */
float orc_slot_scale(const uint32_t *amax, uint32_t slot) {
    if (slot == RMDA_NO_SLOT || amax == NULL) {
        return 1.0f;
    }
    float a = u2f(amax[slot]);
    if (!(a > 0.0f) || isinf(a)) {
        return 1.0f;
    }
    return ldexpf(1.0f, 141 - (int)((amax[slot] >> 23) & 0xffu));
}

/* ------------------------------------------------------------------ */
/* matmul_f16_moe                                                      */
/* ------------------------------------------------------------------ */

typedef struct {
    const rmda_pc_moe_mm_t *pc;
    const uint16_t *a;
    const uint16_t *b;
    float *c;
    const uint32_t *tiles;
    float s;
} orc_mm_job_t;

/* item = one 128-row tile x one 128-column block */
static void orc_mm_item(void *vctx, uint64_t item) {
    orc_mm_job_t *j = vctx;
    const rmda_pc_moe_mm_t *pc = j->pc;
    uint32_t nb = pc->n / RMDA_MM_TILE;
    uint32_t t = (uint32_t)(item / nb);
    uint32_t n0 = (uint32_t)(item % nb) * RMDA_MM_TILE;
    uint32_t e = j->tiles[t];
    if (e == RMDA_NONE) {
        return;
    }
    uint32_t k = pc->k;
    float *bf = malloc(sizeof(float) * (size_t)RMDA_MM_TILE * k);
    float *af = malloc(sizeof(float) * k);
    const uint16_t *be = j->b + (size_t)e * pc->n * k;
    orc_h2f_n(be + (size_t)n0 * k, bf, (size_t)RMDA_MM_TILE * k);
    for (uint32_t r = t * RMDA_MM_TILE; r < (t + 1) * RMDA_MM_TILE && r < pc->m; r += 1) {
        orc_h2f_n(j->a + (size_t)r * k, af, k);
        for (uint32_t c = 0; c < RMDA_MM_TILE; c += 1) {
            float acc = orc_dot16(af, bf + (size_t)c * k, k);
            j->c[(size_t)r * pc->n + n0 + c] = acc * j->s;
        }
    }
    free(af);
    free(bf);
}

/* shader/matmul_f16_moe.comp:70-126: tile t of 128 rows uses expert
 * tiles[t] (skipped when ~0, :71-74); C = acc * (1/(scale(sa)*scale(sb)))
 * (:118-122).  The shader's 16x16x16 coopmat K-steps become orc_dot16. */
void orc_moe_mm(const rmda_pc_moe_mm_t *pc, const uint16_t *a, const uint16_t *b,
                float *c, const uint32_t *amax, const uint32_t *tiles, int threads) {
    orc_mm_job_t j = {.pc = pc, .a = a, .b = b, .c = c, .tiles = tiles};
    j.s = 1.0f / (orc_slot_scale(amax, pc->sa) * orc_slot_scale(amax, pc->sb));
    uint64_t items = (uint64_t)(pc->m / RMDA_MM_TILE) * (pc->n / RMDA_MM_TILE);
    orc_parallel(items, orc_mm_item, &j, threads);
}

/* ------------------------------------------------------------------ */
/* moe_combine                                                         */
/* ------------------------------------------------------------------ */

static float orc_sigmoid(float v) {
    return 1.0f / (1.0f + expf(-v));
}

static float orc_combine_acc(const rmda_pc_moe_combine_t *pc, const float *wt,
                             const uint32_t *slot, const float *y, const float *proj,
                             const float *sh, uint32_t r, uint32_t c) {
    float acc = 0.0f;
    for (uint32_t j = 0; j < pc->topk; j += 1) {
        uint32_t s = slot[(size_t)r * pc->topk + j];
        if (s != RMDA_NONE) {
            acc = acc + wt[(size_t)r * pc->topk + j] * y[(size_t)s * pc->d + c];
        }
    }
    if (sh != NULL) {
        acc = acc + orc_sigmoid(proj[(size_t)r * pc->pstride + pc->sg_off]) * sh[(size_t)r * pc->d + c];
    }
    return acc;
}

/* shader/moe_combine.comp:26-40 */
void orc_moe_combine(const rmda_pc_moe_combine_t *pc, const float *wt, const uint32_t *slot,
                     const float *y, const float *proj, const float *sh, const float *inj,
                     float *h) {
    for (uint32_t r = 0; r < pc->rows; r += 1) {
        for (uint32_t c = 0; c < pc->d; c += 1) {
            float acc = orc_combine_acc(pc, wt, slot, y, proj, sh, r, c);
            for (uint32_t s = 0; s < pc->hc; s += 1) {
                float g = orc_sigmoid(inj[(size_t)r * pc->inj_stride + pc->inj_off + s] / (float)pc->hc);
                h[(size_t)r * pc->hc * pc->d + (size_t)s * pc->d + c] += acc * 2.0f * g;
            }
        }
    }
}

void orc_moe_combine_plain(const rmda_pc_moe_combine_t *pc, const float *wt,
                           const uint32_t *slot, const float *y, const float *proj,
                           const float *sh, float *out) {
    for (uint32_t r = 0; r < pc->rows; r += 1) {
        for (uint32_t c = 0; c < pc->d; c += 1) {
            out[(size_t)r * pc->d + c] = orc_combine_acc(pc, wt, slot, y, proj, sh, r, c);
        }
    }
}

/* ------------------------------------------------------------------ */
/* helpers: qwen_elem, absmax, cast_f16, qwen_bf16                      */
/* ------------------------------------------------------------------ */

static float orc_silu(float v) {
    return v / (1.0f + expf(-v));
}

/* shader/qwen_elem.comp:20-31 */
void orc_qwen_elem(const rmda_pc_qwen_elem_t *pc, const float *a, float *y) {
    for (uint32_t r = 0; r < pc->rows; r += 1) {
        for (uint32_t c = 0; c < pc->n; c += 1) {
            float g = a[(size_t)r * pc->astride + pc->ao + c];
            if (pc->op == 0) {
                y[(size_t)r * pc->n + c] = orc_silu(g) * a[(size_t)r * pc->astride + pc->bo + c];
            } else {
                y[(size_t)r * pc->n + c] = orc_silu(g * pc->scale);
            }
        }
    }
}

/* shader/absmax.comp:13-31: atomicMax on the bit pattern of max |x| */
void orc_absmax(const rmda_pc_absmax_t *pc, const float *x, uint32_t *amax) {
    float m = 0.0f;
    for (uint32_t i = 0; i < pc->n; i += 1) {
        m = fmaxf(m, fabsf(x[i]));
    }
    uint32_t u = f2u(m);
    if (u > amax[pc->slot]) {
        amax[pc->slot] = u;
    }
}

/* shader/cast_f16.comp:30-35 */
void orc_cast_f16(const rmda_pc_cast_t *pc, const float *src, uint16_t *dst, const uint32_t *amax) {
    float s = orc_slot_scale(amax, pc->slot);
    for (uint32_t i = 0; i < pc->n; i += 1) {
        dst[i] = orc_f2h(src[i] * s);
    }
}

/* shader/qwen_bf16.comp:9-15: word = (bf16 hi, bf16 lo) -> packHalf2x16 */
void orc_qwen_bf16(const rmda_pc_qwen_bf16_t *pc, uint32_t *w) {
    for (uint32_t i = 0; i < pc->n; i += 1) {
        uint32_t u = w[i];
        float lo = u2f(u << 16);
        float hi = u2f(u & 0xffff0000u);
        w[i] = (uint32_t)orc_f2h(lo) | ((uint32_t)orc_f2h(hi) << 16);
    }
}

/* ------------------------------------------------------------------ */
/* whole layer                                                         */
/* ------------------------------------------------------------------ */

uint32_t orc_proj_stride(const rmda_moe_shape_t *s) {
    return s->experts + (s->shared > 0 ? 1u : 0u);
}

typedef struct {
    const orc_layer_t *L;
    uint32_t n_pairs;         /* selected pairs */
    const uint32_t *pair_tok; /* token of each selected pair */
    const uint32_t *pair_exp; /* expert (RMDA_NONE = none) */
    const uint16_t *a16;      /* rows x d activations fed to the GEMMs */
    float sa;                 /* 1/scale of a16 */
    float *hp;                /* n_pairs x I */
    uint16_t *hp16;
    float shp;                /* 1/scale of hp16 */
    float *ye;                /* n_pairs x d */
    /* shared expert, per selected token */
    uint32_t n_tok;
    const uint32_t *tok;
    float *hs;                /* n_tok x I_s */
    uint16_t *hs16;
    float shs;
    float *sh;                /* n_tok x d */
} orc_ffn_job_t;

/* gate_up of one selected pair: hp = silu(g[:I]) * g[I:], g = a16 . W_gu[e]^T * sa */
static void orc_ffn_up_item(void *vctx, uint64_t p) {
    orc_ffn_job_t *j = vctx;
    const orc_layer_t *L = j->L;
    uint32_t d = L->shape.d;
    uint32_t I = L->shape.inter;
    uint32_t e = j->pair_exp[p];
    float *hp = j->hp + (size_t)p * I;
    if (e == RMDA_NONE) {
        memset(hp, 0, sizeof(float) * I);
        return;
    }
    float *a = malloc(sizeof(float) * d);
    float *w = malloc(sizeof(float) * d);
    orc_h2f_n(j->a16 + (size_t)j->pair_tok[p] * d, a, d);
    const uint16_t *we = L->w_gate_up + (size_t)e * 2 * I * d;
    float *g = malloc(sizeof(float) * 2 * I);
    for (uint32_t n = 0; n < 2 * I; n += 1) {
        orc_h2f_n(we + (size_t)n * d, w, d);
        g[n] = orc_dot16(a, w, d) * j->sa;
    }
    for (uint32_t c = 0; c < I; c += 1) {
        hp[c] = orc_silu(g[c]) * g[I + c];
    }
    free(g);
    free(w);
    free(a);
}

/* down of one selected pair: ye = hp16 . W_d[e]^T * shp */
static void orc_ffn_down_item(void *vctx, uint64_t p) {
    orc_ffn_job_t *j = vctx;
    const orc_layer_t *L = j->L;
    uint32_t d = L->shape.d;
    uint32_t I = L->shape.inter;
    uint32_t e = j->pair_exp[p];
    float *ye = j->ye + (size_t)p * d;
    if (e == RMDA_NONE) {
        memset(ye, 0, sizeof(float) * d);
        return;
    }
    float *a = malloc(sizeof(float) * I);
    float *w = malloc(sizeof(float) * I);
    orc_h2f_n(j->hp16 + (size_t)p * I, a, I);
    const uint16_t *we = L->w_down + (size_t)e * d * I;
    for (uint32_t n = 0; n < d; n += 1) {
        orc_h2f_n(we + (size_t)n * I, w, I);
        ye[n] = orc_dot16(a, w, I) * j->shp;
    }
    free(w);
    free(a);
}

static void orc_shared_up_item(void *vctx, uint64_t t) {
    orc_ffn_job_t *j = vctx;
    const orc_layer_t *L = j->L;
    uint32_t d = L->shape.d;
    uint32_t I = L->shape.shared;
    float *a = malloc(sizeof(float) * d);
    float *w = malloc(sizeof(float) * d);
    float *g = malloc(sizeof(float) * 2 * I);
    orc_h2f_n(j->a16 + (size_t)j->tok[t] * d, a, d);
    for (uint32_t n = 0; n < 2 * I; n += 1) {
        orc_h2f_n(L->w_sh_gate_up + (size_t)n * d, w, d);
        g[n] = orc_dot16(a, w, d) * j->sa;
    }
    for (uint32_t c = 0; c < I; c += 1) {
        j->hs[(size_t)t * I + c] = orc_silu(g[c]) * g[I + c];
    }
    free(g);
    free(w);
    free(a);
}

static void orc_shared_down_item(void *vctx, uint64_t t) {
    orc_ffn_job_t *j = vctx;
    const orc_layer_t *L = j->L;
    uint32_t d = L->shape.d;
    uint32_t I = L->shape.shared;
    float *a = malloc(sizeof(float) * I);
    float *w = malloc(sizeof(float) * I);
    orc_h2f_n(j->hs16 + (size_t)t * I, a, I);
    for (uint32_t n = 0; n < d; n += 1) {
        orc_h2f_n(L->w_sh_down + (size_t)n * I, w, I);
        j->sh[(size_t)t * d + n] = orc_dot16(a, w, I) * j->shs;
    }
    free(w);
    free(a);
}

/* fp16 cast of n fp32 values with the reference's optional power-of-two
 * slot scale (absmax.comp + cast_f16.comp, src/qwen.c:517-539); returns
 * 1/scale, the factor the consuming GEMM applies (matmul_f16_moe.comp:118). */
static float orc_scaled_cast(const float *src, uint16_t *dst, size_t n, int scaled) {
    uint32_t amax = 0;
    rmda_pc_absmax_t pa = {.n = 0, .slot = 0};
    rmda_pc_cast_t pc = {.n = 0, .slot = scaled ? 0u : RMDA_NO_SLOT};
    if (scaled) {
        /* absmax over the whole buffer, chunked to keep n in uint32 */
        for (size_t i = 0; i < n; i += 1u << 30) {
            size_t m = n - i < (1u << 30) ? n - i : (1u << 30);
            pa.n = (uint32_t)m;
            orc_absmax(&pa, src + i, &amax);
        }
    }
    for (size_t i = 0; i < n; i += 1u << 30) {
        size_t m = n - i < (1u << 30) ? n - i : (1u << 30);
        pc.n = (uint32_t)m;
        orc_cast_f16(&pc, src + i, dst + i, &amax);
    }
    return 1.0f / orc_slot_scale(&amax, pc.slot);
}

static double orc_now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec * 1e3 + (double)ts.tv_nsec * 1e-6;
}

int orc_moe_layer(const orc_layer_t *L) {
    const rmda_moe_shape_t *S = &L->shape;
    uint32_t T = S->rows;
    uint32_t d = S->d;
    uint32_t E = S->experts;
    uint32_t K = S->topk;
    if (d % 32 != 0 || E == 0 || E > RMDA_MAX_EXPERTS || K == 0 || K > RMDA_MAX_TOPK || K > E ||
        S->inter % 16 != 0 || S->shared % 16 != 0 || L->tile == 0) {
        return -1;
    }
    uint32_t ps = orc_proj_stride(S);
    int th = L->threads;
    float *proj = L->proj ? L->proj : malloc(sizeof(float) * (size_t)T * ps + 4);
    uint32_t *idx = L->idx ? L->idx : malloc(sizeof(uint32_t) * (size_t)T * K + 4);
    float *wt = L->wt ? L->wt : malloc(sizeof(float) * (size_t)T * K + 4);
    uint32_t *slot = L->slot ? L->slot : malloc(sizeof(uint32_t) * (size_t)T * K + 4);
    uint32_t *count = L->count ? L->count : malloc(sizeof(uint32_t) * E);
    uint32_t *off = L->off ? L->off : malloc(sizeof(uint32_t) * E);
    uint32_t *fill = calloc(E, sizeof(uint32_t));

    double t_mark = orc_now_ms();
    double st[ORC_LAYER_STAGES] = {0};
#define ORC_STAGE(i)                   \
    do {                               \
        const double t_now = orc_now_ms(); \
        st[i] += t_now - t_mark;       \
        t_mark = t_now;                \
    } while (0)
    /* activations fed to the GEMMs: x, optionally power-of-two scaled
     * (src/qwen.c:844; bit-neutral for in-range values); with fp32 x32 always
     * scaled, as the reference casts its fp32 sc->x, and the router reads the
     * same cast with the scale divided out */
    size_t xn = (size_t)T * d;
    uint16_t *a16 = malloc(sizeof(uint16_t) * xn + 2);
    float sa = 1.0f;
    if (L->x32 != NULL) {
        sa = orc_scaled_cast(L->x32, a16, xn, 1);
    } else if (L->x_scale) {
        float *xf = malloc(sizeof(float) * xn + 4);
        orc_h2f_n(L->x, xf, xn);
        sa = orc_scaled_cast(xf, a16, xn, 1);
        free(xf);
    } else {
        memcpy(a16, L->x, sizeof(uint16_t) * xn);
    }
    /* A0: router projection (x . [W_router; w_shared_gate]^T), canonical order */
    rmda_moe_router_t pr = {.rows = T, .d = d, .cols = ps, .stride = ps, .nbias = E};
    if (L->x32 != NULL) {
        orc_router_scaled(&pr, a16, L->w_router, L->bias, sa, proj, th);
    } else {
        orc_router(&pr, L->x, L->w_router, L->bias, proj, th);
    }
    ORC_STAGE(0);
    /* A1-A3: route, scan, scatter (slots only; the GEMMs read token rows) */
    rmda_pc_moe_route_t pc_r = {.rows = T, .experts = E, .topk = K, .stride = ps};
    orc_moe_route(&pc_r, proj, idx, wt, count);
    ORC_STAGE(1);
    rmda_pc_moe_scan_t pc_s = {.experts = E, .tile = L->tile};
    orc_moe_scan(&pc_s, count, off, NULL, 0);
    ORC_STAGE(2);
    rmda_pc_moe_scatter_t pc_t = {.rows = T, .topk = K, .d8 = d / 8};
    orc_moe_scatter(&pc_t, idx, off, fill, NULL, NULL, slot);
    ORC_STAGE(3);


    /* selected tokens and their pairs */
    uint32_t n_tok = L->rows_sel ? L->n_sel : T;
    uint32_t *tok = malloc(sizeof(uint32_t) * (n_tok + 1));
    for (uint32_t t = 0; t < n_tok; t += 1) {
        tok[t] = L->rows_sel ? L->rows_sel[t] : t;
    }
    uint32_t n_pairs = n_tok * K;
    uint32_t *pair_tok = malloc(sizeof(uint32_t) * (n_pairs + 1));
    uint32_t *pair_exp = malloc(sizeof(uint32_t) * (n_pairs + 1));
    for (uint32_t t = 0; t < n_tok; t += 1) {
        for (uint32_t j = 0; j < K; j += 1) {
            pair_tok[t * K + j] = tok[t];
            pair_exp[t * K + j] = idx[(size_t)tok[t] * K + j];
        }
    }
    uint32_t I = S->inter;
    orc_ffn_job_t job = {
        .L = L, .n_pairs = n_pairs, .pair_tok = pair_tok, .pair_exp = pair_exp,
        .a16 = a16, .sa = sa, .n_tok = n_tok, .tok = tok,
    };
    /* A4-A6: gate_up, SwiGLU, fp16 cast of hp (src/qwen.c:847-877) */
    job.hp = malloc(sizeof(float) * (size_t)n_pairs * I + 4);
    job.hp16 = malloc(sizeof(uint16_t) * (size_t)n_pairs * I + 2);
    orc_parallel(n_pairs, orc_ffn_up_item, &job, th);
    job.shp = orc_scaled_cast(job.hp, job.hp16, (size_t)n_pairs * I, L->hp_scale);
    ORC_STAGE(4);
    /* A7: down (src/qwen.c:878) */
    job.ye = malloc(sizeof(float) * (size_t)n_pairs * d + 4);
    orc_parallel(n_pairs, orc_ffn_down_item, &job, th);
    if (L->ye16) {
        for (size_t i = 0; i < (size_t)n_pairs * d; i += 1) {
            job.ye[i] = orc_h2f(orc_f2h(job.ye[i]));
        }
    }
    ORC_STAGE(5);
    /* A8: shared expert (src/qwen.c:879-886) */
    if (S->shared > 0) {
        uint32_t Is = S->shared;
        job.hs = malloc(sizeof(float) * (size_t)n_tok * Is + 4);
        job.hs16 = malloc(sizeof(uint16_t) * (size_t)n_tok * Is + 2);
        orc_parallel(n_tok, orc_shared_up_item, &job, th);
        job.shs = orc_scaled_cast(job.hs, job.hs16, (size_t)n_tok * Is, L->hp_scale);
        job.sh = malloc(sizeof(float) * (size_t)n_tok * d + 4);
        orc_parallel(n_tok, orc_shared_down_item, &job, th);
        if (L->ye16) {
            for (size_t i = 0; i < (size_t)n_tok * d; i += 1) {
                job.sh[i] = orc_h2f(orc_f2h(job.sh[i]));
            }
        }
    }
    ORC_STAGE(6);
    /* A9: combine, plain mode, in j order (moe_combine.comp:31-35); ye rows
     * are per selected pair, so slot here is the pair's position. */
    for (uint32_t t = 0; t < n_tok; t += 1) {
        uint32_t r = tok[t];
        for (uint32_t c = 0; c < d; c += 1) {
            float acc = 0.0f;
            for (uint32_t j = 0; j < K; j += 1) {
                if (pair_exp[t * K + j] != RMDA_NONE) {
                    acc = acc + wt[(size_t)r * K + j] * job.ye[((size_t)t * K + j) * d + c];
                }
            }
            if (S->shared > 0) {
                acc = acc + orc_sigmoid(proj[(size_t)r * ps + E]) * job.sh[(size_t)t * d + c];
            }
            L->out[(size_t)t * d + c] = acc;
        }
    }
    ORC_STAGE(7);
#undef ORC_STAGE
    if (L->stage_ms != NULL) {
        memcpy(L->stage_ms, st, sizeof(st));
    }
    free(job.hp);
    free(job.hp16);
    free(job.ye);
    if (S->shared > 0) {
        free(job.hs);
        free(job.hs16);
        free(job.sh);
    }
    free(pair_exp);
    free(pair_tok);
    free(tok);
    free(a16);
    free(fill);
    if (L->off == NULL) free(off);
    if (L->count == NULL) free(count);
    if (L->slot == NULL) free(slot);
    if (L->wt == NULL) free(wt);
    if (L->idx == NULL) free(idx);
    if (L->proj == NULL) free(proj);
    return 0;
}
