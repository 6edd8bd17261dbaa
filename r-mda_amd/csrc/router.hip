// Router projection: proj[r, c] = x16[r, :] . w[c, :] (+ bias[c]) in fp32.
//
// Replaces the dense fp16 GEMM that fills the reference's `p` buffer
// (src/qwen.c:845 -> :541-570, shader/matmul_f16(_wide).comp).  Routing must
// be bit-exact, so the logits follow one fixed order that the CPU oracle
// replays: d is cut into 8 contiguous chunks of L = d/8; chunk q's partial is
// a sequential fmaf chain over i = qL .. qL+L-1 starting from 0; the eight
// partials are added left to right, then the bias.
//
// Two kernels compute the same bits:
//
// router_mf_kernel (d % 128 == 0; the layer always uses it) runs the chunk
// chains on the matrix cores: the fp32 MFMA v_mfma_f32_16x16x4f32 applies
// its four k terms as four fused multiply-adds in k order, so chained
// MFMAs are the fmaf chain itself (details at the kernel).
//
// router_tile_kernel (any d % 32 == 0; the standalone entry point uses it
// when d % 128 != 0).  A workgroup owns 16 tokens x 32 columns; 256 threads
// = 8 chunk groups x 32, each thread keeps 4 tokens x 4 columns of one
// chunk's partials in registers and walks its chunk through a
// double-buffered LDS tile.
#include "common.h"

namespace {

constexpr int TM = 16;  // tokens per tile
constexpr int TC = 32;  // columns per tile
constexpr int BK = 16;  // k per step inside a chunk
constexpr int NQ = 8;   // chunks

struct Smem {
    union {
        struct {
            float xs[2][NQ][BK][TM];  // [buf][chunk][i][token]
            float ws[2][NQ][BK][TC];  // [buf][chunk][i][column]
        } s;
        float red[NQ][TM][TC];        // chunk partials after the k loop
    } u;
};

__global__ __launch_bounds__(256) void router_tile_kernel(const uint16_t *__restrict__ x16,
                                                     const float *__restrict__ w,
                                                     const float *__restrict__ bias,
                                                     float *__restrict__ proj, uint32_t rows,
                                                     uint32_t d, uint32_t cols, uint32_t stride,
                                                     uint32_t nbias, uint32_t *zero_words,
                                                     uint32_t n_zero) {
    __shared__ Smem sm;
    const uint32_t tid = threadIdx.x;
    const uint32_t t0 = blockIdx.x * TM;
    const uint32_t c0 = blockIdx.y * TC;
    if (zero_words != nullptr && blockIdx.x == 0 && blockIdx.y == 0) {
        for (uint32_t i = tid; i < n_zero; i += 256) {
            zero_words[i] = 0;
        }
    }
    const uint32_t L = d / NQ;
    const uint32_t steps = L / BK;

    // loader roles: x: (chunk, token, half of the 16-element step); w: (chunk, column)
    const uint32_t lq = tid / 32;
    const uint32_t lx = (tid % 32) / 2;
    const uint32_t lh = tid % 2;
    const uint32_t lc = tid % 32;
    const bool xok = t0 + lx < rows;
    const bool wok = c0 + lc < cols;
    const uint16_t *xrow = x16 + (size_t)(xok ? t0 + lx : 0) * d + lq * L + lh * 8;
    const float *wrow = w + (size_t)(wok ? c0 + lc : 0) * d + lq * L;

    // compute roles: (chunk q, 4 tokens tb*4.., 4 columns cb*4..)
    const uint32_t q = tid / 32;
    const uint32_t tb = (tid % 32) / 8;
    const uint32_t cb = tid % 8;

    uint4 xr;
    float4 wr[4];
    auto gload = [&](uint32_t s) {
        xr = xok ? *reinterpret_cast<const uint4 *>(xrow + s * BK) : make_uint4(0, 0, 0, 0);
        const float4 *wp = reinterpret_cast<const float4 *>(wrow + s * BK);
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
            wr[i] = wok ? wp[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto lstore = [&](int buf) {
        const uint16_t *xh = reinterpret_cast<const uint16_t *>(&xr);
        const float *wf = reinterpret_cast<const float *>(wr);
#pragma unroll
        for (int i = 0; i < 8; i += 1) {
            sm.u.s.xs[buf][lq][lh * 8 + i][lx] = rmda_h2f(xh[i]);
        }
#pragma unroll
        for (int i = 0; i < BK; i += 1) {
            sm.u.s.ws[buf][lq][i][lc] = wf[i];
        }
    };

    float acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a += 1) {
#pragma unroll
        for (int b = 0; b < 4; b += 1) {
            acc[a][b] = 0.0f;
        }
    }

    gload(0);
    lstore(0);
    __syncthreads();
    for (uint32_t s = 0; s < steps; s += 1) {
        const int buf = s & 1;
        if (s + 1 < steps) {
            gload(s + 1);
        }
#pragma unroll 8
        for (int i = 0; i < BK; i += 1) {
            const float4 xa = *reinterpret_cast<const float4 *>(&sm.u.s.xs[buf][q][i][tb * 4]);
            const float4 wv = *reinterpret_cast<const float4 *>(&sm.u.s.ws[buf][q][i][cb * 4]);
            const float xv[4] = {xa.x, xa.y, xa.z, xa.w};
            const float wf[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int a = 0; a < 4; a += 1) {
#pragma unroll
                for (int b = 0; b < 4; b += 1) {
                    acc[a][b] = __builtin_fmaf(xv[a], wf[b], acc[a][b]);
                }
            }
        }
        if (s + 1 < steps) {
            lstore(buf ^ 1);
        }
        __syncthreads();
    }

    // chunk partials -> LDS, then sum in chunk order (the xs/ws buffers are dead)
#pragma unroll
    for (int a = 0; a < 4; a += 1) {
#pragma unroll
        for (int b = 0; b < 4; b += 1) {
            sm.u.red[q][tb * 4 + a][cb * 4 + b] = acc[a][b];
        }
    }
    __syncthreads();
    for (uint32_t o = tid; o < TM * TC; o += 256) {
        const uint32_t t = o / TC;
        const uint32_t c = o % TC;
        float s = sm.u.red[0][t][c];
#pragma unroll
        for (int qq = 1; qq < NQ; qq += 1) {
            s = s + sm.u.red[qq][t][c];
        }
        if (bias != nullptr && c0 + c < nbias) {
            s = s + bias[c0 + c];
        }
        if (t0 + t < rows && c0 + c < cols) {
            proj[(size_t)(t0 + t) * stride + c0 + c] = s;
        }
    }
}

typedef float rmda_f32x4 __attribute__((ext_vector_type(4)));

constexpr int MF_TOK = 16;  // tokens per 16x16 MFMA tile (A rows)
constexpr int MF_TT = 2;    // token tiles per workgroup (32 tokens)
constexpr int MF_TPW = 2;   // 16-column tiles per wave
constexpr int MF_NCOL = 16 * MF_TPW;  // columns per workgroup
constexpr int MF_NW = NQ;   // waves per workgroup: the 8 d chunks
// Small tile for few tokens: 16 tokens x 16 columns, so that T = 128 still
// spreads over 64 workgroups instead of 16
constexpr int MF_TT_SMALL = 1;
constexpr int MF_TPW_SMALL = 1;
constexpr uint32_t MF_MIN_WGS = 128;  // below this many 32 x 32 workgroups, use the small tile
constexpr int MF_KS = 16;   // k per sub-tile (4 MFMA steps)
constexpr int MF_D = 3;     // sub-tiles a wave's loads run ahead of its MFMAs

__device__ __forceinline__ float h_lo(uint32_t v) { return rmda_h2f((uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float h_hi(uint32_t v) { return rmda_h2f((uint16_t)(v >> 16)); }

// Router on the matrix cores, bit-exact with the canonical order.
//
// v_mfma_f32_16x16x4f32 takes A[i][kk] from lane 16*kk + i, B[kk][j] from
// lane 16*kk + j, and updates accumulator element v of lane 16*m + j, the
// output D[4m+v][j], as four fused multiply-adds in kk order (c + a0*b0
// rounded, + a1*b1 rounded, ...).  A chain of such steps over k = 4s + kk,
// s = 0, 1, ... is therefore exactly the sequential fmaf chain of one d
// chunk, which is what the canonical order asks for; the chunk partials
// are then added left to right as before.
//
// Workgroup = 32 tokens x 32 columns (2 x 2 output tiles, TT = TPW = 2);
// its 8 waves are the 8 d chunks, each computing all four tiles of its
// chunk.  With few tokens (decode) the workgroup is 16 x 16 (TT = TPW = 1):
// the same chunk chains, more workgroups.  The matrix
// cores are not the limit (16x16x4 f32 issues at ~150 TF/s even from two
// waves per SIMD): what a workgroup waits for is its operands, every one
// of which misses L1 (weights are re-read by every token block, activations
// by every column block).  32 x 32 gives the fewest bytes per FLOP at which
// T = 2048 still puts a workgroup on every CU; measured against 16 x 64,
// 64 x 16, 16 x 128 and 32 x 64 it was fastest at configs 3 and 5.  Waves
// start at different chunks, which spreads the workgroups' reads over the
// matrix.
//
// Per wave, loads run MF_D sub-tiles ahead in registers.  Activations pass
// through a wave-private LDS sub-tile (32 tokens x 16 k, fp32, stored
// [token][kk][step] so lane (kk, token) reads its four steps with one
// 16-byte read), double-buffered so that the next sub-tile's write and
// read-back overlap the current sub-tile's MFMAs.  The LDS performs one
// wave's operations in issue order, so no barrier sits between its writes
// and reads.  Packed weights ([d/16][cpad][4 kk][4 steps],
// router_pack_kernel) give each lane four steps of one column as one
// float4, one 1 KiB contiguous load per column tile per 16 k.  HF [cols][d]
// weights are read as four dwords per lane instead.
//
// FUSE (top-k fused in; cols <= 32, one column slice): the workgroup holds
// every logit of its tokens in LDS and routes them there, so the routing
// needs no second launch.  Wider rows are routed by route_kernel: handing
// logits between workgroups would need device-scope ordering across XCDs.
template <bool W_PACKED, bool FUSE, int TT, int TPW>
__global__ __launch_bounds__(MF_NW * RMDA_WAVE) void router_mf_kernel(
    const uint16_t *__restrict__ x16, const float *__restrict__ w, const float *__restrict__ bias,
    float *__restrict__ proj, uint32_t rows, uint32_t d, uint32_t cols, uint32_t cpad, uint32_t stride,
    uint32_t nbias, uint32_t *zero_words, uint32_t n_zero, rmda_route_fuse_t fz, uint32_t col0,
    const uint32_t *xscale) {
    constexpr uint32_t NCOL = 16 * TPW;
    constexpr int KS = MF_KS;
    constexpr uint32_t NW = MF_NW;
    static_assert(NQ * NCOL / (16 * TPW) == NW, "one wave per d chunk and column slice");
    constexpr uint32_t NT = NW * RMDA_WAVE;
    constexpr uint32_t TOK = MF_TOK * TT;
    constexpr int SPS = KS / 4;   // MFMA steps per sub-tile
    constexpr int G16 = KS / 16;  // 16-k weight groups per sub-tile
    constexpr int XS = KS + 4;    // padded LDS token row: a wave's 16-byte reads of 16 rows hit distinct banks
    static_assert(KS == 16 || KS == 32, "sub-tile");
    __shared__ float xs[NW][2][TOK][XS];
    __shared__ float red[NQ][TOK][NCOL];
    __shared__ float lg[TOK][NCOL];

    const uint32_t lane = threadIdx.x % RMDA_WAVE;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x / RMDA_WAVE);
    const uint32_t q = (wv + blockIdx.x) % NQ;  // d chunk
    const uint32_t cl = (wv / NQ) * TPW * 16;   // the wave's first column within the workgroup
    if (zero_words != nullptr && blockIdx.x == 0 && blockIdx.y == 0) {
        for (uint32_t i = threadIdx.x; i < n_zero; i += NT) {
            zero_words[i] = 0;
        }
    }
    const uint32_t L = d / NQ;
    const uint32_t nsub = L / KS;  // d % (8*KS) == 0 is a launch condition
    const uint32_t t0 = blockIdx.x * TOK;
    const uint32_t c0 = col0 + blockIdx.y * NCOL;  // columns from col0 (the wide tile's remainder)
    const float xinv = rmda_slot_inv(xscale);     // 1 unless x16 was cast with a slot
    const uint32_t kk = lane / 16;
    const uint32_t ln = lane % 16;  // A: token row; B: column within a tile

    // B operand, one pointer per column tile; columns past the matrix read a
    // valid one and are never stored
    const float *wb[TPW];
#pragma unroll
    for (int b = 0; b < TPW; b += 1) {
        const uint32_t c = c0 + cl + 16 * b + ln;
        if (W_PACKED) {
            wb[b] = w + (((size_t)(q * L / 16) * cpad + (c < cpad ? c : cpad - 1)) * 4 + kk) * 4;
        } else {
            wb[b] = w + (size_t)(c < cols ? c : 0) * d + q * L + kk;
        }
    }
    // activation fill: lane loads tokens lane/4 + 16*tt, k = SPS*(lane%4) ..
    // +SPS-1 of the sub-tile (steps G16*(lane%4) .., all four kk); token rows
    // past `rows` re-read the last row and are never stored
    const uint32_t ft = lane / 4;
    const uint32_t fq = lane % 4;
    const uint16_t *xp[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt += 1) {
        const uint32_t tok = t0 + 16 * tt + ft;
        xp[tt] = x16 + (size_t)(tok < rows ? tok : rows - 1) * d + q * L + SPS * fq;
    }
    float *xw = &xs[wv][0][ft][G16 * fq];  // + buffer * TOK * XS
    const float *xr = &xs[wv][0][ln][SPS * kk];

    typedef uint32_t xvec_t __attribute__((ext_vector_type(G16 * 2)));
    auto load_x = [&](uint32_t s, xvec_t (&o)[TT]) {
#pragma unroll
        for (int tt = 0; tt < TT; tt += 1) {
            o[tt] = *reinterpret_cast<const xvec_t *>(xp[tt] + (size_t)s * KS);
        }
    };
    auto load_w = [&](uint32_t s, float4 (&o)[G16][TPW]) {
#pragma unroll
        for (int g = 0; g < G16; g += 1) {
#pragma unroll
            for (int b = 0; b < TPW; b += 1) {
                if (W_PACKED) {
                    o[g][b] = *reinterpret_cast<const float4 *>(wb[b] + ((size_t)s * G16 + g) * cpad * 16);
                } else {
                    const float *p = wb[b] + (size_t)s * KS + 16 * g;
                    o[g][b] = make_float4(p[0], p[4], p[8], p[12]);
                }
            }
        }
    };

    rmda_f32x4 acc[TT][TPW];
#pragma unroll
    for (int tt = 0; tt < TT; tt += 1) {
#pragma unroll
        for (int b = 0; b < TPW; b += 1) {
            acc[tt][b] = rmda_f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    // Software pipeline over sub-tiles.  Loads run MF_D sub-tiles ahead in a
    // register ring of R = MF_D + 1 slots (sub-tile s in slot s % R); loads
    // past the last sub-tile re-read it (in bounds, never used), so every
    // step issues the same loads and the compiler's waits stay static.  In
    // step s the wave converts sub-tile s+1's activations into LDS buffer
    // (s+1) % 2 and reads back its A operands while sub-tile s's MFMAs run,
    // so no LDS round trip sits in front of the MFMAs.
    constexpr int R = MF_D + 1;
    static_assert(R % 2 == 0, "sub-tile s uses LDS buffer s % 2 == slot parity");
    float4 wbuf[R][G16][TPW];
    xvec_t xbuf[R][TT];
    float a_cur[TT][SPS];
    float a_nxt[TT][SPS];
    auto fill_x = [&](int buf, const xvec_t (&xv)[TT]) {
        // element e of a lane's load is step G16*fq + e/4, kk = e%4
#pragma unroll
        for (int tt = 0; tt < TT; tt += 1) {
#pragma unroll
            for (int e = 0; e < SPS; e += 1) {
                const uint32_t word = xv[tt][e / 2];
                xw[(buf * TOK + 16 * tt) * XS + (e % 4) * SPS + e / 4] = (e % 2) ? h_hi(word) : h_lo(word);
            }
        }
    };
    auto read_a = [&](int buf, float (&av)[TT][SPS]) {
#pragma unroll
        for (int tt = 0; tt < TT; tt += 1) {
#pragma unroll
            for (int g = 0; g < G16; g += 1) {
                const float4 a = *reinterpret_cast<const float4 *>(xr + (buf * TOK + 16 * tt) * XS + 4 * g);
                av[tt][4 * g] = a.x;
                av[tt][4 * g + 1] = a.y;
                av[tt][4 * g + 2] = a.z;
                av[tt][4 * g + 3] = a.w;
            }
        }
    };
    // wave-scope ordering between this wave's LDS writes and reads (the LDS
    // performs one wave's operations in issue order; this only keeps the
    // compiler from moving them)
    auto wave_order = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
    };
#pragma unroll
    for (int j = 0; j < MF_D; j += 1) {
        const uint32_t sl = (uint32_t)j < nsub ? (uint32_t)j : nsub - 1;
        load_x(sl, xbuf[j]);
        load_w(sl, wbuf[j]);
    }
    fill_x(0, xbuf[0]);
    wave_order();
    read_a(0, a_cur);
    for (uint32_t s0 = 0; s0 < nsub; s0 += R) {
#pragma unroll
        for (int j = 0; j < R; j += 1) {
            const uint32_t s = s0 + j;
            const uint32_t sn = s + MF_D < nsub ? s + MF_D : nsub - 1;
            load_x(sn, xbuf[(j + MF_D) % R]);
            load_w(sn, wbuf[(j + MF_D) % R]);
            if (s + 1 < nsub) {
                wave_order();
                fill_x((j + 1) % 2, xbuf[(j + 1) % R]);
                wave_order();
                read_a((j + 1) % 2, a_nxt);
            }
            if (s < nsub) {
#pragma unroll
                for (int st = 0; st < SPS; st += 1) {
#pragma unroll
                    for (int b = 0; b < TPW; b += 1) {
                        const float4 bq = wbuf[j][st / 4][b];
                        const int jj = st % 4;
                        const float bv = jj == 0 ? bq.x : jj == 1 ? bq.y : jj == 2 ? bq.z : bq.w;
#pragma unroll
                        for (int tt = 0; tt < TT; tt += 1) {
                            acc[tt][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a_cur[tt][st], bv, acc[tt][b], 0, 0, 0);
                        }
                    }
                }
            }
#pragma unroll
            for (int tt = 0; tt < TT; tt += 1) {
#pragma unroll
                for (int st = 0; st < SPS; st += 1) {
                    a_cur[tt][st] = a_nxt[tt][st];
                }
            }
        }
    }

    // D[4*kk + v][ln] of tile (tt, b) is token 16*tt + 4*kk + v, column cl + 16b + ln
#pragma unroll
    for (int tt = 0; tt < TT; tt += 1) {
#pragma unroll
        for (int b = 0; b < TPW; b += 1) {
#pragma unroll
            for (int v = 0; v < 4; v += 1) {
                red[q][16 * tt + 4 * kk + v][cl + 16 * b + ln] = acc[tt][b][v];
            }
        }
    }
    __syncthreads();
    for (uint32_t o = threadIdx.x; o < TOK * NCOL; o += NT) {
        const uint32_t t = o / NCOL;
        const uint32_t l = o % NCOL;
        const uint32_t cc = c0 + l;
        float v = red[0][t][l];
#pragma unroll
        for (int qq = 1; qq < NQ; qq += 1) {
            v = v + red[qq][t][l];
        }
        v = v * xinv;
        if (bias != nullptr && cc < nbias) {
            v = v + bias[cc];
        }
        lg[t][l] = v;
        if (t0 + t < rows && cc < cols) {
            proj[(size_t)(t0 + t) * stride + cc] = v;
        }
    }
    if (!FUSE) {
        return;
    }
    // fused top-k (fz.experts <= NCOL): wave w routes tokens t0 + w, t0 + w + NW, ...
    __syncthreads();
    for (uint32_t tt = wv; tt < TOK && t0 + tt < rows; tt += NW) {
        const uint32_t t = t0 + tt;
        rmda_route_row<(NCOL >= RMDA_WAVE ? NCOL / RMDA_WAVE : 1), false>(&lg[tt][0], fz.experts, fz.topk, fz.idx + (size_t)t * fz.topk,
                                                fz.wt + (size_t)t * fz.topk, nullptr);
    }
}

// Wide tile for many tokens and many columns (T = 4096, 512 experts): the
// same chunk chains, bit for bit, with the work cut the other way.  A
// workgroup owns 64 tokens x 128 columns; each of its 8 waves owns 16 of the
// columns for all 64 tokens and runs all 8 d-chunk chains of them, so the
// eight partials of an output sit in one lane's registers and are added
// there, left to right, with no LDS reduction.  The activations are staged
// once per workgroup in LDS (fp32, double-buffered, one 16-k step of every
// chunk at a time) and read by all eight waves; the weights come straight
// from memory, each value used for four token tiles.  Against the 32 x 32
// tile above this reads the activations 4x and the weights 2x less often
// from L2 (config 5: 0.33 GB of L2-to-CU traffic instead of 0.81 GB) and keeps
// the MFMAs fed from registers and LDS.
//
// Per 16-k step s the workgroup stages x[64 tokens][chunk q][16 k] for all 8
// chunks into LDS as xs[buf][q][tt][lane] float4 (lane = 16*kk + i holds
// token 16*tt + i, k = 16*(q*nsub + s) + 4*st + kk for st = 0..3, i.e. the A
// operand of four consecutive MFMA steps), then each wave runs, per chunk,
// four steps of v_mfma_f32_16x16x4f32 on its four token tiles.  The weight
// float4 of chunk q for the next step is loaded as soon as this step's has
// been used, a full step (8 chunks) ahead.
// TT token tiles of 16 per wave and workgroup: 4 (64 tokens) by default, 2
// (32 tokens) when 64-token workgroups would be too few
constexpr uint32_t RW_NW = 8;              // waves per workgroup
constexpr uint32_t RW_COL = 16 * RW_NW;    // columns per workgroup
constexpr uint32_t RW_NT = RW_NW * RMDA_WAVE;
constexpr uint32_t RW_MIN_WGS = 192;       // use the wide tile when it gives at least this many workgroups

__device__ __forceinline__ void rw_barrier() {
    // LDS stores and reads of this wave done, then the workgroup barrier
    // (no vmcnt wait: the weight loads of the next step stay in flight)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <uint32_t TT>
__global__ __launch_bounds__(RW_NT) void router_wide_kernel(const uint16_t *__restrict__ x16,
                                                            const float *__restrict__ w,
                                                            const float *__restrict__ bias,
                                                            float *__restrict__ proj, uint32_t rows, uint32_t d,
                                                            uint32_t cols, uint32_t cpad, uint32_t stride,
                                                            uint32_t nbias, uint32_t *zero_words, uint32_t n_zero,
                                                            const uint32_t *xscale) {
    constexpr uint32_t TOK = 16 * TT;
    __shared__ float4 xs[2][NQ][TT][RMDA_WAVE];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % RMDA_WAVE;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid / RMDA_WAVE);
    if (zero_words != nullptr && blockIdx.x == 0 && blockIdx.y == 0) {
        for (uint32_t i = tid; i < n_zero; i += RW_NT) {
            zero_words[i] = 0;
        }
    }
    const uint32_t L = d / NQ;
    const uint32_t nsub = L / 16;  // d % 128 == 0 is a launch condition
    const uint32_t t0 = blockIdx.x * TOK;
    const uint32_t kk = lane / 16;
    const uint32_t c = blockIdx.y * RW_COL + wv * 16 + lane % 16;  // < cpad: the grid covers whole 128-column blocks
    // weight float4 of chunk q, step s: steps 0..3 of lane (kk, column c)
    const float *wc = w + ((size_t)c * 4 + kk) * 4;
    const size_t wq = (size_t)nsub * cpad * 16;  // one chunk further
    const size_t ws = (size_t)cpad * 16;         // one 16-k step further

    // staging: thread tid takes the 8-element halves p = tid + r * RW_NT
    // (r < NH) of the step's 8 x TOK x 2 halves: chunk p / (2 TOK), token
    // (p % (2 TOK)) / 2, half p % 2 (k 8h .. 8h+7 of the step)
    constexpr uint32_t NH = NQ * TOK * 2 / RW_NT;
    static_assert(NH * RW_NT == NQ * TOK * 2, "whole halves per thread");
    const uint16_t *xsrc[NH];
    uint32_t xdst[NH];  // float index in xs[0] of the token's float4 for kk = 0, plus 2h
#pragma unroll
    for (uint32_t r = 0; r < NH; r += 1) {
        const uint32_t pc = tid + r * RW_NT;
        const uint32_t q = pc / (2 * TOK);
        const uint32_t tok = (pc % (2 * TOK)) / 2;
        const uint32_t h = pc % 2;
        const uint32_t row = t0 + tok < rows ? t0 + tok : rows - 1;  // rows past the matrix: never stored
        xsrc[r] = x16 + (size_t)row * d + q * L + 8 * h;
        xdst[r] = ((q * TT + tok / 16) * RMDA_WAVE + tok % 16) * 4 + 2 * h;
    }
    float *const xsf = reinterpret_cast<float *>(&xs[0][0][0][0]);
    constexpr uint32_t XBUF = NQ * TT * RMDA_WAVE * 4;  // floats per buffer
    uint4 xv[NH];
    auto load_x = [&](uint32_t s) {
#pragma unroll
        for (uint32_t r = 0; r < NH; r += 1) {
            xv[r] = *reinterpret_cast<const uint4 *>(xsrc[r] + (size_t)s * 16);
        }
    };
    // element o of a half is k offset 8h + o: kk = o % 4, step 2h + o / 4
    auto store_x = [&](uint32_t buf) {
#pragma unroll
        for (uint32_t r = 0; r < NH; r += 1) {
            const uint32_t u[4] = {xv[r].x, xv[r].y, xv[r].z, xv[r].w};
#pragma unroll
            for (uint32_t k4 = 0; k4 < 4; k4 += 1) {
                // o = k4 and o = k4 + 4: words k4 / 2 and 2 + k4 / 2, half k4 % 2
                const uint32_t lo = u[k4 / 2];
                const uint32_t hi = u[2 + k4 / 2];
                const float a = (k4 % 2) ? h_hi(lo) : h_lo(lo);
                const float b = (k4 % 2) ? h_hi(hi) : h_lo(hi);
                *reinterpret_cast<float2 *>(xsf + buf * XBUF + xdst[r] + k4 * 16 * 4) = make_float2(a, b);
            }
        }
    };

    rmda_f32x4 acc[TT][NQ];
#pragma unroll
    for (uint32_t tt = 0; tt < TT; tt += 1) {
#pragma unroll
        for (uint32_t q = 0; q < NQ; q += 1) {
            acc[tt][q] = rmda_f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    // weights in two register sets that trade roles every step (a step
    // multiplies with one and fills the other for the next step), so no
    // register copies, and no wait for the loads in flight, sit at the loop's
    // back edge
    float4 wa[NQ], wn[NQ];
#pragma unroll
    for (uint32_t q = 0; q < NQ; q += 1) {
        wa[q] = *reinterpret_cast<const float4 *>(wc + q * wq);
    }
    load_x(0);
    store_x(0);
    rw_barrier();
    // Every step issues the same loads (the last one re-reads its own step,
    // in bounds, and stores it to the idle buffer, never read), so the
    // compiler's vmcnt waits count the weight loads a full step ahead.  The
    // scheduling fences keep the issue order as written: the next step's
    // activation loads first, then per chunk its fragment reads, MFMAs and
    // the next step's weight load (left to itself the compiler sinks the
    // loads to the end of the step and then waits for them there).
    auto step = [&](uint32_t s, float4 (&wcur)[NQ], float4 (&wnext)[NQ]) __attribute__((always_inline)) {
        const uint32_t buf = s % 2;
        const uint32_t sn = s + 1 < nsub ? s + 1 : s;
        load_x(sn);
        __builtin_amdgcn_sched_barrier(0);
        const float4 *xa = &xs[buf][0][0][lane];
#pragma unroll
        for (uint32_t q = 0; q < NQ; q += 1) {
            float4 a[TT];
#pragma unroll
            for (uint32_t tt = 0; tt < TT; tt += 1) {
                a[tt] = xa[(q * TT + tt) * RMDA_WAVE];
            }
            const float4 bq = wcur[q];
            wnext[q] = *reinterpret_cast<const float4 *>(wc + q * wq + (size_t)sn * ws);
#pragma unroll
            for (uint32_t tt = 0; tt < TT; tt += 1) {
                acc[tt][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[tt].x, bq.x, acc[tt][q], 0, 0, 0);
            }
#pragma unroll
            for (uint32_t tt = 0; tt < TT; tt += 1) {
                acc[tt][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[tt].y, bq.y, acc[tt][q], 0, 0, 0);
            }
#pragma unroll
            for (uint32_t tt = 0; tt < TT; tt += 1) {
                acc[tt][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[tt].z, bq.z, acc[tt][q], 0, 0, 0);
            }
#pragma unroll
            for (uint32_t tt = 0; tt < TT; tt += 1) {
                acc[tt][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[tt].w, bq.w, acc[tt][q], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        store_x(1 - buf);  // the other buffer: every wave finished reading it before the last barrier
        rw_barrier();
    };
    uint32_t s = 0;
    for (; s + 1 < nsub; s += 2) {
        step(s, wa, wn);
        step(s + 1, wn, wa);
    }
    if (s < nsub) {
        step(s, wa, wn);
    }
    // D[4*kk + v][lane % 16] of token tile tt is token 16*tt + 4*kk + v
    const bool cok = c < cols;
    const float bv = bias != nullptr && c < nbias ? bias[c] : 0.0f;
    const float xinv = rmda_slot_inv(xscale);
#pragma unroll
    for (uint32_t tt = 0; tt < TT; tt += 1) {
#pragma unroll
        for (uint32_t v = 0; v < 4; v += 1) {
            float sum = acc[tt][0][v];
#pragma unroll
            for (uint32_t q = 1; q < NQ; q += 1) {
                sum = sum + acc[tt][q][v];
            }
            sum = sum * xinv;
            if (bias != nullptr && c < nbias) {
                sum = sum + bv;
            }
            const uint32_t t = t0 + 16 * tt + 4 * kk + v;
            if (t < rows && cok) {
                proj[(size_t)t * stride + c] = sum;
            }
        }
    }
}

// HF router weights [cols][d] -> packed [d/16][cpad][4][4]: element (k, c)
// at ((k/16)*cpad + c)*16 + (k%4)*4 + (k%16)/4, zero columns past `cols`.
// One thread per packed float; a one-time load-time reorder.
__global__ __launch_bounds__(256) void router_pack_kernel(const float *__restrict__ w, float *__restrict__ out,
                                                          uint32_t cols, uint32_t cpad, uint32_t d) {
    const size_t n = (size_t)d * cpad;
    for (size_t o = (size_t)blockIdx.x * 256 + threadIdx.x; o < n; o += (size_t)gridDim.x * 256) {
        const uint32_t j = (uint32_t)(o % 16);
        const uint32_t c = (uint32_t)((o / 16) % cpad);
        const uint32_t k = (uint32_t)(o / (16 * (size_t)cpad)) * 16 + (j % 4) * 4 + j / 4;
        out[o] = c < cols ? w[(size_t)c * d + k] : 0.0f;
    }
}

}  // namespace

uint32_t rmda_router_cpad(uint32_t cols) { return (cols + RMDA_WAVE - 1) / RMDA_WAVE * RMDA_WAVE; }

namespace {

// columns [col0, cols) of the 32 x 32 (or 16 x 16) tile
template <bool FUSE, int TT, int TPW>
void launch_mf_tile(hipStream_t s, uint32_t rows, uint32_t cols, bool w_packed, const uint16_t *x16, const float *w,
                    const float *bias, float *proj, uint32_t d, uint32_t cpad, uint32_t stride, uint32_t nbias,
                    uint32_t *zero_words, uint32_t n_zero, const rmda_route_fuse_t &fz, uint32_t col0,
                    const uint32_t *xscale) {
    const dim3 grid((rows + MF_TOK * TT - 1) / (MF_TOK * TT), FUSE ? 1 : (cols - col0 + 16 * TPW - 1) / (16 * TPW));
    const dim3 block(MF_NW * RMDA_WAVE);
    if (w_packed) {
        hipLaunchKernelGGL((router_mf_kernel<true, FUSE, TT, TPW>), grid, block, 0, s, x16, w, bias, proj, rows, d,
                           cols, cpad, stride, nbias, zero_words, n_zero, fz, col0, xscale);
    } else {
        hipLaunchKernelGGL((router_mf_kernel<false, FUSE, TT, TPW>), grid, block, 0, s, x16, w, bias, proj, rows, d,
                           cols, cpad, stride, nbias, zero_words, n_zero, fz, col0, xscale);
    }
}

template <bool FUSE>
void launch_mf(hipStream_t s, uint32_t rows, uint32_t cols, bool w_packed, const uint16_t *x16, const float *w,
               const float *bias, float *proj, uint32_t d, uint32_t cpad, uint32_t stride, uint32_t nbias,
               uint32_t *zero_words, uint32_t n_zero, const rmda_route_fuse_t &fz, const uint32_t *xscale) {
    uint32_t col0 = 0;
    if (!FUSE && w_packed) {
        // the wide tile takes whole 128-column blocks when they give the GPU
        // enough workgroups; the columns past them (the shared-expert gate)
        // go to the tile below
        // (64-token workgroups, or 32-token ones when those are too few: the
        // teacher's T = 2048 x 512 experts, 71.5 us on the 32 x 32 tile ->
        // 53.9 us)
        const uint32_t nbw = cols / RW_COL;
        const bool w64 = (rows + 63) / 64 * nbw >= RW_MIN_WGS;
        const bool w32 = !w64 && (rows + 31) / 32 * nbw >= RW_MIN_WGS;
        if (nbw > 0 && (w64 || w32)) {
            if (w64) {
                hipLaunchKernelGGL(router_wide_kernel<4>, dim3((rows + 63) / 64, nbw), dim3(RW_NT), 0, s, x16, w,
                                   bias, proj, rows, d, cols, cpad, stride, nbias, zero_words, n_zero, xscale);
            } else {
                hipLaunchKernelGGL(router_wide_kernel<2>, dim3((rows + 31) / 32, nbw), dim3(RW_NT), 0, s, x16, w,
                                   bias, proj, rows, d, cols, cpad, stride, nbias, zero_words, n_zero, xscale);
            }
            col0 = nbw * RW_COL;
            zero_words = nullptr;
            if (col0 == cols) {
                return;
            }
        }
    }
    const uint32_t wgs = (rows + MF_TOK * MF_TT - 1) / (MF_TOK * MF_TT) *
                         (FUSE ? 1u : (cols - col0 + MF_NCOL - 1) / MF_NCOL);
    // a remainder of at most 16 columns (the shared gate) takes 16-column
    // workgroups: a 32-column one would do twice the work for dead columns
    const bool small = (wgs < MF_MIN_WGS || (col0 > 0 && cols - col0 <= 16u * MF_TPW_SMALL)) &&
                       (!FUSE || cols <= 16u * MF_TPW_SMALL);
    if (small) {
        launch_mf_tile<FUSE, MF_TT_SMALL, MF_TPW_SMALL>(s, rows, cols, w_packed, x16, w, bias, proj, d, cpad, stride,
                                                        nbias, zero_words, n_zero, fz, col0, xscale);
    } else {
        launch_mf_tile<FUSE, MF_TT, MF_TPW>(s, rows, cols, w_packed, x16, w, bias, proj, d, cpad, stride, nbias,
                                            zero_words, n_zero, fz, col0, xscale);
    }
}

}  // namespace

hipError_t rmda_launch_router(hipStream_t s, const uint16_t *x16, const float *w, int w_packed, const float *bias,
                              float *proj, uint32_t rows, uint32_t d, uint32_t cols, uint32_t stride,
                              uint32_t nbias, uint32_t *zero_words, uint32_t n_zero,
                              const rmda_route_fuse_t *fuse, const uint32_t *xscale) {
    const bool mf = d % 128 == 0 && rows > 0;
    if ((w_packed || fuse != nullptr || xscale != nullptr) && !mf) {
        return hipErrorInvalidValue;
    }
    if (fuse != nullptr && (fuse->experts > cols || cols > rmda_route_fuse_max_cols())) {
        return hipErrorInvalidValue;
    }
    if (mf) {
        const uint32_t cpad = rmda_router_cpad(cols);
        if (fuse != nullptr) {
            launch_mf<true>(s, rows, cols, w_packed, x16, w, bias, proj, d, cpad, stride, nbias, zero_words, n_zero,
                            *fuse, xscale);
        } else {
            launch_mf<false>(s, rows, cols, w_packed, x16, w, bias, proj, d, cpad, stride, nbias, zero_words, n_zero,
                             rmda_route_fuse_t{}, xscale);
        }
        return hipGetLastError();
    }
    dim3 grid((rows + TM - 1) / TM, (cols + TC - 1) / TC);
    if (rows == 0) {
        grid.x = 1;  // still run block (0,0) for the zero fill
    }
    hipLaunchKernelGGL(router_tile_kernel, grid, dim3(256), 0, s, x16, w, bias, proj, rows, d, cols, stride,
                       nbias, zero_words, n_zero);
    return hipGetLastError();
}

uint32_t rmda_route_fuse_max_cols() { return MF_NCOL; }

hipError_t rmda_launch_router_pack(hipStream_t s, const float *w, float *out, uint32_t cols, uint32_t d) {
    const uint32_t cpad = rmda_router_cpad(cols);
    const size_t n = (size_t)d * cpad;
    const uint32_t blocks = (uint32_t)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    hipLaunchKernelGGL(router_pack_kernel, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, s, w, out, cols, cpad, d);
    return hipGetLastError();
}
