// Shared device helpers and the launch interface between the C-ABI layer
// (api.hip) and the kernel files.  gfx950 only: wave64, fp16 MFMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/rmda_moe.h"

#define RMDA_WAVE 64

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

// qwen_elem op 0 (shader/qwen_elem.comp:20-31): silu(g) * u, one expression
// for every kernel that computes it, so they agree bit for bit
__device__ __forceinline__ float rmda_swiglu(float g, float u) {
    return g / (1.0f + expf(-g)) * u;
}

// The fused layer's SwiGLU, in the gate_up epilogue of both GEMM tiles (one
// expression, so the tiles agree bit for bit): the hardware exp and
// reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp each) in place of expf and
// the IEEE division, whose instruction sequences held the MFMA waves at every
// task's end (sustained: config 3 gate_up 156.0 -> 153.0-153.5 us, config 4
// 113.6 -> 109.3 us).  The result is rounded to fp16, so the difference is
// below the layer's tolerance; the reference-mode recording keeps
// rmda_swiglu.
__device__ __forceinline__ float rmda_swiglu_fast(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

__device__ __forceinline__ float rmda_h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint16_t rmda_f2h(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Device-scope (L2-coherent) load, for data another workgroup of the same
// grid wrote before a fence + atomic hand-off.
__device__ __forceinline__ uint32_t rmda_load_agent(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float rmda_sigmoidf(float v) {
    return 1.0f / (1.0f + expf(-v));
}

// One combine term over 8 consecutive columns: acc[v] += w * y[v] for the
// 8 fp16 values in q, as one fused multiply-add each.  The fused layer's
// combine kernel and the down GEMM's folded-in combine both sum through this,
// so their outputs agree bit for bit.
__device__ __forceinline__ void rmda_comb_acc8(float acc[8], float w, uint4 q) {
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int v = 0; v < 4; v += 1) {
        acc[2 * v] = __builtin_fmaf(w, rmda_h2f((uint16_t)(u[v] & 0xffffu)), acc[2 * v]);
        acc[2 * v + 1] = __builtin_fmaf(w, rmda_h2f((uint16_t)(u[v] >> 16)), acc[2 * v + 1]);
    }
}

// The hyper-connection update of one token's 8 columns in one stream:
// h[c + v] += acc[v] * gate (gate = 2 * sigmoid(inj / hc)), h 16-byte aligned.
__device__ __forceinline__ void rmda_hc_acc8(float *h, const float acc[8], float gate) {
    float4 *hp = reinterpret_cast<float4 *>(h);
    float4 a = hp[0];
    float4 b = hp[1];
    a.x = __builtin_fmaf(acc[0], gate, a.x);
    a.y = __builtin_fmaf(acc[1], gate, a.y);
    a.z = __builtin_fmaf(acc[2], gate, a.z);
    a.w = __builtin_fmaf(acc[3], gate, a.w);
    b.x = __builtin_fmaf(acc[4], gate, b.x);
    b.y = __builtin_fmaf(acc[5], gate, b.y);
    b.z = __builtin_fmaf(acc[6], gate, b.z);
    b.w = __builtin_fmaf(acc[7], gate, b.w);
    hp[0] = a;
    hp[1] = b;
}

__device__ __forceinline__ uint4 rmda_pack8_f16(const float acc[8]) {
    uint32_t u[4];
#pragma unroll
    for (int v = 0; v < 4; v += 1) {
        u[v] = (uint32_t)rmda_f2h(acc[2 * v]) | ((uint32_t)rmda_f2h(acc[2 * v + 1]) << 16);
    }
    return make_uint4(u[0], u[1], u[2], u[3]);
}

// Order-preserving map of a non-NaN float to uint32 (-0 and +0 map equal).
__device__ __forceinline__ uint32_t rmda_float_key(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    if ((u & 0x7fffffffu) == 0) {
        u = 0;
    }
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float rmda_key_float(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __builtin_bit_cast(float, u);
}

// Maximum (MAX) or minimum over the wave, returned to every lane; the whole
// wave must be active.  Register-only: DPP within each 16-lane row (swap
// neighbours, swap pairs, mirror halves, mirror the row), then
// v_permlane16_swap and v_permlane32_swap exchange rows and halves, so no
// step goes through the LDS pipeline the way a generic lane shuffle
// (ds_bpermute) does.
template <bool MAX>
__device__ __forceinline__ uint32_t rmda_wave_red_u32(uint32_t v) {
    auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0u, v, 0xB1, 0xF, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0u, v, 0x4E, 0xF, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0u, v, 0x141, 0xF, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0u, v, 0x140, 0xF, 0xF, false));
    {
        const auto x = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        v = op(x[0], x[1]);
    }
    {
        const auto x = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        v = op(x[0], x[1]);
    }
    return v;
}

// The reference's fp16 slot scale (shader/cast_f16.comp): a value cast with
// slot word amax is multiplied by 2^(141 - biased exponent of amax), or by 1
// when the slot word is zero, not finite or absent.  rmda_slot_inv is the
// factor that undoes it (a power of two, so exact for normal results), 1 for
// amax == NULL: the fused layer's epilogues multiply by it always, which
// leaves the unscaled path's bits unchanged.
// The slot word is read through the scalar cache (a constant-address-space
// load, counted by lgkmcnt), so the GEMM kernels' hand-counted vmcnt waits
// see nothing but their stage loads.
__device__ __forceinline__ float rmda_slot_inv(const uint32_t *amax) {
    if (amax == nullptr) {
        return 1.0f;
    }
    const uint32_t u = *(const __attribute__((address_space(4))) uint32_t *)amax;
    const float a = __builtin_bit_cast(float, u);
    if (!(a > 0.0f) || __builtin_isinf(a)) {
        return 1.0f;
    }
    return ldexpf(1.0f, (int)((u >> 23) & 0xffu) - 141);
}

// The slot-scaled mode's fp16 expert rows (packed weights).  bound is the
// down weights' largest row sum of |w| (rows whose sum is not finite left
// out), written when the weights are packed.  A SwiGLU output cast with its
// slot is below 2^15 in magnitude, so every down product hp16 . w is below
// 2^15 * bound; multiplied by rmda_ye_mul(bound) = 2^-c with 2^c > bound
// (c >= 0) it stays below 2^15 and fits fp16 with fp16's relative
// precision.  The combine multiplies it back by 2^c (exact: a power of two).
// Read through the scalar cache, as rmda_slot_inv.
__device__ __forceinline__ float rmda_ye_mul(const uint32_t *bound) {
    const uint32_t u = *(const __attribute__((address_space(4))) uint32_t *)bound;
    const uint32_t e = (u >> 23) & 0xffu;  // bound in [2^(e-127), 2^(e-126))
    if (e < 127u || e == 0xffu) {
        return 1.0f;  // below 1 (c = 0), or not finite
    }
    return ldexpf(1.0f, 126 - (int)e);
}

// The slot-scaled mode's SwiGLU absmax is gathered in RMDA_AMAX_PARTS partial
// words, RMDA_AMAX_STRIDE words apart (one 128-byte line each), which the hp
// cast folds, so that the GEMM waves' device-scope atomics spread over 64
// lines instead of queueing on one word.
#define RMDA_AMAX_PARTS 64u
#define RMDA_AMAX_STRIDE 32u
#define RMDA_AMAX_BYTES (RMDA_AMAX_PARTS * RMDA_AMAX_STRIDE * 4u)

// A wave's largest |v| into its partial word of parts (absmax.comp's
// atomicMax on the float bits of non-negative values; each lane passes fmaxf
// over its values, so NaN is skipped as absmax_kernel skips it).  Called once
// per wave at the end of a persistent kernel, with the lane's maximum over
// all its tasks.  The whole wave must be active.
__device__ __forceinline__ void rmda_wave_amax(uint32_t *parts, float m) {
    const uint32_t r = rmda_wave_red_u32<true>(__builtin_bit_cast(uint32_t, m));
    if (threadIdx.x % RMDA_WAVE == 0) {
        const uint32_t part = (blockIdx.x * 13u + threadIdx.x / RMDA_WAVE) % RMDA_AMAX_PARTS;
        atomicMax(parts + part * RMDA_AMAX_STRIDE, r);
    }
}

// Top-k of one row of logits by one wave (shader/moe_route.comp:20-61),
// as rmda_route_row = rmda_route_load (the row into registers) then
// rmda_route_select (the rounds):
// topk rounds, each taking the largest untaken logit by strict '>' from
// -3.0e38, so the lowest column wins ties and NaN / values <= -3e38 are never
// taken; idx in selection order; z = sum_k exp(l_k - l_0) summed in
// selection order; wt_k = exp(l_k - l_0) / z; count[e] += 1 per selection
// when count != NULL.  Lane l holds columns l, l+64, ...; a round is one
// lane-local scan, one wave-wide max of the order-preserving float key and
// the lowest column among the lanes holding that maximum.  AGENT: read the logits
// with device-scope loads (rows written by other workgroups of the running
// kernel).
template <int NV, bool AGENT>
__device__ __forceinline__ void rmda_route_load(const float *l, uint32_t experts, float (&v)[NV]) {
    const uint32_t lane = threadIdx.x % RMDA_WAVE;
#pragma unroll
    for (int j = 0; j < NV; j += 1) {
        const uint32_t c = lane + RMDA_WAVE * j;
        if (c < experts) {
            v[j] = AGENT ? __builtin_bit_cast(float, rmda_load_agent(reinterpret_cast<const uint32_t *>(l) + c))
                         : l[c];
        } else {
            v[j] = -3.0e38f;  // -3e38 is never selectable
        }
    }
}

// The selection rounds of rmda_route_row on values already in registers
// (lane l holds columns l, l+64, ...).  sel_row, when not NULL, receives the
// selected columns as well (e.g. an LDS copy for the caller's next step);
// AGENT_IDX stores idx_row at device scope.
template <int NV, bool AGENT_IDX = false>
__device__ __forceinline__ void rmda_route_select(const float (&v)[NV], uint32_t topk, uint32_t *idx_row,
                                                  float *wt_row, uint32_t *count, uint32_t *sel_row) {
    const uint32_t lane = threadIdx.x % RMDA_WAVE;
    uint32_t taken = 0;
    // lane k keeps round k's selection; z is summed after the rounds, still
    // in selection order
    float sv0 = 0.0f;
    uint32_t my_sel = RMDA_NONE;
    float my_val = 0.0f;
    for (uint32_t k = 0; k < topk; k += 1) {
        float lb = -3.0e38f;
        int lv = -1;
#pragma unroll
        for (int j = 0; j < NV; j += 1) {
            if (((taken >> j) & 1u) == 0 && v[j] > lb) {
                lb = v[j];
                lv = j;
            }
        }
        // the largest value over the wave (a selectable value's key is
        // never 0), then the lowest column holding it: the column of the
        // one lane holding it, or, on a tie across lanes, the least of the
        // tied lanes' columns (each lane's scan already kept its lowest)
        const uint32_t k32 = lv >= 0 ? rmda_float_key(lb) : 0u;
        const uint32_t m32 = rmda_wave_red_u32<true>(k32);
        uint32_t col = RMDA_NONE;
        float val = -3.0e38f;
        if (m32 != 0) {
            const uint32_t mine = lane + RMDA_WAVE * (uint32_t)lv;
            const uint64_t tied = __ballot(k32 == m32);
            if (__popcll(tied) == 1) {
                col = __builtin_amdgcn_readlane(mine, (uint32_t)__ffsll((unsigned long long)tied) - 1u);
            } else {
                col = rmda_wave_red_u32<false>(k32 == m32 ? mine : 0xffffffffu);
            }
            val = rmda_key_float(m32);
            if (col % RMDA_WAVE == lane) {
                taken |= 1u << (col / RMDA_WAVE);
            }
        }
        if (k == 0) {
            sv0 = val;
        }
        if (lane == k) {
            my_sel = col;
            my_val = val;
        }
    }
    // exp(l_k - l_0) once, on lane k, instead of by every lane in every
    // round; z = ((e_0 + e_1) + e_2) + ... as the rounds added it
    const float e = expf(my_val - sv0);
    float z = 0.0f;
    for (uint32_t k = 0; k < topk; k += 1) {
        z = z + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), (int)k));
    }
    if (lane < topk) {
        if (AGENT_IDX) {
            // read back by another workgroup of the same launch
            __hip_atomic_store(&idx_row[lane], my_sel, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            idx_row[lane] = my_sel;
        }
        wt_row[lane] = e / z;
        if (sel_row != nullptr) {
            sel_row[lane] = my_sel;
        }
        if (count != nullptr && my_sel != RMDA_NONE) {
            atomicAdd(&count[my_sel], 1u);
        }
    }
}

template <int NV, bool AGENT>
__device__ __forceinline__ void rmda_route_row(const float *l, uint32_t experts, uint32_t topk,
                                               uint32_t *idx_row, float *wt_row, uint32_t *count) {
    float v[NV];
    rmda_route_load<NV, AGENT>(l, experts, v);
    rmda_route_select<NV>(v, topk, idx_row, wt_row, count, nullptr);
}

// Router kernel with the top-k fused in: when one workgroup's column slice
// covers the row (cols <= rmda_route_fuse_max_cols()), it routes its
// tokens from LDS.
struct rmda_route_fuse_t {
    uint32_t experts;
    uint32_t topk;
    uint32_t *idx;       // [rows][topk]
    float *wt;           // [rows][topk]
};
uint32_t rmda_route_fuse_max_cols();

// ---- launch helpers implemented by the kernel files ----
// Every launcher validates nothing: api.hip checks shapes first.  They return
// hipGetLastError() after the launch.

// router.hip
// xscale (or NULL): the slot word x16 was cast with; each logit's chunk sum
// is multiplied by rmda_slot_inv(xscale) before the bias is added (packed or
// HF-layout tiles for d % 128 == 0 only).
hipError_t rmda_launch_router(hipStream_t s, const uint16_t *x16, const float *w, int w_packed, const float *bias,
                              float *proj, uint32_t rows, uint32_t d, uint32_t cols, uint32_t stride,
                              uint32_t nbias, uint32_t *zero_words, uint32_t n_zero,
                              const rmda_route_fuse_t *fuse, const uint32_t *xscale = nullptr);
// Packed router weights: [d/16][rmda_router_cpad(cols)][4][4] fp32, element
// (k, c) at ((k/16)*cpad + c)*16 + (k%4)*4 + (k%16)/4.
uint32_t rmda_router_cpad(uint32_t cols);
hipError_t rmda_launch_router_pack(hipStream_t s, const float *w, float *out, uint32_t cols, uint32_t d);

// route.hip: top-k per row; count gets atomic adds (caller zeroes it first).
hipError_t rmda_launch_route(hipStream_t s, const float *proj, uint32_t *idx, float *wt,
                             uint32_t *count, uint32_t rows, uint32_t experts, uint32_t topk,
                             uint32_t stride);

// scan.hip
hipError_t rmda_launch_zero(hipStream_t s, uint32_t *p, size_t n, uint32_t value);
hipError_t rmda_launch_scan(hipStream_t s, const uint32_t *count, uint32_t *off, uint32_t *tiles,
                            uint32_t n_tiles, uint32_t experts, uint32_t tile);

// Ranking for the stable permutation.  Pairs are cut into blocks of
// RMDA_RANK_BLOCK; lrank = rank of the pair among equal experts inside its
// block, hist[b][e] = the block's per-expert count.  The last block to finish
// turns hist into base offsets (boff[b][e] = off[e] + sum_{b'<b} hist[b'][e]),
// writes off/count, and, when items != NULL, the grouped-GEMM work list.
#define RMDA_RANK_BLOCK 1024u
struct rmda_rank_args_t {
    const uint32_t *idx;
    uint32_t npairs;
    uint32_t experts;
    uint32_t tile;      // segment padding P for off
    uint32_t *lrank;    // [npairs]
    uint32_t *hist;     // [nblocks][experts], becomes boff in place
    uint32_t *count;    // [experts] out, or NULL
    uint32_t *off;      // [experts] out, or NULL
    const uint32_t *off_in; // [experts] caller's offsets (then tile is unused), or NULL
    uint32_t *done;     // one word, zero on entry; left zero, except by a routed
                        // launch (route_proj), which leaves its grid size there
    // work list (optional)
    uint32_t *items;    // uint4 per item {expert, row0, rows, 0}
    uint32_t *n_items;  // one word
    uint32_t bm;        // rows per work item
    // load-bucket tile choice (optional): when n_items_hot != NULL and the
    // experts with >= hot_min rows hold at least half of all rows, the list
    // is cut into bm_hot-row items counted in *n_items_hot (and *n_items = 0),
    // else into bm-row items (and *n_items_hot = 0)
    uint32_t *n_items_hot;
    uint32_t bm_hot;
    uint32_t hot_min;
    uint32_t force;       // 0: the choice above; 1: always bm items; 2: always bm_hot items
    uint32_t *hint_out;   // or NULL: receives the choice above (1 = bm, 2 = bm_hot),
                          // a host-visible word written with a system-scope store
    uint32_t shared_rows; // rows of the shared-expert group (0 = none)
    uint32_t shared_row0; // sorted-row base of the shared group
    // permutation written by the kernel itself when all pairs fit one rank
    // block (npairs <= RMDA_RANK_BLOCK); ignored otherwise
    uint32_t *slot;     // [npairs], or NULL
    uint32_t *rowtok;   // [sorted rows] row -> token, or NULL
    uint32_t topk;
    // nonzero: every block counts all npairs itself (LDS histograms of the
    // pairs before and after it), so no block waits for another, the blocks
    // write slot/rowtok themselves (slot must be set), block 0 writes
    // count/off/the work list, and hist/done are not used.  O(npairs) L2
    // reads per block: for npairs <= RMDA_RANK_ALL_MAX; idx 16-byte aligned.
    uint32_t count_all;
    // folded combine (optional): fc_cnt[t][b] = has_shared + the number of
    // selectable pairs of token t, for every b < fc_nblk; a token with no
    // rows at all gets a zero row in fc_zero_out (when not NULL), the value
    // the combine would write.  idx holds fc_rows * topk pairs.
    uint32_t *fc_cnt;
    uint32_t fc_nblk;
    uint32_t fc_rows;
    uint32_t fc_shared;
    uint16_t *fc_zero_out;
    uint32_t fc_d;
    // top-k folded in (optional; done zero on entry; npairs <= RMDA_RANK_BLOCK,
    // or count_all with slot set and 16-byte aligned idx): one block per 8
    // rows routes route_rows rows of logits (route_proj, row stride
    // route_stride) as route_kernel does, into route_idx (which must be idx)
    // and route_wt; the last ceil(npairs / RMDA_RANK_BLOCK) of them to finish
    // rank
    const float *route_proj;
    uint32_t route_rows;
    uint32_t route_stride;
    uint32_t *route_idx;
    float *route_wt;
};
#define RMDA_RANK_ALL_MAX (1u << 16)
hipError_t rmda_launch_rank(hipStream_t s, const rmda_rank_args_t *a);
// scan.hip: count[e] = |{pr < npairs : idx[pr] == e}| in one workgroup (an
// LDS histogram); for up to RMDA_COUNT1_MAX_PAIRS pairs
#define RMDA_COUNT1_MAX_PAIRS (1u << 16)
hipError_t rmda_launch_count(hipStream_t s, const uint32_t *idx, uint32_t npairs, uint32_t experts,
                             uint32_t *count);

// scatter.hip: slot[pr] = boff[pr/BLOCK][e] + lrank[pr]; optional row copy
// (xp) and inverse map (rowtok[slot] = token).
hipError_t rmda_launch_permute(hipStream_t s, const uint32_t *idx, const uint32_t *lrank,
                               const uint32_t *boff, uint32_t npairs, uint32_t topk,
                               uint32_t experts, uint32_t *slot, uint32_t *rowtok,
                               const uint16_t *x16, uint16_t *xp, uint32_t d8);
// scatter.hip: the drop-in scatter with row copy in one launch (each block
// counts the pairs before its own); O(npairs^2) L2 reads in all, so bounded.
#define RMDA_SCATTER1_MAX_PAIRS (1u << 16)
hipError_t rmda_launch_scatter1(hipStream_t s, const uint32_t *idx, const uint32_t *off, uint32_t *fill,
                                uint32_t rows, uint32_t topk, uint32_t experts, uint32_t *slot,
                                const uint16_t *x16, uint16_t *xp, uint32_t d8);

// gemm.hip: grouped GEMM over a device work list.
enum {
    RMDA_GEMM_SWIGLU = 0, // gate_up: A rows gathered via rowtok, out fp16 silu(g)*u
    RMDA_GEMM_F16 = 1,    // down: A rows direct, out fp16
    RMDA_GEMM_F32 = 2     // reference matmul_f16_moe: A rows direct, out fp32 * scale
};
// hyper-connection epilogue of the fused combine (h == NULL: none)
struct rmda_hc_t {
    float *h;
    const float *inj;
    uint32_t inj_stride;
    uint32_t inj_off;
    uint32_t hc;
};
#define RMDA_MAX_HC 8u

// The combine folded into the down GEMM (F16 mode, streaming tile).  cnt
// holds one arrival counter per (token, 64 output columns), preset by the
// rank kernel to the number of rows the token sends through the down GEMM
// (its selected experts, plus the shared expert's row).  A wave that has
// stored its 64 columns of a row takes one from the row's counter; the wave
// that takes the last one sums the token's rows for those 64 columns in j
// order, then the sigmoid-gated shared row, as the combine kernel does.
#define RMDA_FC_COLS 64u
struct rmda_fc_t {
    uint32_t *cnt;           // [rows][nblk], or NULL: no folded combine
    uint32_t nblk;           // d / RMDA_FC_COLS
    const uint32_t *rowtok;  // sorted row -> token (routed rows)
    const uint32_t *slot;    // [rows][topk]
    const float *wt;         // [rows][topk]
    const float *proj;       // router logits: the shared gate at [r * pstride + sg_off]
    uint32_t pstride;
    uint32_t sg_off;
    uint32_t topk;
    uint32_t has_shared;
    uint16_t *out;           // [rows][d] fp16, or NULL
    rmda_hc_t hc;            // hc.h != NULL: hyper-connection streams
};

struct rmda_gemm_args_t {
    int mode;
    const uint16_t *a;        // A base
    const uint32_t *rowtok;   // SWIGLU: sorted row -> token
    uint32_t a_rows;          // SWIGLU: rows of A; a gathered token index is clamped below it
    uint32_t lda;             // elements
    const uint16_t *w;        // [groups][n_w][k]
    const uint16_t *w_shared; // group == shared_group uses this [n_w][k]
    uint32_t shared_group;    // RMDA_NONE if none
    uint32_t shared_row0;     // SWIGLU: token = row - shared_row0 for the shared group
    uint32_t n_w;             // rows of one group's weight matrix
    uint32_t k;
    uint32_t n_out;           // output columns (SWIGLU: inter; else n_w)
    uint32_t inter;           // SWIGLU: up rows start at inter
    void *out;
    uint32_t ldo;             // elements
    const uint32_t *items;    // uint4 {group, row0, rows, 0}
    const uint32_t *n_items;  // device word, or NULL: use max_items
    uint32_t max_items;       // grid bound
    const uint32_t *tiles;    // F32 mode: reference tile map instead of items
    // F32 mode, optional (NULL: every row of a named tile): the segments'
    // offsets and row counts; rows r of tile t at or past off[e] + count[e]
    // (e = tiles[t]) are then neither computed nor stored
    const uint32_t *live_off;
    const uint32_t *live_count;
    // F32 mode, optional: out is silu(C[:, j]) * C[:, n_w/2 + j] (qwen_elem
    // op 0 on C) as [m][n_w/2] fp32, and amax[so] takes the absmax of what is
    // stored (atomicMax of the bits, as rmda_launch_elem_absmax); needs the
    // persistent kernel (rmda_ref_mm_supported) and n_w % 256 == 0
    int f32_swiglu;
    uint32_t so;
    const uint32_t *amax;
    uint32_t sa, sb;
    rmda_fc_t fc;             // F16 mode: the folded-in combine (fc.cnt == NULL: none)
    // The fused layer's slot-scaled mode (fp32 activations; all NULL
    // otherwise).  SWIGLU: g and u are multiplied by rmda_slot_inv(xscale)
    // before SiLU, and with hp32 set the SwiGLU output goes to hp32 as fp32
    // (same blocked index as the fp16 hp) instead of fp16 to out, and its
    // absmax into the partial words hp_amax (RMDA_AMAX_BYTES, zeroed before).  F16, one of: ye32 set, the
    // output is multiplied by rmda_slot_inv(yscale) and stored to ye32 as
    // fp32; ye_bound set (packed weights' row-sum bound word), it is
    // multiplied by rmda_ye_mul(ye_bound) and stored as fp16 to out.
    const uint32_t *xscale;
    float *hp32;
    uint32_t *hp_amax;
    const uint32_t *yscale;
    float *ye32;
    const uint32_t *ye_bound;
    // F16, fp16 rows, packed weights: non-zero asks for non-temporal row
    // stores (both tiles' default configurations)
    uint32_t ye_nt;
};
hipError_t rmda_launch_gemm(hipStream_t s, const rmda_gemm_args_t *a);
// gemm_ref.hip: the F32 (reference matmul_f16_moe) contract on the
// persistent LDS-DMA pipeline, for n % 256 == 0, k % 64 == 0 and at most
// 4096 row tiles; rmda_launch_gemm covers the rest.
bool rmda_ref_mm_supported(const rmda_gemm_args_t *a);
hipError_t rmda_launch_ref_mm(hipStream_t s, const rmda_gemm_args_t *a, uint32_t grid);
#define RMDA_GEMM_BM 128u

// gemm2.hip: the fused layer's grouped GEMM (SWIGLU and F16 modes) over
// work items of up to RMDA_GEMM2_BM rows, reading HF-layout or packed
// weights.  A configuration is (N tile, K step, pipeline depth); variant
// numbers name the ones built (rmda_gemm2_variant; 0 = default).  Requires
// n_w % 128 == 0 and k % bk == 0.
#define RMDA_GEMM2_BM 192u
// The rank kernel sorts the work list by rows in 16-row classes
#define RMDA_ITEM_CLASSES 16u
static_assert(RMDA_GEMM2_BM <= 16u * RMDA_ITEM_CLASSES, "work-item row classes");
struct rmda_gemm2_cfg_t {
    uint32_t bn;
    uint32_t bk;
    uint32_t stages;
    uint32_t grid;  // persistent workgroups (the device's CU count)
    uint32_t bpol;  // cache-policy bits of the weight (B) loads: 2 = non-temporal (streamed once)
    uint32_t spec;  // dedicated load-issue waves (0: every MFMA wave issues its share)
};
// rows of padding after the gathered-row index buffer (rowtok) that the
// grouped GEMM's scalar index reads may touch
#define RMDA_ROWTOK_PAD 256u
// The fused layer's sorted rows: every expert segment (and the shared
// expert's rows) starts at a multiple of RMDA_HP_ROWS, and the gate_up output
// hp is stored in 1 KiB blocks of RMDA_HP_ROWS rows x 32 columns: element
// (row R, column c) of an I-column hp at
//   ((R / 16) * (I / 32) + c / 32) * 512 + (R % 16) * 32 + c % 32,
// so the down GEMM loads a 16-row x 32-k tile of it as one contiguous KiB.
#define RMDA_HP_ROWS 16u
__host__ __device__ __forceinline__ size_t rmda_hp_index(uint32_t row, uint32_t col, uint32_t inter) {
    return ((size_t)(row / 16) * (inter / 32) + col / 32) * 512 + (row % 16) * 32 + col % 32;
}
rmda_gemm2_cfg_t rmda_gemm2_variant(int variant);
// gemm_hot.hip: the compute tile for hot experts, over work items of up to
// RMDA_GEMM_HOT_BM rows (packed weights only; same modes and bits as gemm2).
// An expert is hot when it receives at least RMDA_GEMM_HOT_MIN rows.
#define RMDA_GEMM_HOT_BM 256u
#define RMDA_GEMM_HOT_MIN 256u
static_assert(RMDA_GEMM_HOT_BM <= 16u * RMDA_ITEM_CLASSES && RMDA_GEMM_HOT_BM <= RMDA_ROWTOK_PAD,
              "hot work items: row classes and the rowtok padding its gathers may read");
// stages: LDS ring depth (4 or 5); sched: 0 = task_sched_t, 1 = chunk_sched_t
hipError_t rmda_launch_gemm_hot(hipStream_t s, const rmda_gemm_args_t *a, uint32_t grid, int stages, int sched);
hipError_t rmda_launch_gemm2(hipStream_t s, const rmda_gemm_args_t *a, rmda_gemm2_cfg_t c, int packed);
// Reorder `groups` row-major [n_w][k] matrices (fp16, or bf16 when bf16_in)
// into the packed slab order of K step bk (SWIGLU: gate/up interleave).
hipError_t rmda_launch_pack(hipStream_t s, const uint16_t *src, uint16_t *dst, uint32_t groups, uint32_t n_w,
                            uint32_t k, uint32_t inter, int swiglu, int bk, int bf16_in);
// The largest row sum of |w| over `groups` packed (non-SwiGLU) matrices
// [n_w][k] of K step bk, rows whose sum is not finite left out, atomicMax'ed
// as float bits into *bound (which the caller zeroes first).
hipError_t rmda_launch_row_abs_max(hipStream_t s, const uint16_t *packed, uint32_t groups, uint32_t n_w, uint32_t k,
                                   int bk, uint32_t *bound);

// combine.hip
hipError_t rmda_launch_combine(hipStream_t s, const rmda_pc_moe_combine_t *pc, const float *wt,
                               const uint32_t *slot, const float *y, const float *proj,
                               const float *sh, const float *inj, float *h, uint16_t *out);
// fused-layer combine: y fp16 rows, optional shared rows at shared_row0 + r.
// run_if (or NULL): the kernel returns at once unless *run_if != 0 (the
// layer passes the compute tile's item count when the down GEMM may have
// folded the combine in).  yscale and ybound (or NULL): the slot-scaled
// mode's fp16 rows, which stand for y * rmda_slot_inv(yscale) /
// rmda_ye_mul(ybound); the weights are multiplied by that power of two.
hipError_t rmda_launch_combine16(hipStream_t s, const float *wt, const uint32_t *slot,
                                 const uint16_t *y, const float *proj, uint32_t pstride,
                                 uint32_t sg_off, uint32_t shared_row0, int has_shared,
                                 uint16_t *out, uint32_t rows, uint32_t d, uint32_t topk,
                                 const rmda_hc_t *hc, const uint32_t *run_if, const uint32_t *yscale = nullptr,
                                 const uint32_t *ybound = nullptr);

// elem.hip
hipError_t rmda_launch_elem(hipStream_t s, const rmda_pc_qwen_elem_t *pc, const float *a, float *y);
hipError_t rmda_launch_absmax(hipStream_t s, const rmda_pc_absmax_t *pc, const float *x, uint32_t *amax);
// elem op 0 with the absmax of its output folded in (amax[slot] as
// rmda_launch_absmax would leave it over y)
hipError_t rmda_launch_elem_absmax(hipStream_t s, const rmda_pc_qwen_elem_t *pc, const float *a, float *y,
                                   uint32_t *amax, uint32_t slot);
// Rows of a P-padded permuted row space (moe_scan's segments) that hold
// routed pairs: row r is live when e = tiles[r / tile] names an expert and
// r - off[e] < count[e].  The recording's SwiGLU, absmax and cast skip the
// padding rows with it (their absmax is 0, the zero rows' own value).
struct rmda_rowmask_t {
    const uint32_t *tiles;
    const uint32_t *off;
    const uint32_t *count;
    uint32_t tile;
};
// elem op 0 + absmax, and the scaled cast, over the live rows only (other
// rows of y / dst are left as they were); rows of whole float4s
hipError_t rmda_launch_elem_absmax_rows(hipStream_t s, const rmda_pc_qwen_elem_t *pc, const float *a, float *y,
                                        uint32_t *amax, uint32_t slot, const rmda_rowmask_t *mask);
hipError_t rmda_launch_cast_rows(hipStream_t s, uint32_t rows, uint32_t n, const float *src, uint16_t *dst,
                                 const uint32_t *amax, uint32_t slot, const rmda_rowmask_t *mask);
hipError_t rmda_launch_cast(hipStream_t s, const rmda_pc_cast_t *pc, const float *src, uint16_t *dst,
                            const uint32_t *amax);
hipError_t rmda_launch_bf16(hipStream_t s, uint32_t n, uint32_t *w);
hipError_t rmda_launch_fill_normal(hipStream_t s, void *dst, size_t n, int f16, uint64_t stream,
                                   uint64_t seed, float std);
// The fused layer's fp32-activation input, in two launches (the reference's
// absmax.comp + cast_f16.comp with a fresh slot, src/qwen.c:517-539, with no
// zero-filled slot word needed beforehand): part[b] = the absmax bits of
// block b's share of x (nparts blocks), then every block folds the parts,
// casts its share of x with the slot scale into x16, and block 0 stores the
// absmax to *x_slot and zeroes the RMDA_AMAX_PARTS partial words at
// hp_parts.  n % 4 == 0, x and x16 16-byte aligned.
#define RMDA_XCAST_PARTS 256u
hipError_t rmda_launch_x_absmax(hipStream_t s, const float *x, size_t n, uint32_t *part);
hipError_t rmda_launch_x_cast(hipStream_t s, const float *x, size_t n, const uint32_t *part, uint16_t *x16,
                              uint32_t *x_slot, uint32_t *hp_parts);
// hp16[i] = fp16(hp32[i] * scale(amax)) over the blocked hp of the slot-scaled
// mode, for the routed rows [0, off[E-1] + count[E-1] rounded up to 16) and,
// when sh_rows > 0, the shared expert's rows [sh_row0, sh_row0 + sh_rows
// rounded up to 16); inter % 4 == 0.  amax is the fold of the partial words
// at hp_parts, which block 0 also stores to *slot for the down GEMM.
hipError_t rmda_launch_hp_cast(hipStream_t s, const float *hp32, uint16_t *hp16, const uint32_t *hp_parts,
                               uint32_t *slot, const uint32_t *off, const uint32_t *count, uint32_t experts,
                               uint32_t inter, uint32_t sh_row0, uint32_t sh_rows);
