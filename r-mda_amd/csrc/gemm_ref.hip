// The reference's grouped GEMM contract (matmul_f16_moe, rmda_moe_mm) on the
// LDS-DMA pipeline: C[m][n] = A[m]·B[tiles[m/128]][n]ᵀ / (scale(sa)·scale(sb))
// for every 128-row tile t of A whose tiles[t] names an expert
// (shader/matmul_f16_moe.comp:70-126, src/qwen.c:770-786).  A is the
// permuted activation copy xp [m][k] and B the HF-layout expert weights
// [E][n][k], both fp16 row-major, C fp32.
//
//   * Persistent: one 768-thread workgroup per CU walks tasks (valid tile,
//     256-column N tile).  Each workgroup first compacts the valid tiles of
//     tiles[] into LDS, so tiles marked RMDA_NONE cost nothing and any order
//     of tiles[] is accepted; tasks are dealt to the XCDs in contiguous runs
//     (chunk_sched_t), so the N tiles of a row tile and the tiles of one
//     expert meet in one L2 and its weight lines are fetched from HBM once.
//   * K step 64: every A row and every weight row of a stage is one whole
//     128-byte line (the HF layout read 32 halves at a time would split each
//     line over two stages).  A (128 x 64) and B (256 x 64) go straight into
//     LDS with global_load_lds_dwordx4 through a 3-stage ring of 48 KiB; a
//     row's 16-byte chunk c sits at slot c ^ ((r >> 1) & 7), which keeps the
//     16-lane fragment reads free of bank conflicts.
//   * A task's K loop starts at step 5e mod (k/64) for expert e and wraps
//     round.  With every task starting at k = 0, all CUs would read the same
//     128 bytes of each 4 KiB weight row at once; those addresses agree in
//     their low 12 bits and crowd into few HBM channels (rows 4 KiB apart
//     streamed in step: 4.3 TB/s, against 5.4-5.9 with staggered starts,
//     measured on MI355X; gate_up at config 3: 234 -> 213 us).  The start
//     depends on the expert only, so every variant sums each output in the
//     same order, and an expert's row tiles still read its weights together.
//   * 8 MFMA waves = 2 (M, 64 rows) x 4 (N, 64 columns),
//     v_mfma_f32_16x16x32_f16, fp32 accumulate; they also write C.  Four more
//     waves issue all of the DMA (4 A and 8 B instructions per stage each) and
//     nothing else.  On gfx950 a wave's stores count in vmcnt like its
//     loads, so a wave that both streamed the stages and wrote a finished
//     tile's 128 KiB of fp32 C would drain its whole load pipeline at every
//     wait after a tile; measured at T = 2048, 128 experts, top-8, the stores
//     then cost gate_up 122 of 327 us.  With the split the issue waves' waits
//     count their own loads only (gate_up 327 -> 260 us), and C goes out with
//     non-temporal stores, written once and not read again here
//     (260 -> 247 us).
//   * LIVE (the recording's own calls, rmda_gemm_args_t::live_count): a
//     tile's rows past its segment's routed rows are padding whose results
//     nothing reads, so a wave whose 64 rows are all padding reads no
//     fragments and runs no MFMAs, padding rows are not stored, and their A
//     loads read the tile's first row again instead of HBM.  A partly live
//     wave computes all four of its 16-row groups: skipping the dead ones
//     branches inside the MFMA sequence (measured on MI355X: the recording's
//     gate_up about 7 us faster without that, 238 -> 231 and 231 -> 224 us
//     on two boxes, its down unchanged).  At T = 2048,
//     128 experts, top-8 a third of the used tiles' rows are padding.
//   * SWI (rmda_gemm_args_t::f32_swiglu, the recording's gate_up): the N
//     tile is 128 gate columns j and their 128 up columns n_w/2 + j, laid out
//     so that each MFMA wave holds 32 of each for the same 32 outputs (LDS
//     rows 64w .. 64w+31 gate, 64w+32 .. 64w+63 up); the epilogue writes
//     silu(g) * u in place of the two fp32 columns and folds the absmax
//     that the next cast needs, so C never goes to memory.
#include "common.h"
#include "gemm_sched.h"

namespace {

using namespace rmda_gemm;

constexpr uint32_t RM = 128;   // rows per tile (the reference's P)
constexpr uint32_t RN = 256;   // N tile
constexpr uint32_t RK = 64;    // K step
constexpr uint32_t RMW = 8;    // MFMA waves: 2 (M, 64 rows) x 4 (N, 64 columns)
constexpr uint32_t RIW = 4;    // DMA issue waves
constexpr uint32_t RSTAGES = 3;
constexpr uint32_t MAX_TILES = 4096;  // compacted tile list in LDS (u16 entries)

__device__ __forceinline__ float ref_slot_scale(const uint32_t *amax, uint32_t slot) {
    if (slot == RMDA_NO_SLOT || amax == nullptr) {
        return 1.0f;
    }
    const uint32_t u = amax[slot];
    const float a = __builtin_bit_cast(float, u);
    if (!(a > 0.0f) || __builtin_isinf(a)) {
        return 1.0f;
    }
    return ldexpf(1.0f, 141 - (int)((u >> 23) & 0xffu));
}

template <bool LIVE, bool SWI>
__global__ __launch_bounds__(768) void ref_mm_kernel(rmda_gemm_args_t g) {
    constexpr uint32_t CH = RK / 8;                 // 16-byte chunks per row
    constexpr uint32_t RPI = 64 / CH;               // rows per DMA instruction
    constexpr uint32_t A_BYTES = RM * RK * 2;       // 16 KiB
    constexpr uint32_t B_BYTES = RN * RK * 2;       // 32 KiB
    constexpr uint32_t STAGE_BYTES = A_BYTES + B_BYTES;
    constexpr uint32_t A_PER = RM / RPI / RIW;      // 4 A instructions per issue wave per stage
    constexpr uint32_t B_PER = RN / RPI / RIW;      // 8 B instructions
    constexpr uint32_t L_PER = A_PER + B_PER;
    static_assert(A_PER * RPI * RIW == RM && B_PER * RPI * RIW == RN, "DMA split");
    static_assert(2 * L_PER < 64, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[RSTAGES * STAGE_BYTES];
    __shared__ uint16_t tl[MAX_TILES];
    __shared__ uint8_t tlive[LIVE ? MAX_TILES : 1];  // LIVE: rows of the compacted tile to compute, 0..RM
    __shared__ uint32_t nv_w[RMW + RIW];
    __shared__ uint32_t swi_max, swi_done;  // SWI: the workgroup's absmax bits, MFMA waves merged

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % RMDA_WAVE;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid / RMDA_WAVE);

    if (SWI && tid == 0) {
        swi_max = 0u;
        swi_done = 0u;
    }
    // ---- compact the valid tiles (tiles[t] != NONE) into tl[], in order ----
    constexpr uint32_t NTH = (RMW + RIW) * RMDA_WAVE;
    const uint32_t n_all = g.max_items;
    uint32_t n_valid = 0;
    for (uint32_t base = 0; base < n_all; base += NTH) {
        const uint32_t t = base + tid;
        const bool ok = t < n_all && g.tiles[t] != RMDA_NONE;
        const uint64_t m = __ballot(ok);
        if (lane == 0) {
            nv_w[w] = (uint32_t)__popcll(m);
        }
        __syncthreads();
        uint32_t before = n_valid;
        uint32_t all = 0;
        for (uint32_t q = 0; q < RMW + RIW; q += 1) {
            before += q < w ? nv_w[q] : 0u;
            all += nv_w[q];
        }
        if (ok) {
            const uint64_t below = lane == 0 ? 0ull : (~0ull >> (RMDA_WAVE - lane));
            const uint32_t ci = before + (uint32_t)__popcll(m & below);
            tl[ci] = (uint16_t)t;
            if constexpr (LIVE) {
                // rows [t*RM, off + count) of the segment; a map whose segment
                // starts past the tile keeps the whole tile
                const uint32_t e = g.tiles[t];
                const uint64_t lo = (uint64_t)t * RM;
                const uint64_t off = g.live_off[e];
                const uint64_t end = off + g.live_count[e];
                tlive[ci] = (uint8_t)(off > lo ? RM : end <= lo ? 0u : (uint32_t)min(end - lo, (uint64_t)RM));
            }
        }
        n_valid += all;
        __syncthreads();
    }
    const uint32_t ntiles = g.n_w / RN;
    const chunk_sched_t sched(n_valid, ntiles);
    const uint32_t ntask = sched.ntask;
    if (ntask == 0) {
        return;
    }
    const uint32_t steps = g.k / RK;
    const uint32_t nstage = ntask * steps;

    if (w >= RMW) {
        // ================= issue waves: DMA only, so their vmcnt counts loads only =================
        const uint32_t dw = w - RMW;
        const uint32_t lrow = lane / CH;
        const uint32_t lch = lane % CH;
        const uint16_t *a_src[A_PER];
        const uint16_t *b_src[B_PER];
        uint32_t k_rot = 0;  // the task's first K step
        auto setup = [&](uint32_t q) __attribute__((always_inline)) {
            uint32_t nt;
            const uint32_t ci = sched.item(q, nt);
            const uint32_t t = __builtin_amdgcn_readfirstlane(tl[ci]);
            const uint32_t grp = g.tiles[t];
            k_rot = grp * 5 % steps;
            const uint16_t *wg = g.w + (size_t)grp * g.n_w * g.k;
            // LIVE: padding rows load the tile's first row instead (a cache
            // hit, not an HBM read); their results are not stored
            const uint32_t lv = LIVE ? (uint32_t)tlive[ci] : RM;
#pragma unroll
            for (uint32_t j = 0; j < A_PER; j += 1) {
                const uint32_t r = (dw * A_PER + j) * RPI + lrow;
                const uint32_t ra = r < lv ? r : 0u;
                a_src[j] = g.a + (size_t)(t * RM + ra) * g.lda + (lch ^ swz<RK>(r)) * 8;
            }
#pragma unroll
            for (uint32_t j = 0; j < B_PER; j += 1) {
                const uint32_t n = (dw * B_PER + j) * RPI + lrow;  // LDS row
                // SWI: LDS rows 64w + c (c < 32) hold gate column 128 nt + 32w + c,
                // 64w + 32 + c the matching up column n_w / 2 + 128 nt + 32w + c
                const uint32_t wr = SWI ? (n % 64 < 32 ? 0u : g.n_w / 2) + nt * (RN / 2) + (n / 64) * 32 + n % 32
                                        : nt * RN + n;
                b_src[j] = wg + (size_t)wr * g.k + (lch ^ swz<RK>(n)) * 8;
            }
        };
        uint32_t i_task = 0;
        uint32_t i_s = 0;
        setup(0);
        auto issue = [&](uint32_t buf) __attribute__((always_inline)) {
            if (i_s == steps) {
                i_task += 1;
                i_s = 0;
                setup(i_task);
            }
            uint8_t *base = smem + buf * STAGE_BYTES;
            const uint32_t kk = i_s + k_rot < steps ? i_s + k_rot : i_s + k_rot - steps;
#pragma unroll
            for (uint32_t j = 0; j < A_PER; j += 1) {
                __builtin_amdgcn_global_load_lds((const void *)(a_src[j] + kk * RK),
                                                 (lds_void_t *)(base + (dw * A_PER + j) * RPI * (RK * 2)), 16, 0, 0);
            }
#pragma unroll
            for (uint32_t j = 0; j < B_PER; j += 1) {
                __builtin_amdgcn_global_load_lds(
                    (const void *)(b_src[j] + kk * RK),
                    (lds_void_t *)(base + A_BYTES + (dw * B_PER + j) * RPI * (RK * 2)), 16, 0, 0);
            }
            i_s += 1;
        };
        // two barriers per stage: the second one, after the MFMA waves have
        // read the stage into registers, frees its buffer, so all RSTAGES
        // buffers are in flight
#pragma unroll
        for (uint32_t st = 0; st < RSTAGES; st += 1) {
            if (st < nstage) {
                issue(st);
            }
        }
        uint32_t ibuf = 0;
        for (uint32_t gs = 0; gs < nstage; gs += 1) {
            wait_after<L_PER>(min(nstage - 1 - gs, RSTAGES - 1));
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_s_barrier();
            if (gs + RSTAGES < nstage) {
                issue(ibuf);
                ibuf = ibuf + 1 == RSTAGES ? 0 : ibuf + 1;
            }
        }
        return;
    }

    // ================= MFMA waves: fragments, MFMAs and the fp32 stores =================
    const uint32_t wm = w / 4;
    const uint32_t wn = w % 4;
    const uint32_t fr = lane % 16;
    const uint32_t fq = lane / 16;
    const uint32_t a_row = (wm * 64 + fr) * (RK * 2);
    const uint32_t b_row = A_BYTES + (wn * 64 + fr) * (RK * 2);
    const uint32_t c0 = ((0u + fq) ^ swz<RK>(fr)) * 16;  // chunk of K half 0
    const uint32_t c1 = ((4u + fq) ^ swz<RK>(fr)) * 16;  // chunk of K half 1
    const uint32_t rq = 4 * fq;
    const float sc = 1.0f / (ref_slot_scale(g.amax, g.sa) * ref_slot_scale(g.amax, g.sb));
    float *C = reinterpret_cast<float *>(g.out);
    floatx4_t acc[4][4];
    float amx = 0.0f;  // SWI: absmax of the stored outputs
    uint32_t kc = 0;
    uint32_t ks = 0;
    uint32_t cbuf = 0;
    uint32_t lrows = RM;  // LIVE: rows of the current task's tile to compute and store
    uint32_t ngrp = 4;    // LIVE: 4 if any of this wave's 64 rows holds such rows, else 0
    for (uint32_t gs = 0; gs < nstage; gs += 1) {
        lds_barrier();
        if (LIVE && ks == 0) {
            uint32_t nt;
            lrows = __builtin_amdgcn_readfirstlane(tlive[sched.item(kc, nt)]);
            ngrp = lrows > wm * 64 ? 4u : 0u;
        }
        const uint8_t *base = smem + cbuf * STAGE_BYTES;
        cbuf = cbuf + 1 == RSTAGES ? 0 : cbuf + 1;
        half8_t fa[2][4], fb[2][4];
        if (!LIVE || ngrp > 0) {
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
                fa[0][i] = *reinterpret_cast<const half8_t *>(base + a_row + i * 16 * (RK * 2) + c0);
                fb[0][i] = *reinterpret_cast<const half8_t *>(base + b_row + i * 16 * (RK * 2) + c0);
                fa[1][i] = *reinterpret_cast<const half8_t *>(base + a_row + i * 16 * (RK * 2) + c1);
                fb[1][i] = *reinterpret_cast<const half8_t *>(base + b_row + i * 16 * (RK * 2) + c1);
            }
        }
        lds_barrier();  // the stage is in registers: the issue waves may refill its buffer
        if (ks == 0) {
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
#pragma unroll
                for (int j = 0; j < 4; j += 1) {
                    acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
        if (!LIVE || ngrp != 0) {
#pragma unroll
            for (uint32_t kk = 0; kk < 2; kk += 1) {
#pragma unroll
                for (int i = 0; i < 4; i += 1) {
#pragma unroll
                    for (int j = 0; j < 4; j += 1) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[kk][i], fb[kk][j], acc[i][j], 0, 0, 0);
                    }
                }
            }
        }
        if (ks == steps - 1) {
            // acc[i][j][v] = C[tile row wm*64 + i*16 + 4*(lane/16) + v][wn*64 + j*16 + lane%16]
            uint32_t nt;
            const uint32_t t = tl[sched.item(kc, nt)];
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
                if (LIVE && ngrp == 0) {
                    continue;
                }
#pragma unroll
                for (int v = 0; v < 4; v += 1) {
                    const uint32_t rt = wm * 64 + i * 16 + rq + v;  // row within the tile
                    if (LIVE && rt >= lrows) {
                        continue;
                    }
                    const size_t r = (size_t)t * RM + rt;
                    if constexpr (SWI) {
                        // columns j (gate) and j + 2 (up) of this wave are the same outputs
#pragma unroll
                        for (int j = 0; j < 2; j += 1) {
                            const float h = rmda_swiglu(acc[i][j][v] * sc, acc[i][j + 2][v] * sc);
                            amx = fmaxf(amx, fabsf(h));
                            __builtin_nontemporal_store(h, &C[r * g.ldo + nt * (RN / 2) + wn * 32 + j * 16 + fr]);
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; j += 1) {
                            __builtin_nontemporal_store(acc[i][j][v] * sc,
                                                        &C[r * g.ldo + nt * RN + wn * 64 + j * 16 + fr]);
                        }
                    }
                }
            }
        }
        ks += 1;
        if (ks == steps) {
            ks = 0;
            kc += 1;
        }
    }
    if constexpr (SWI) {
        // the same fmaxf of fabsf as the absmax kernels, over the wave; the
        // MFMA waves merge theirs in LDS (an LDS atomicMax of the bits: the
        // values are non-negative) and the last of them to arrive makes the
        // workgroup's one device atomicMax, so the one slot word takes 256
        // device atomics instead of one per wave
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            amx = fmaxf(amx, __shfl_xor(amx, o));
        }
        if (lane == 0) {
            atomicMax(&swi_max, __builtin_bit_cast(uint32_t, amx));
            // the LDS performs this wave's two atomics in order, so the wave
            // that takes the last arrival sees every wave's maximum
            if (atomicAdd(&swi_done, 1u) == RMW - 1 && g.so != RMDA_NO_SLOT) {
                atomicMax(const_cast<uint32_t *>(&g.amax[g.so]), atomicMax(&swi_max, 0u));
            }
        }
    }
}

}  // namespace

bool rmda_ref_mm_supported(const rmda_gemm_args_t *a) {
    return a->n_w % RN == 0 && a->k % RK == 0 && a->max_items <= MAX_TILES;
}

hipError_t rmda_launch_ref_mm(hipStream_t s, const rmda_gemm_args_t *a, uint32_t grid) {
    if (!rmda_ref_mm_supported(a)) {
        return hipErrorInvalidValue;
    }
    if (a->max_items == 0) {
        return hipSuccess;
    }
    const dim3 gr(grid >= 8 ? grid / 8 * 8 : 8);
    const dim3 bl((RMW + RIW) * RMDA_WAVE);
    if ((a->live_count != nullptr) != (a->live_off != nullptr) ||
        (a->f32_swiglu && (a->amax == nullptr && a->so != RMDA_NO_SLOT))) {
        return hipErrorInvalidValue;
    }
    if (a->f32_swiglu) {
        if (a->live_count != nullptr) {
            hipLaunchKernelGGL((ref_mm_kernel<true, true>), gr, bl, 0, s, *a);
        } else {
            hipLaunchKernelGGL((ref_mm_kernel<false, true>), gr, bl, 0, s, *a);
        }
    } else if (a->live_count != nullptr) {
        hipLaunchKernelGGL((ref_mm_kernel<true, false>), gr, bl, 0, s, *a);
    } else {
        hipLaunchKernelGGL((ref_mm_kernel<false, false>), gr, bl, 0, s, *a);
    }
    return hipGetLastError();
}
