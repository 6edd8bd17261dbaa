// Grouped expert GEMM, compute tile: the fused layer's gate_up (SwiGLU
// epilogue) and down GEMMs when most token rows go to a few hot experts
// (ten experts hold 97% of the rows, up to 2048 each).
//
// Why a second tile.  The weight-streaming tile (gemm2.hip) is sized for
// experts of ~128 rows, where every weight byte is needed once and HBM is the
// bound.  A hot expert's weights are reused by thousands of rows, so the
// arithmetic intensity is far past the ridge and the limit becomes the CU:
// its MFMA pipe and how many LDS bytes each MFMA needs.  A wave that owns a
// 64 x 64 output tile reads 8 KiB of fragments from LDS for 16 MFMAs; here a
// wave owns 128 x 64 (12 KiB for 32 MFMAs), a third fewer LDS bytes per
// flop, and two waves share each SIMD so one wave's fragment reads overlap
// the other's MFMAs (measured on MI355X: 2.03 PFLOP/s for this wave shape on
// an MFMA + LDS loop, against 1.27 for four 128 x 128 waves, which have
// nobody to overlap with).
//
//   * Work item: (group, first sorted row, up to 256 rows); task = (item,
//     256-column N tile).  8 waves = 2 (M, 128 rows) x 4 (N, 64 columns);
//     waves w and w + 4 share a SIMD.
//   * K step 32.  A (256 x 32) and B (256 x 32) go from global memory into
//     LDS with global_load_lds_dwordx4 through a STAGES-deep ring of 32 KiB
//     stages; every wave issues 2 A and 2 B instructions per stage, so the
//     vmcnt waits are compile-time constants, as in gemm2.hip.
//   * The A rows of gate_up are gathered through rowtok; down reads hp in
//     its 16-row x 32-column blocks.  B comes from the packed slabs of
//     rmda_moe_pack_weights (one contiguous KiB per DMA instruction).
//   * The LDS image uses the same chunk swizzle as gemm2.hip, so fragment
//     reads are free of bank conflicts and the packed slabs need no change.
//   * Per output element the MFMA sequence (v_mfma_f32_16x16x32_f16 over K
//     steps of 32, in order, from a zero accumulator) and the epilogue are
//     those of gemm2.hip, so either tile gives bitwise the same result.
#include "common.h"
#include "gemm_sched.h"

namespace {

using namespace rmda_gemm;

constexpr uint32_t HM = RMDA_GEMM_HOT_BM;  // rows per work item
constexpr uint32_t HN = 256;               // N tile = one packed slab
constexpr uint32_t HK = 32;                // K step
constexpr uint32_t NW = 8;                 // waves

template <int MODE, int STAGES, typename SCHED, bool PP, int BPOL, bool SC = false, bool YNT = false>
__global__ __launch_bounds__(512) void hot_gemm_kernel(rmda_gemm_args_t g) {
    constexpr uint32_t CH = HK / 8;                  // 16-byte chunks per row
    constexpr uint32_t RPI = 64 / CH;                // rows per DMA instruction
    constexpr uint32_t A_BYTES = HM * HK * 2;
    constexpr uint32_t B_BYTES = HN * HK * 2;
    constexpr uint32_t STAGE_BYTES = A_BYTES + B_BYTES;
    constexpr uint32_t A_PER = HM / RPI / NW;        // A instructions per wave per stage
    constexpr uint32_t B_PER = HN / RPI / NW;        // B instructions per wave per stage
    constexpr uint32_t L_PER = A_PER + B_PER;
    constexpr uint32_t A_STEP = MODE == RMDA_GEMM_F16 ? RMDA_HP_ROWS * HK : HK;  // hp is in 16 x 32 blocks
    static_assert(RPI == RMDA_HP_ROWS, "one A instruction = one hp block");
    static_assert(STAGES >= 2 && STAGES <= 5 && STAGES * STAGE_BYTES <= 160 * 1024, "pipeline depth");
    // All of the kernel's LDS is this one array: with a second __shared__
    // array the compiler cannot tell the fragment reads from the DMA targets
    // and waits for every outstanding DMA (s_waitcnt vmcnt(0)) before each
    // stage's reads, which halves the tile's speed.
    __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE_BYTES];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % RMDA_WAVE;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid / RMDA_WAVE);
    const uint32_t wm = w / 4;
    const uint32_t wn = w % 4;

    const_u32p items = (const_u32p)g.items;
    // the slot-scaled mode's inverse scales (1 otherwise, which changes no bits)
    const float xinv = SC && MODE == RMDA_GEMM_SWIGLU ? rmda_slot_inv(g.xscale) : 1.0f;
    const float yinv = down_mul<SC, MODE>(g);
    const uint32_t ntiles = g.n_w / HN;
    const uint32_t n_items = g.n_items != nullptr ? *(const_u32p)g.n_items : g.max_items;
    const SCHED sched(n_items, ntiles);
    const uint32_t ntask = sched.ntask;
    if (ntask == 0) {
        return;
    }
    const uint32_t steps = g.k / HK;
    const uint32_t nstage = ntask * steps;

    // ---- issue side: this wave's DMA sources for the task being loaded ----
    const uint32_t lrow = lane / CH;  // row within an instruction's 16
    const uint32_t lch = lane % CH;   // LDS chunk slot of this lane
    const uint16_t *a_src[A_PER];
    const uint16_t *b_src[B_PER];
    auto setup = [&](uint32_t q) __attribute__((always_inline)) {
        uint32_t nt;
        const uint32_t item = sched.item(q, nt);
        const uint32_t grp = items[item * 4 + 0];
        const uint32_t row0 = items[item * 4 + 1];
        const uint32_t rows = items[item * 4 + 2];
        const bool is_shared = grp == g.shared_group;
        const uint16_t *wg = is_shared ? g.w_shared : g.w + (size_t)grp * g.n_w * g.k;
#pragma unroll
        for (uint32_t j = 0; j < A_PER; j += 1) {
            const uint32_t blk = (w + j * NW) * RPI;  // first tile row of this instruction
            const uint32_t r = blk + lrow;
            if (MODE == RMDA_GEMM_SWIGLU) {
                uint32_t arow;
                if (is_shared) {
                    arow = row0 + (r < rows ? r : 0u) - g.shared_row0;
                } else {
                    // gathered token rows (scalar loads; rowtok is padded by
                    // RMDA_ROWTOK_PAD >= HM entries, so these reads stay inside it)
                    const const_u32p rt = (const_u32p)g.rowtok + row0 + blk;
                    uint32_t tok[RPI];
#pragma unroll
                    for (uint32_t c = 0; c < RPI; c += 1) {
                        tok[c] = rt[c];
                    }
                    uint32_t t = tok[0];
#pragma unroll
                    for (uint32_t c = 1; c < RPI; c += 1) {
                        t = lrow == c ? tok[c] : t;
                    }
                    arow = r < rows ? t : ((const_u32p)g.rowtok + row0)[0];
                    arow = arow < g.a_rows ? arow : 0u;  // a bad index reads a valid row, never out of bounds
                }
                a_src[j] = g.a + (size_t)arow * g.lda + (lch ^ swz<HK>(r)) * 8;
            } else {
                // rows past the item re-read its first block
                a_src[j] = g.a + rmda_hp_index(row0 + (blk < rows ? blk : 0u), 0, g.lda) + lrow * 32 +
                           (lch ^ swz<HK>(r)) * 8;
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < B_PER; j += 1) {
            const uint32_t nin = (w + j * NW) * RPI;
            b_src[j] = wg + (size_t)nt * steps * (HN * HK) + nin * HK + lane * 8;
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
#pragma unroll
        for (uint32_t j = 0; j < A_PER; j += 1) {
            __builtin_amdgcn_global_load_lds((const void *)(a_src[j] + i_s * A_STEP),
                                             (lds_void_t *)(base + (w + j * NW) * RPI * (HK * 2)), 16, 0, 0);
        }
#pragma unroll
        for (uint32_t j = 0; j < B_PER; j += 1) {
            __builtin_amdgcn_global_load_lds((const void *)(b_src[j] + (size_t)i_s * (HN * HK)),
                                             (lds_void_t *)(base + A_BYTES + (w + j * NW) * RPI * (HK * 2)), 16, 0,
                                             BPOL);
        }
        i_s += 1;
    };

    // ---- compute side ----
    const uint32_t fr = lane % 16;
    const uint32_t fq = lane / 16;
    const uint32_t a_off = (wm * 128 + fr) * (HK * 2) + (fq ^ swz<HK>(fr)) * 16;
    const uint32_t b_off = A_BYTES + (wn * 64 + fr) * (HK * 2) + (fq ^ swz<HK>(fr)) * 16;
    const uint32_t rq = 4 * fq;
    floatx4_t acc[8][4];
    float hmax_run = 0.0f;  // slot-scaled mode: this lane's largest |SwiGLU| over its tasks
    half8_t fa[8], fb[4];
    uint32_t c_row0 = 0;
    uint32_t c_rows = 0;
    uint32_t c_nt = 0;
    uint32_t kc = 0;
    uint32_t ks = 0;
    bool live = false;  // some of this wave's 128 rows hold task rows
    auto load_frags = [&](uint32_t buf) __attribute__((always_inline)) {
        const uint8_t *base = smem + buf * STAGE_BYTES;
#pragma unroll
        for (int j = 0; j < 4; j += 1) {
            fb[j] = *reinterpret_cast<const half8_t *>(base + b_off + j * 16 * (HK * 2));
        }
#pragma unroll
        for (int i = 0; i < 8; i += 1) {
            fa[i] = *reinterpret_cast<const half8_t *>(base + a_off + i * 16 * (HK * 2));
        }
    };
    // one K step on the fragments in registers, with the task bookkeeping
    // and, after a task's last K step, its epilogue
    auto compute = [&]() __attribute__((always_inline)) {
        if (ks == 0) {
            const uint32_t item = sched.item(kc, c_nt);
            c_row0 = items[item * 4 + 1];
            c_rows = items[item * 4 + 2];
            live = wm * 128 < c_rows;
#pragma unroll
            for (int i = 0; i < 8; i += 1) {
#pragma unroll
                for (int j = 0; j < 4; j += 1) {
                    acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
        // a wave whose 128 rows all lie past the item skips its MFMAs; a
        // partly live wave runs all eight row groups (its dead rows hold
        // copies of a live row and are not stored): skipping per 16-row group
        // needs branches that push the accumulators out of registers
        if (live) {
#pragma unroll
            for (int i = 0; i < 8; i += 1) {
#pragma unroll
                for (int j = 0; j < 4; j += 1) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (live && ks == steps - 1) {
            // acc[i][j][v] = C[wm*128 + i*16 + 4*(lane/16) + v][B row wn*64 + j*16 + lane%16]
            uint16_t *O = reinterpret_cast<uint16_t *>(g.out);
            if (MODE == RMDA_GEMM_F16) {
#pragma unroll
                for (int i = 0; i < 8; i += 1) {
#pragma unroll
                    for (int v = 0; v < 4; v += 1) {
                        const uint32_t rr = wm * 128 + i * 16 + rq + v;
                        if (rr < c_rows) {
#pragma unroll
                            for (int j = 0; j < 4; j += 1) {
                                const uint32_t col = c_nt * HN + wn * 64 + j * 16 + fr;
                                down_store<SC, YNT>(g, O, (size_t)(c_row0 + rr) * g.ldo + col,
                                                    acc[i][j][v] * yinv);
                            }
                        }
                    }
                }
            } else {
                // slab rows wn*64 .. +64 are 32 gate rows then the 32 matching
                // up rows: blocks j (gate) and j + 2 (up) share output columns
                const uint32_t colbase = c_nt * (HN / 2) + wn * 32;
#pragma unroll
                for (int i = 0; i < 8; i += 1) {
#pragma unroll
                    for (int v = 0; v < 4; v += 1) {
                        const uint32_t rr = wm * 128 + i * 16 + rq + v;
                        if (rr < c_rows) {
#pragma unroll
                            for (int j = 0; j < 2; j += 1) {
                                const float gt = acc[i][j][v] * xinv;
                                const float up = acc[i][j + 2][v] * xinv;
                                const float h = rmda_swiglu_fast(gt, up);
                                swiglu_store<SC, false>(g, O, rmda_hp_index(c_row0 + rr, colbase + j * 16 + fr, g.ldo), h, hmax_run);
                            }
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
    };

#pragma unroll
    for (uint32_t s = 0; s < STAGES - 1; s += 1) {
        if (s < nstage) {
            issue(s);
        }
    }
    uint32_t ibuf = STAGES - 1;
    uint32_t cbuf = 0;
    if (!PP) {
        // lockstep: one barrier per stage, every wave reads then multiplies
        for (uint32_t gs = 0; gs < nstage; gs += 1) {
            // this wave's loads of stage gs have landed (later stages may fly),
            // then everyone's have, and every wave is done reading stage gs - 1
            wait_after<L_PER>(min(nstage - 1 - gs, (uint32_t)STAGES - 2));
            lds_barrier();
            if (gs + STAGES - 1 < nstage) {
                issue(ibuf);  // into the buffer stage gs - 1 used
                ibuf = ibuf + 1 == STAGES ? 0 : ibuf + 1;
            }
            load_frags(cbuf);
            cbuf = cbuf + 1 == STAGES ? 0 : cbuf + 1;
            compute();
        }
        if (SC && MODE == RMDA_GEMM_SWIGLU) {
            rmda_wave_amax(g.hp_amax, hmax_run);
        }
        return;
    }
    // Ping-pong: the waves of row block 0 (w < 4) and of row block 1 (w >= 4)
    // share the SIMDs pairwise and run half a stage apart, two barriers per
    // stage.  Between consecutive barriers one group reads a stage's
    // fragments from LDS and issues its share of a later stage's DMA (M)
    // while the other group multiplies the fragments it read before (C):
    //   group 0:      M(0) | C(0) | M(1) | C(1) | ...
    //   group 1: idle | M(0) | C(0) | M(1) | ...
    // Stage g is complete before either group reads it: group 0 waits for its
    // own loads of stage g at the end of C(g-1), group 1 at the end of
    // M(g-1), both before the barrier that precedes group 0's M(g).  The DMA
    // of stage g + STAGES - 1 (issued in M(g)) refills the buffer of stage
    // g - 1, whose last reader (group 1's M(g-1)) finished before that same
    // barrier.  Both groups execute 2 * nstage barriers after the prologue.
    const bool g1 = wm != 0;
    wait_after<L_PER>(min(nstage - 1, (uint32_t)STAGES - 2));
    __builtin_amdgcn_s_barrier();  // stage 0 complete
    if (g1) {
        __builtin_amdgcn_s_barrier();  // group 0's M(0)
    }
    for (uint32_t gs = 0; gs < nstage; gs += 1) {
        // M(gs)
        if (gs + STAGES - 1 < nstage) {
            issue(ibuf);
            ibuf = ibuf + 1 == STAGES ? 0 : ibuf + 1;
        }
        load_frags(cbuf);
        cbuf = cbuf + 1 == STAGES ? 0 : cbuf + 1;
        if (g1 && gs + 1 < nstage) {
            wait_after<L_PER>(min(nstage - 2 - gs, (uint32_t)STAGES - 2));  // stage gs + 1 landed
        }
        lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // C(gs)
        compute();
        if (!g1 && gs + 1 < nstage) {
            wait_after<L_PER>(min(nstage - 2 - gs, (uint32_t)STAGES - 2));  // stage gs + 1 landed
        }
        __builtin_amdgcn_sched_barrier(0);
        if (!g1 || gs + 1 < nstage) {
            __builtin_amdgcn_s_barrier();
        }
    }
    if (SC && MODE == RMDA_GEMM_SWIGLU) {
        rmda_wave_amax(g.hp_amax, hmax_run);
    }
}

// sched: bit 0 = contiguous chunks per XCD (else task_sched_t), bit 1 = lockstep
// (else ping-pong), bit 2 = non-temporal weight loads (else default policy)
template <int MODE, int STAGES, typename SCHED, bool PP>
void launch_pol(hipStream_t s, const rmda_gemm_args_t *a, dim3 gr, int sched) {
    const dim3 blk(NW * RMDA_WAVE);
    if ((sched & 4) != 0) {
        hipLaunchKernelGGL((hot_gemm_kernel<MODE, STAGES, SCHED, PP, 2>), gr, blk, 0, s, *a);
    } else {
        hipLaunchKernelGGL((hot_gemm_kernel<MODE, STAGES, SCHED, PP, 0>), gr, blk, 0, s, *a);
    }
}

template <int MODE, int STAGES>
void launch_sched(hipStream_t s, const rmda_gemm_args_t *a, dim3 gr, int sched) {
    switch (sched & 3) {
    case 0: launch_pol<MODE, STAGES, task_sched_t, true>(s, a, gr, sched); break;
    case 1: launch_pol<MODE, STAGES, chunk_sched_t, true>(s, a, gr, sched); break;
    case 2: launch_pol<MODE, STAGES, task_sched_t, false>(s, a, gr, sched); break;
    default: launch_pol<MODE, STAGES, chunk_sched_t, false>(s, a, gr, sched); break;
    }
}

template <int MODE>
void launch_mode(hipStream_t s, const rmda_gemm_args_t *a, dim3 gr, int stages, int sched) {
    if (stages == 5) {
        launch_sched<MODE, 5>(s, a, gr, sched);
    } else {
        launch_sched<MODE, 4>(s, a, gr, sched);
    }
}

}  // namespace

hipError_t rmda_launch_gemm_hot(hipStream_t s, const rmda_gemm_args_t *a, uint32_t grid, int stages, int sched) {
    if (a->k % HK != 0 || a->n_w % HN != 0) {
        return hipErrorInvalidValue;
    }
    if (a->max_items == 0) {
        return hipSuccess;
    }
    const dim3 gr(grid >= 8 ? grid / 8 * 8 : 8);  // persistent: one workgroup per CU, whole XCDs
    if (a->hp32 != nullptr || a->ye32 != nullptr || a->ye_bound != nullptr) {
        // the slot-scaled mode: the default configuration only
        if ((a->mode == RMDA_GEMM_SWIGLU) != (a->hp32 != nullptr) ||
            (a->mode == RMDA_GEMM_F16) != ((a->ye32 != nullptr) != (a->ye_bound != nullptr)) || stages != 4 ||
            sched != 0) {
            return hipErrorInvalidValue;
        }
        if (a->mode == RMDA_GEMM_SWIGLU) {
            hipLaunchKernelGGL((hot_gemm_kernel<RMDA_GEMM_SWIGLU, 4, task_sched_t, true, 0, true>), gr,
                               dim3(NW * RMDA_WAVE), 0, s, *a);
        } else if (a->ye_nt != 0) {
            hipLaunchKernelGGL((hot_gemm_kernel<RMDA_GEMM_F16, 4, task_sched_t, true, 0, true, true>), gr,
                               dim3(NW * RMDA_WAVE), 0, s, *a);
        } else {
            hipLaunchKernelGGL((hot_gemm_kernel<RMDA_GEMM_F16, 4, task_sched_t, true, 0, true>), gr,
                               dim3(NW * RMDA_WAVE), 0, s, *a);
        }
        return hipGetLastError();
    }
    if (a->mode == RMDA_GEMM_F16 && a->ye_nt != 0 && stages == 4 && sched == 0) {
        // the default configuration with non-temporal row stores
        hipLaunchKernelGGL((hot_gemm_kernel<RMDA_GEMM_F16, 4, task_sched_t, true, 0, false, true>), gr,
                           dim3(NW * RMDA_WAVE), 0, s, *a);
        return hipGetLastError();
    }
    if (a->mode == RMDA_GEMM_SWIGLU) {
        launch_mode<RMDA_GEMM_SWIGLU>(s, a, gr, stages, sched);
    } else {
        launch_mode<RMDA_GEMM_F16>(s, a, gr, stages, sched);
    }
    return hipGetLastError();
}
