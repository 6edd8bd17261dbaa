// Grouped expert GEMM of the fused layer: weight-streaming design for gfx950.
// Serves the gate_up GEMM (SwiGLU epilogue) and the down GEMM, and packs the
// expert weights into the order it streams them.
//
// Why this shape.  At the benchmark shapes every expert's weight slice is
// needed by ~128 token rows, so the GEMM is bound by streaming the weights
// from HBM (arithmetic intensity ~120 FLOP/B against a ridge of ~312).  Two
// things decide the speed: every weight byte leaves HBM once, and enough
// bytes are in flight to cover HBM latency.
//   * A work item is (group, first row, up to 192 rows): one workgroup owns
//     all rows of an expert (up to 192) for one 256-wide N tile, so each
//     weight tile is read once.  The 192 rows are three 64-row blocks; a
//     16-row MFMA group past the item's end runs no MFMAs.
//   * Operand tiles go straight from global memory into LDS with gfx950's
//     global_load_lds_dwordx4 (no register staging), through a ring of
//     STAGES buffers, so several stages are in flight while one is
//     multiplied.  Completion is tracked with explicit vmcnt waits (each
//     issuing wave knows how many loads it issued per stage) and a bare
//     s_barrier, so no compiler-inserted full wait drains the pipeline.
//   * LDS rows are BK halves; the 16-byte chunks of row r sit XOR-swizzled
//     (swz below) so MFMA fragment reads are free of bank conflicts.  A DMA
//     instruction writes 64 consecutive 16-byte slots, so the swizzle is
//     applied on the global side: each lane fetches the chunk that belongs
//     at its slot.
//   * Packed weights (rmda_moe_pack_weights) store every 256-row x BK slab
//     (one N tile's K step) in exactly its LDS image order, so each DMA
//     instruction reads one contiguous KiB and a whole stage of B is one
//     contiguous 16 KiB block (the HF [out][in] layout would read BK-wide
//     pieces of 256 rows 4 KiB apart).
//   * Weight loads carry the non-temporal hint: every weight byte is read
//     once per launch, and keeping it out of the caches leaves them to the
//     gathered activation rows and to the next kernel's inputs (gate_up
//     176 vs 178 us, combine 14.7 vs 15.6 us at BASELINE config 3).
//   * Tasks are dealt XCD-aware from the real work count read on the device
//     (task_sched_t): whole items go to XCDs, so the N tiles of one item
//     (which share A rows) meet in one L2, and the list's row-count order
//     lets alternating rounds even out every XCD's and workgroup's load.
// MFMA: v_mfma_f32_16x16x32_f16, fp32 accumulate; 12 MFMA waves = 3 (M) x
// 4 (N), 64 x 64 per wave.
//
// Three kernels share this design:
//   * gemm2_kernel: every MFMA wave also issues its share of each stage's
//     DMA, between its MFMA groups (HF-layout weights, and measurement
//     variants for packed ones).
//   * gemm4_kernel (gate_up when experts average 32 rows or more): as
//     gemm3_kernel below, with the gathered activation rows in a ring of
//     their own, two K steps per slot, so each row is one 128-byte line per
//     pair of K steps.
//   * gemm3_kernel (packed weights, the default): four more waves issue all
//     of the DMA and nothing else, so a stage's loads leave right after the
//     stage barrier instead of queueing behind MFMAs; a second barrier
//     after the fragment reads frees a buffer before its MFMAs run, so all
//     STAGES buffers are in flight.  Measured at config 3 against
//     gemm2_kernel on the same boxes: gate_up 175.3 -> 172.6 us, down
//     106.1 -> 104.9 us.  The second barrier was first kept for gate_up
//     only; with the non-temporal SwiGLU stores in place, giving it to the
//     down GEMM as well takes the layer at config 3 from 303 to 297 us and
//     from 289 to 286-288 us on two boxes, at config 5 from 789 to 775 and
//     756 to 750 us, from fp32 activations at config 3 from 336 to 327-331
//     us; configs 2 and 4 are unchanged and the teacher's shape from fp32
//     activations 0.4% slower.  Most of the gain shows in the next call's
//     gate_up, not in down itself (at 512 experts down is 2% slower).
#include "common.h"
#include "gemm_sched.h"

namespace {

using namespace rmda_gemm;

constexpr uint32_t BM = RMDA_GEMM2_BM;  // rows per work item (three 64-row blocks)
constexpr uint32_t SLAB = 256;          // packed slab height (B rows) = the N tile

// B row of a group's weight matrix that slab row n of slab `slab` holds.
// A SWIGLU slab is SLAB/64 groups of 32 gate rows followed by the 32
// matching up rows, so one wave's accumulators hold gate and up of the same
// output columns.
template <int MODE>
__device__ __forceinline__ uint32_t slab_row(uint32_t slab, uint32_t n, uint32_t inter) {
    if (MODE == RMDA_GEMM_SWIGLU) {
        const uint32_t bw = n / 64;
        const uint32_t within = n % 64;
        const uint32_t c = slab * (SLAB / 2) + bw * 32 + (within % 32);
        return within < 32 ? c : inter + c;
    }
    return slab * SLAB + n;
}

// Persistent workgroup: MB (=3) blocks of 64 rows x BN/64 (=4) column
// blocks of 64, one wave each (12 waves).  Waves w and w + 4 share a SIMD, so
// the four waves of a row block sit on four different SIMDs and any number of
// live row blocks keeps the SIMDs balanced.
//
// One workgroup per CU walks a strided list of (work item, N tile) tasks.
// All tasks of a launch have the same K, so the workgroup's stages form one
// stream: stage g is K step g % steps of its task g / steps, and the ring
// keeps STAGES-1 stages in flight across task boundaries (the next task's
// first stages load while the current one finishes and stores its tile).
// Task descriptors and gathered row indices come in through scalar loads
// (constant address space, counted by lgkmcnt), so the vmcnt bookkeeping of
// the ring sees nothing but the stage loads: every wave issues the same
// number of loads per stage (A rows of idle row blocks re-read row 0), and
// the stores of a finished tile are never counted in a wait's allowance, so
// each wait is exact or conservative.

template <int MODE, int BN, int BK, int STAGES, bool PACKED, int BPOL, bool SC = false>
__global__ __launch_bounds__(768) void gemm2_kernel(rmda_gemm_args_t g) {
    constexpr uint32_t MB = BM / 64;             // row blocks
    constexpr uint32_t NB = BN / 64;             // column blocks
    constexpr uint32_t NWAVES = MB * NB;
    constexpr uint32_t CH = BK / 8;              // 16-byte chunks per row
    constexpr uint32_t RPI = 64 / CH;            // rows per wave-wide DMA instruction
    constexpr uint32_t A_BYTES = BM * BK * 2;
    constexpr uint32_t B_BYTES = BN * BK * 2;
    constexpr uint32_t STAGE_BYTES = A_BYTES + B_BYTES;
    constexpr uint32_t AW = 64 / NB;             // A rows loaded per wave
    constexpr uint32_t A_PER = AW / RPI;         // A instructions per wave per stage
    constexpr uint32_t B_ALL = BN / RPI;         // B instructions per stage, dealt round-robin
    constexpr uint32_t B_HI = (B_ALL + NWAVES - 1) / NWAVES;
    constexpr uint32_t B_LO = B_ALL / NWAVES;
    static_assert(A_PER >= 1 && AW % RPI == 0 && AW <= 16, "A rows per wave must fill DMA instructions");
    // K step of an A load: the down GEMM's A (hp) is in 16-row x 32-column blocks
    constexpr uint32_t A_STEP = MODE == RMDA_GEMM_F16 ? RMDA_HP_ROWS * BK : BK;
    static_assert(MODE != RMDA_GEMM_F16 || (BK == 32 && RPI == RMDA_HP_ROWS), "hp block = one K step of one A instruction");
    static_assert(STAGES >= 2 && STAGES <= 6, "pipeline depth");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE_BYTES];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % RMDA_WAVE;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid / RMDA_WAVE);
    const uint32_t wm = w / NB;
    const uint32_t wn = w % NB;

    // ---- this workgroup's tasks (task_sched_t) ----
    const_u32p items = (const_u32p)g.items;
    // the slot-scaled mode's inverse scales (1 otherwise, which changes no bits)
    const float xinv = SC && MODE == RMDA_GEMM_SWIGLU ? rmda_slot_inv(g.xscale) : 1.0f;
    const float yinv = down_mul<SC, MODE>(g);
    const uint32_t n_slabs = g.n_w / SLAB;
    const uint32_t ntiles = n_slabs / (BN / SLAB);
    const uint32_t n_items = g.n_items != nullptr ? *(const_u32p)g.n_items : g.max_items;
    const task_sched_t sched(n_items, ntiles);
    const uint32_t ntask = sched.ntask;
    if (ntask == 0) {
        return;
    }
    const uint32_t steps = g.k / BK;
    const uint32_t nstage = ntask * steps;
    const bool b_hi = w < B_ALL % NWAVES || B_ALL % NWAVES == 0;
    const uint32_t n_b = b_hi ? B_HI : B_LO;

    const uint32_t lrow = lane / CH;   // row within one instruction's block
    const uint32_t lch = lane % CH;    // LDS chunk slot

    // ---- issue side: per-lane DMA sources of the task being loaded ----
    const uint16_t *a_src[A_PER];
    uint32_t a_dst[A_PER];
    const uint16_t *b_src[B_HI];
    uint32_t b_dst[B_HI];
#pragma unroll
    for (uint32_t j = 0; j < A_PER; j += 1) {
        a_dst[j] = (wm * 64 + wn * AW + j * RPI) * (BK * 2);
    }
#pragma unroll
    for (uint32_t j = 0; j < B_HI; j += 1) {
        const uint32_t bi = j < n_b ? w + j * NWAVES : w;
        b_dst[j] = A_BYTES + bi * RPI * (BK * 2);
    }
    auto setup = [&](uint32_t k) __attribute__((always_inline)) {
        uint32_t nt;
        const uint32_t item = sched.item(k, nt);
        const uint32_t grp = items[item * 4 + 0];
        const uint32_t row0 = items[item * 4 + 1];
        const uint32_t rows = items[item * 4 + 2];
        const bool is_shared = grp == g.shared_group;
        const uint16_t *wg = is_shared ? g.w_shared : g.w + (size_t)grp * g.n_w * g.k;
        // gathered token rows of this wave's AW A rows (scalar loads; the
        // index buffer is padded so the 16-entry read never leaves it)
        const uint32_t rbase = wm * 64 + wn * AW;
        uint32_t tok[16];
        uint32_t tok0 = 0;
        if (MODE == RMDA_GEMM_SWIGLU && !is_shared) {
            const const_u32p rt = (const_u32p)g.rowtok + row0;
            tok0 = rt[0];
#pragma unroll
            for (uint32_t c = 0; c < 16; c += 1) {
                tok[c] = rt[rbase + c];
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < A_PER; j += 1) {
            const uint32_t rl = j * RPI + lrow;  // row within the wave's AW rows
            const uint32_t r = rbase + rl;
            const uint32_t rr = r < rows ? r : 0u;
            uint32_t arow;
            if (MODE == RMDA_GEMM_SWIGLU) {
                if (is_shared) {
                    arow = row0 + rr - g.shared_row0;
                } else {
                    uint32_t t = tok[0];
#pragma unroll
                    for (uint32_t c = 1; c < 16; c += 1) {
                        t = rl == c ? tok[c] : t;
                    }
                    arow = r < rows ? t : tok0;
                    arow = arow < g.a_rows ? arow : 0u;  // a bad index reads a valid row, never out of bounds
                }
            } else {
                arow = row0 + rr;
            }
            if (MODE == RMDA_GEMM_F16) {
                // hp is stored in 16-row x 32-column blocks: this instruction's 16 rows
                // at one K step are one contiguous KiB (blocks past the item re-read its first)
                const uint32_t blk = rbase + j * RPI;
                a_src[j] = g.a + rmda_hp_index(row0 + (blk < rows ? blk : 0u), 0, g.lda) + lrow * 32 +
                           (lch ^ swz<BK>(r)) * 8;
            } else {
                a_src[j] = g.a + (size_t)arow * g.lda + (lch ^ swz<BK>(r)) * 8;
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < B_HI; j += 1) {
            const uint32_t bi = j < n_b ? w + j * NWAVES : w;
            const uint32_t nbase = bi * RPI;
            const uint32_t slab = nt * (BN / SLAB) + nbase / SLAB;
            const uint32_t nin = nbase % SLAB;
            if (PACKED) {
                b_src[j] = wg + (size_t)slab * steps * (SLAB * BK) + nin * BK + lane * 8;
            } else {
                const uint32_t n = nin + lrow;
                b_src[j] = wg + (size_t)slab_row<MODE>(slab, n, g.inter) * g.k + (lch ^ swz<BK>(n)) * 8;
            }
        }
    };
    uint32_t i_task = 0;  // task ordinal and K step of the next stage to issue
    uint32_t i_s = 0;
    setup(0);
    // The stage's DMA instructions are issued one at a time between MFMA
    // groups (see the main loop), so the CU's load path is fed while the
    // matrix pipe works instead of all waves stalling on it at once.
    uint8_t *ibase = smem;
    auto issue_begin = [&](uint32_t buf) __attribute__((always_inline)) {
        if (i_s == steps) {
            i_task += 1;
            i_s = 0;
            setup(i_task);
        }
        ibase = smem + buf * STAGE_BYTES;
    };
    // instruction q of this wave's stage: A rows first, then its B slices
    auto issue_one = [&](uint32_t q) __attribute__((always_inline)) {
        if (q < A_PER) {
            __builtin_amdgcn_global_load_lds((const void *)(a_src[q] + i_s * A_STEP), (lds_void_t *)(ibase + a_dst[q]), 16,
                                             0, 0);
        } else if (q - A_PER < n_b) {
            const uint32_t j = q - A_PER;
            const uint16_t *src = PACKED ? b_src[j] + (size_t)i_s * (SLAB * BK) : b_src[j] + i_s * BK;
            __builtin_amdgcn_global_load_lds((const void *)src, (lds_void_t *)(ibase + b_dst[j]), 16, 0, BPOL);
        }
    };
    auto issue_end = [&]() __attribute__((always_inline)) { i_s += 1; };
    auto issue_next = [&](uint32_t buf) __attribute__((always_inline)) {
        issue_begin(buf);
#pragma unroll
        for (uint32_t q = 0; q < A_PER + B_HI; q += 1) {
            issue_one(q);
        }
        issue_end();
    };

    // ---- compute side ----
    const uint32_t fr = lane % 16;
    const uint32_t fq = lane / 16;
    uint32_t ch_off[BK / 32];
#pragma unroll
    for (uint32_t kk = 0; kk < BK / 32; kk += 1) {
        ch_off[kk] = ((kk * 4 + fq) ^ swz<BK>(fr)) * 16;
    }
    const uint32_t a_row_off = (wm * 64 + fr) * (BK * 2);
    const uint32_t b_row_off = A_BYTES + (wn * 64 + fr) * (BK * 2);
    const uint32_t rq = 4 * fq;
    floatx4_t acc[4][4];
    float hmax_run = 0.0f;  // slot-scaled mode: this lane's largest |SwiGLU| over its tasks
    uint32_t c_row0 = 0;
    uint32_t c_rows = 0;
    uint32_t c_nt = 0;
    uint32_t kc = 0;  // compute task ordinal and K step
    uint32_t ks = 0;
    bool live = false;
    uint32_t nlive = 0;  // 16-row blocks of this wave's 64 rows that hold task rows
    constexpr uint32_t KK = BK / 32;
    typedef half8_t frag_t[KK][4];
    frag_t fa0, fb0;
    auto load_frags = [&](uint32_t buf, frag_t &fa, frag_t &fb) __attribute__((always_inline)) {
        const uint8_t *base = smem + buf * STAGE_BYTES;
#pragma unroll
        for (uint32_t kk = 0; kk < KK; kk += 1) {
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
                fa[kk][i] = *reinterpret_cast<const half8_t *>(base + a_row_off + i * 16 * (BK * 2) + ch_off[kk]);
                fb[kk][i] = *reinterpret_cast<const half8_t *>(base + b_row_off + i * 16 * (BK * 2) + ch_off[kk]);
            }
        }
    };
    // one stage of MMA on fragments (fa, fb) in four groups of four MFMAs,
    // with the task bookkeeping; `between(q)` runs after group q (q < 3)
    auto compute_begin = [&]() __attribute__((always_inline)) {
        if (ks == 0) {
            const uint32_t item = sched.item(kc, c_nt);
            c_row0 = items[item * 4 + 1];
            c_rows = items[item * 4 + 2];
            live = wm * 64 < c_rows;
            nlive = live ? min(4u, (c_rows - wm * 64 + 15) / 16) : 0u;
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
#pragma unroll
                for (int j = 0; j < 4; j += 1) {
                    acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
    };
    auto mfma_group = [&](const frag_t &fa, const frag_t &fb, int i) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t kk = 0; kk < KK; kk += 1) {
#pragma unroll
            for (int j = 0; j < 4; j += 1) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[kk][i], fb[kk][j], acc[i][j], 0, 0, 0);
            }
        }
    };
    auto compute_end = [&]() __attribute__((always_inline)) {
        if (live && ks == steps - 1) {
            // tile epilogue: acc[i][j][v] is
            // C[wm*64 + i*16 + 4*(lane/16) + v][B row wn*64 + j*16 + lane%16]
            uint16_t *O = reinterpret_cast<uint16_t *>(g.out);
            if (MODE == RMDA_GEMM_F16) {
#pragma unroll
                for (int i = 0; i < 4; i += 1) {
#pragma unroll
                    for (int v = 0; v < 4; v += 1) {
                        const uint32_t rr = wm * 64 + i * 16 + rq + v;
                        if (rr < c_rows) {
#pragma unroll
                            for (int j = 0; j < 4; j += 1) {
                                const uint32_t col = c_nt * BN + wn * 64 + j * 16 + fr;
                                down_store<SC>(g, O, (size_t)(c_row0 + rr) * g.ldo + col, acc[i][j][v] * yinv);
                            }
                        }
                    }
                }
            } else {
                // a 64-row group of B rows is 32 gate rows then the 32
                // matching up rows: blocks j (gate) and j + 2 (up) hold the
                // same output columns
                const uint32_t slab = c_nt * (BN / SLAB) + (wn * 64) / SLAB;
                const uint32_t colbase = slab * (SLAB / 2) + (((wn * 64) % SLAB) / 64) * 32;
#pragma unroll
                for (int i = 0; i < 4; i += 1) {
#pragma unroll
                    for (int v = 0; v < 4; v += 1) {
                        const uint32_t rr = wm * 64 + i * 16 + rq + v;
                        if (rr < c_rows) {
#pragma unroll
                            for (int j = 0; j < 2; j += 1) {
                                const float gt = acc[i][j][v] * xinv;
                                const float up = acc[i][j + 2][v] * xinv;
                                const float h = rmda_swiglu_fast(gt, up);
                                swiglu_store<SC, true>(g, O, rmda_hp_index(c_row0 + rr, colbase + j * 16 + fr, g.ldo), h, hmax_run);
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
    auto compute = [&](const frag_t &fa, const frag_t &fb) __attribute__((always_inline)) {
        compute_begin();
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
            if ((uint32_t)i < nlive) {
                mfma_group(fa, fb, i);
            }
        }
        compute_end();
    };

    // Iteration g: wait for stage g (later issued stages stay in flight),
    // barrier, multiply stage g while issuing stage g + STAGES - 1 into the
    // buffer stage g - 1 used (every wave passed this barrier after its reads
    // of that buffer).
    constexpr int LHI = (int)(A_PER + B_HI);
    constexpr int LLO = (int)(A_PER + B_LO);
#pragma unroll
    for (uint32_t s = 0; s < STAGES - 1; s += 1) {
        if (s < nstage) {
            issue_next(s);
        }
    }
    uint32_t ibuf = (STAGES - 1) % STAGES;  // buffer of the next stage to issue
    uint32_t cbuf = 0;                      // buffer of the stage to multiply
    uint32_t gs = 0;
    // steady state: STAGES-2 later stages in flight and one to issue
    const uint32_t steady = nstage > STAGES - 1 ? nstage - (STAGES - 1) : 0;
#pragma nounroll
    for (; gs < steady; gs += 1) {
        if (b_hi) {
            wait_vm<(STAGES - 2) * LHI>();
        } else {
            wait_vm<(STAGES - 2) * LLO>();
        }
        lds_barrier();
        // MFMA groups and this wave's DMA instructions alternate: issuing
        // DMA stalls while the CU's load path drains other waves' requests,
        // and the stall then overlaps MFMAs already in the pipe
        load_frags(cbuf, fa0, fb0);
        cbuf = cbuf + 1 == STAGES ? 0 : cbuf + 1;
        compute_begin();
        issue_begin(ibuf);
        ibuf = ibuf + 1 == STAGES ? 0 : ibuf + 1;
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
            if ((uint32_t)i < nlive) {
                mfma_group(fa0, fb0, i);
            }
            if ((uint32_t)i < A_PER + B_HI) {
                issue_one((uint32_t)i);
            }
        }
        issue_end();
        compute_end();
    }
    // drain: nothing left to issue
#pragma nounroll
    for (; gs < nstage; gs += 1) {
        const uint32_t later = nstage - 1 - gs;
        if (b_hi) {
            wait_after<LHI>(later);
        } else {
            wait_after<LLO>(later);
        }
        lds_barrier();
        load_frags(cbuf, fa0, fb0);
        cbuf = cbuf + 1 == STAGES ? 0 : cbuf + 1;
        compute(fa0, fb0);
    }
    if (SC && MODE == RMDA_GEMM_SWIGLU) {
        rmda_wave_amax(g.hp_amax, hmax_run);
    }
}

// Folded combine (rmda_fc_t), one token's 8 columns [col, col + 8): its
// selected rows in j order, then the sigmoid-gated shared row, summed exactly
// as combine16_kernel sums them.  The rows were stored by other waves, maybe
// on other XCDs, with device-scope stores: they are read at device scope.
__device__ __forceinline__ uint4 fc_load16(const uint16_t *p) {
    const uint64_t *q = reinterpret_cast<const uint64_t *>(p);
    const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
}

__device__ __forceinline__ void fc_combine8(const rmda_gemm_args_t &g, const uint16_t *ye, uint32_t tk, uint32_t col) {
    const rmda_fc_t &f = g.fc;
    const uint32_t d = g.n_w;
    float acc[8];
#pragma unroll
    for (int v = 0; v < 8; v += 1) {
        acc[v] = 0.0f;
    }
    for (uint32_t j = 0; j < f.topk; j += 1) {
        const uint32_t s = f.slot[(size_t)tk * f.topk + j];
        if (s == RMDA_NONE) {
            continue;
        }
        rmda_comb_acc8(acc, f.wt[(size_t)tk * f.topk + j], fc_load16(ye + (size_t)s * g.ldo + col));
    }
    if (f.has_shared) {
        rmda_comb_acc8(acc, rmda_sigmoidf(f.proj[(size_t)tk * f.pstride + f.sg_off]),
                       fc_load16(ye + (size_t)(g.shared_row0 + tk) * g.ldo + col));
    }
    if (f.out != nullptr) {
        *reinterpret_cast<uint4 *>(f.out + (size_t)tk * d + col) = rmda_pack8_f16(acc);
    }
    if (f.hc.h != nullptr) {
        for (uint32_t st = 0; st < f.hc.hc; st += 1) {
            const float gate =
                2.0f * rmda_sigmoidf(f.hc.inj[(size_t)tk * f.hc.inj_stride + f.hc.inj_off + st] / (float)f.hc.hc);
            rmda_hc_acc8(f.hc.h + ((size_t)tk * f.hc.hc + st) * d + col, acc, gate);
        }
    }
}

// The arrival step, run by one MFMA wave right after it stored columns
// [cb * 64, cb * 64 + 64) of its 64 rows of a task (rows [row0, row0 + rows)
// of the sorted row space; lane l holds tile row r = the wave's first row + l).
// Ordering: the wave's device-scope ye stores are acknowledged at the device
// coherence point before s_waitcnt vmcnt(0) lets the counter decrements issue
// (the MFMA waves have no other vector-memory operations outstanding), so a
// wave that sees a counter reach zero issues its device-scope loads only after
// every row of that counter was stored and acknowledged.  No fence: an
// agent-scope release/acquire would write back and invalidate this XCD's
// whole L2 on every task.
__device__ __forceinline__ void fc_arrive(const rmda_gemm_args_t &g, const uint16_t *ye, uint32_t row0, uint32_t rows,
                                          bool shared, uint32_t cb, uint32_t r, uint32_t lane, uint32_t *list) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const rmda_fc_t &f = g.fc;
    bool last = false;
    uint32_t t = 0;
    if (r < rows) {
        const uint32_t row = row0 + r;
        t = shared ? row - g.shared_row0 : f.rowtok[row];
        last = __hip_atomic_fetch_sub(&f.cnt[(size_t)t * f.nblk + cb], 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == 1u;
    }
    const uint64_t mask = __ballot(last);
    if (mask == 0) {
        return;
    }
    // the tokens this wave completes, compacted into its LDS list
    const uint32_t pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
    if (last) {
        list[pos] = t;
    }
    __builtin_amdgcn_wave_barrier();
    // 8 lanes per token, 8 columns (16 bytes) per lane, 8 tokens at a time
    const uint32_t n = (uint32_t)__popcll(mask);
    const uint32_t q = lane / 8;
    const uint32_t col = cb * RMDA_FC_COLS + (lane % 8) * 8;
    for (uint32_t b0 = 0; b0 < n; b0 += 8) {
        if (b0 + q < n) {
            fc_combine8(g, ye, list[b0 + q], col);
        }
    }
}

// One task's work item as the MFMA waves need it (scalar loads).
struct task_desc_t {
    uint32_t grp, row0, rows, nt;
};
__device__ __forceinline__ task_desc_t task_desc(const task_sched_t &sched, const_u32p items, uint32_t q) {
    task_desc_t t;
    const uint32_t item = sched.item(q, t.nt);
    t.grp = items[item * 4 + 0];
    t.row0 = items[item * 4 + 1];
    t.rows = items[item * 4 + 2];
    return t;
}

// Dedicated-issue variant: the 12 MFMA waves issue no loads; NDW more waves
// issue every stage's DMA (A rows and packed B slabs) and do nothing else.
// Each stage: the issue waves wait for their loads of stage g (exact vmcnt:
// every issue wave issues the same L_PER loads per stage), all waves meet
// at the stage barrier, then the issue waves put stage g + STAGES - 1 into
// the buffer stage g - 1 used while the MFMA waves multiply stage g.  So a
// stage's loads go out right after the barrier instead of between MFMA
// groups, and no MFMA wave waits on vmcnt.  Packed weights only.
//
// FC (F16 mode): the combine folded in (rmda_fc_t).  The MFMA waves store
// their ye tile with device-scope stores, wait for them, take one from the
// arrival counter of each stored row's (token, 64 columns), and the wave that
// takes a counter's last one sums that token's rows for its 64 columns.
template <int MODE, int STAGES, int BPOL, int NDW, bool DB, bool FC = false, bool SC = false, bool YNT = false>
__global__ __launch_bounds__(1024) void gemm3_kernel(rmda_gemm_args_t g) {
    constexpr uint32_t BN = 256;
    constexpr uint32_t BK = 32;
    constexpr uint32_t MB = BM / 64;
    constexpr uint32_t NB = BN / 64;
    constexpr uint32_t NMW = MB * NB;           // 12 MFMA waves
    constexpr uint32_t CH = BK / 8;             // 16-byte chunks per row
    constexpr uint32_t RPI = 64 / CH;           // rows per wave-wide DMA instruction
    constexpr uint32_t A_BYTES = BM * BK * 2;
    constexpr uint32_t B_BYTES = BN * BK * 2;
    constexpr uint32_t STAGE_BYTES = A_BYTES + B_BYTES;
    constexpr uint32_t A_PER = BM / RPI / NDW;  // A instructions per issue wave per stage
    constexpr uint32_t B_PER = BN / RPI / NDW;  // B instructions per issue wave per stage
    constexpr uint32_t L_PER = A_PER + B_PER;
    constexpr uint32_t AROWS = A_PER * RPI;     // A rows per issue wave
    static_assert(BM / RPI % NDW == 0 && BN / RPI % NDW == 0, "issue waves split a stage evenly");
    static_assert(AROWS <= 48, "gathered rows per issue wave");
    constexpr uint32_t A_STEP = MODE == RMDA_GEMM_F16 ? RMDA_HP_ROWS * BK : BK;  // hp is in 16 x 32 blocks
    static_assert((NMW + NDW) * RMDA_WAVE <= 1024, "workgroup size");
    static_assert(!FC || MODE == RMDA_GEMM_F16, "the combine folds into the down GEMM only");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE_BYTES];
    __shared__ uint32_t fc_list[FC ? NMW * RMDA_WAVE : 1];  // per MFMA wave: tokens whose counter it emptied

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % RMDA_WAVE;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid / RMDA_WAVE);

    // ---- this workgroup's tasks (task_sched_t) ----
    const_u32p items = (const_u32p)g.items;
    // the slot-scaled mode's inverse scales (1 otherwise, which changes no bits)
    const float xinv = SC && MODE == RMDA_GEMM_SWIGLU ? rmda_slot_inv(g.xscale) : 1.0f;
    const float yinv = down_mul<SC, MODE>(g);
    const uint32_t n_slabs = g.n_w / SLAB;
    const uint32_t ntiles = n_slabs / (BN / SLAB);
    const uint32_t n_items = g.n_items != nullptr ? *(const_u32p)g.n_items : g.max_items;
    const task_sched_t sched(n_items, ntiles);
    const uint32_t ntask = sched.ntask;
    if (ntask == 0) {
        return;
    }
    const uint32_t steps = g.k / BK;
    const uint32_t nstage = ntask * steps;

    if (w >= NMW) {
        // ================= issue waves =================
        const uint32_t dw = w - NMW;
        const uint32_t lrow = lane / CH;
        const uint32_t lch = lane % CH;
        const uint16_t *a_src[A_PER];
        const uint16_t *b_src[B_PER];
        auto setup = [&](uint32_t k) __attribute__((always_inline)) {
            uint32_t nt;
            const uint32_t item = sched.item(k, nt);
            const uint32_t grp = items[item * 4 + 0];
            const uint32_t row0 = items[item * 4 + 1];
            const uint32_t rows = items[item * 4 + 2];
            const bool is_shared = grp == g.shared_group;
            const uint16_t *wg = is_shared ? g.w_shared : g.w + (size_t)grp * g.n_w * g.k;
            const uint32_t rbase = dw * AROWS;
#pragma unroll
            for (uint32_t j = 0; j < A_PER; j += 1) {
                const uint32_t r = rbase + j * RPI + lrow;
                const uint32_t rr = r < rows ? r : 0u;
                uint32_t arow;
                if (MODE == RMDA_GEMM_SWIGLU) {
                    if (is_shared) {
                        arow = row0 + rr - g.shared_row0;
                    } else {
                        // gathered token rows (scalar loads; the index buffer is
                        // padded so these reads never leave it)
                        const const_u32p rt = (const_u32p)g.rowtok + row0 + rbase + j * RPI;
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
                } else {
                    arow = row0 + rr;
                }
                if (MODE == RMDA_GEMM_F16) {
                    const uint32_t blk = rbase + j * RPI;
                    a_src[j] = g.a + rmda_hp_index(row0 + (blk < rows ? blk : 0u), 0, g.lda) + lrow * 32 +
                               (lch ^ swz<BK>(r)) * 8;
                } else {
                    a_src[j] = g.a + (size_t)arow * g.lda + (lch ^ swz<BK>(r)) * 8;
                }
            }
#pragma unroll
            for (uint32_t j = 0; j < B_PER; j += 1) {
                const uint32_t nbase = (dw * B_PER + j) * RPI;
                const uint32_t slab = nt * (BN / SLAB) + nbase / SLAB;
                const uint32_t nin = nbase % SLAB;
                b_src[j] = wg + (size_t)slab * steps * (SLAB * BK) + nin * BK + lane * 8;
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
                                                 (lds_void_t *)(base + (dw * AROWS + j * RPI) * (BK * 2)), 16, 0, 0);
            }
#pragma unroll
            for (uint32_t j = 0; j < B_PER; j += 1) {
                __builtin_amdgcn_global_load_lds((const void *)(b_src[j] + (size_t)i_s * (SLAB * BK)),
                                                 (lds_void_t *)(base + A_BYTES + (dw * B_PER + j) * RPI * (BK * 2)),
                                                 16, 0, BPOL);
            }
            i_s += 1;
        };
        // DB: a second barrier per stage, after the MFMA waves have read the
        // stage's fragments into registers, frees its buffer before the
        // MFMAs run, so all STAGES buffers can be in flight
        constexpr uint32_t AHEAD = DB ? STAGES : STAGES - 1;
#pragma unroll
        for (uint32_t s = 0; s < AHEAD; s += 1) {
            if (s < nstage) {
                issue(s);
            }
        }
        uint32_t ibuf = AHEAD % STAGES;
        for (uint32_t gs = 0; gs < nstage; gs += 1) {
            const uint32_t later = min(nstage - 1 - gs, AHEAD - 1);
            wait_after<L_PER>(later);
            __builtin_amdgcn_s_barrier();
            if (DB) {
                __builtin_amdgcn_s_barrier();
            }
            if (gs + AHEAD < nstage) {
                issue(ibuf);
                ibuf = ibuf + 1 == STAGES ? 0 : ibuf + 1;
            }
        }
        return;
    }

    // ================= MFMA waves =================
    const uint32_t wm = w / NB;
    const uint32_t wn = w % NB;
    const uint32_t fr = lane % 16;
    const uint32_t fq = lane / 16;
    const uint32_t ch_off = (fq ^ swz<BK>(fr)) * 16;
    const uint32_t a_row_off = (wm * 64 + fr) * (BK * 2);
    const uint32_t b_row_off = A_BYTES + (wn * 64 + fr) * (BK * 2);
    const uint32_t rq = 4 * fq;
    floatx4_t acc[4][4];
    float hmax_run = 0.0f;  // slot-scaled mode: this lane's largest |SwiGLU| over its tasks
    uint32_t c_row0 = 0;
    uint32_t c_rows = 0;
    uint32_t c_nt = 0;
    bool c_shared = false;
    uint32_t kc = 0;
    uint32_t ks = 0;
    bool live = false;
    uint32_t nlive = 0;
    uint32_t cbuf = 0;
    // the next task's descriptor, read one stage before its first K step, so
    // that step's fragment reads already know which row groups are live
    task_desc_t nx = task_desc(sched, items, 0u);
    for (uint32_t gs = 0; gs < nstage; gs += 1) {
        lds_barrier();
        const uint8_t *base = smem + cbuf * STAGE_BYTES;
        cbuf = cbuf + 1 == STAGES ? 0 : cbuf + 1;
        if (ks == 0) {
            c_row0 = nx.row0;
            c_rows = nx.rows;
            c_nt = nx.nt;
            if (FC) {
                c_shared = nx.grp == g.shared_group;
            }
            live = wm * 64 < c_rows;
            nlive = live ? min(4u, (c_rows - wm * 64 + 15) / 16) : 0u;
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
#pragma unroll
                for (int j = 0; j < 4; j += 1) {
                    acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
        // a wave whose rows all lie past the item reads no fragments
        half8_t fa[4], fb[4];
        if (live) {
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
                fa[i] = *reinterpret_cast<const half8_t *>(base + a_row_off + i * 16 * (BK * 2) + ch_off);
                fb[i] = *reinterpret_cast<const half8_t *>(base + b_row_off + i * 16 * (BK * 2) + ch_off);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
                fa[i] = half8_t{};
                fb[i] = half8_t{};
            }
        }
        if (DB) {
            lds_barrier();  // this stage's buffer is in registers: the issue waves may refill it
        }
        if (ks == steps - 1 && kc + 1 < ntask) {
            nx = task_desc(sched, items, kc + 1);
        }
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
            if ((uint32_t)i < nlive) {
#pragma unroll
                for (int j = 0; j < 4; j += 1) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (live && ks == steps - 1) {
            uint16_t *O = reinterpret_cast<uint16_t *>(g.out);
            if (MODE == RMDA_GEMM_F16) {
#pragma unroll
                for (int i = 0; i < 4; i += 1) {
#pragma unroll
                    for (int v = 0; v < 4; v += 1) {
                        const uint32_t rr = wm * 64 + i * 16 + rq + v;
                        if (rr < c_rows) {
#pragma unroll
                            for (int j = 0; j < 4; j += 1) {
                                const uint32_t col = c_nt * BN + wn * 64 + j * 16 + fr;
                                uint16_t *dst = &O[(size_t)(c_row0 + rr) * g.ldo + col];
                                if (FC) {
                                    // through to the device coherence point: the
                                    // token's combine may run on another XCD
                                    __hip_atomic_store(dst, rmda_f2h(acc[i][j][v] * yinv), __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
                                } else {
                                    down_store<SC, YNT>(g, O, (size_t)(c_row0 + rr) * g.ldo + col,
                                                        acc[i][j][v] * yinv);
                                }
                            }
                        }
                    }
                }
                if (FC) {
                    fc_arrive(g, O, c_row0, c_rows, c_shared, c_nt * (BN / RMDA_FC_COLS) + wn, wm * 64 + lane, lane,
                              fc_list + w * RMDA_WAVE);
                }
            } else {
                const uint32_t slab = c_nt * (BN / SLAB) + (wn * 64) / SLAB;
                const uint32_t colbase = slab * (SLAB / 2) + (((wn * 64) % SLAB) / 64) * 32;
#pragma unroll
                for (int i = 0; i < 4; i += 1) {
#pragma unroll
                    for (int v = 0; v < 4; v += 1) {
                        const uint32_t rr = wm * 64 + i * 16 + rq + v;
                        if (rr < c_rows) {
#pragma unroll
                            for (int j = 0; j < 2; j += 1) {
                                const float gt = acc[i][j][v] * xinv;
                                const float up = acc[i][j + 2][v] * xinv;
                                const float h = rmda_swiglu_fast(gt, up);
                                swiglu_store<SC, true>(g, O, rmda_hp_index(c_row0 + rr, colbase + j * 16 + fr, g.ldo), h, hmax_run);
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
    }
    if (SC && MODE == RMDA_GEMM_SWIGLU) {
        rmda_wave_amax(g.hp_amax, hmax_run);
    }
}

// gate_up with the gathered activation rows in a ring of their own, two K
// steps per slot.  gemm3_kernel fetches each gathered row as one 64-byte
// piece per K step; here every row is one 128-byte line per pair of K steps
// (8 rows per DMA instruction), so the activation rows need half the load
// requests.  Weights keep their STAGES-deep ring of one K step each.
//   * The six activation instructions of a pair (per issue wave) are issued
//     with the pair's first stage, into slot (pair % 3).  The slot's previous
//     pair was last read five stages earlier, before the barrier that lets
//     this stage be issued, so three slots cover the five stages in flight.
//   * Even stages carry 6 + 4 loads per issue wave, odd ones 4: any four
//     consecutive stages hold 28, so the waits stay compile-time constants.
//   * LDS: 5 x 16 KiB of weights + 3 x 24 KiB of activations = 152 KiB.  An
//     activation row is 128 bytes; chunk c of row r sits at c ^ ((r>>1)&7),
//     so each 16-lane fragment read touches 16 distinct bank groups.
// Needs k % 64 == 0 (pairs never straddle a task).
template <int STAGES, int BPOL, int NDW, bool SC = false>
__global__ __launch_bounds__(1024) void gemm4_kernel(rmda_gemm_args_t g) {
    constexpr uint32_t BN = 256;
    constexpr uint32_t BK = 32;
    constexpr uint32_t MB = BM / 64;
    constexpr uint32_t NB = BN / 64;
    constexpr uint32_t NMW = MB * NB;             // 12 MFMA waves
    constexpr uint32_t CH = BK / 8;               // 16-byte chunks per weight row
    constexpr uint32_t RPI = 64 / CH;             // weight rows per DMA instruction
    constexpr uint32_t B_BYTES = BN * BK * 2;     // one weight stage
    constexpr uint32_t B_PER = BN / RPI / NDW;    // weight instructions per issue wave per stage
    constexpr uint32_t AK = 2 * BK;               // activation slot: two K steps per row
    constexpr uint32_t ACH = AK / 8;              // 16-byte chunks per activation row
    constexpr uint32_t ARPI = 64 / ACH;           // activation rows per DMA instruction
    constexpr uint32_t A_SLOT = BM * AK * 2;
    constexpr uint32_t A_SLOTS = 3;
    constexpr uint32_t A_PER = BM / ARPI / NDW;   // activation instructions per issue wave per pair
    constexpr uint32_t AROWS = A_PER * ARPI;      // activation rows per issue wave
    constexpr uint32_t AHEAD = STAGES;            // two barriers per stage: every buffer in flight
    constexpr uint32_t LE = A_PER + B_PER;        // loads of an even (pair-opening) stage
    constexpr uint32_t LO = B_PER;                // loads of an odd stage
    static_assert(STAGES == 5 && 2 * A_SLOTS == AHEAD + 1, "slot reuse argument above");
    static_assert(BM % (ARPI * NDW) == 0 && BN / RPI % NDW == 0, "issue waves split a stage evenly");
    static_assert(2 * (LE + LO) < 64, "vmcnt range");
    static_assert((NMW + NDW) * RMDA_WAVE <= 1024, "workgroup size");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * B_BYTES + A_SLOTS * A_SLOT];
    uint8_t *const bring = smem;
    uint8_t *const aring = smem + STAGES * B_BYTES;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % RMDA_WAVE;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid / RMDA_WAVE);

    const_u32p items = (const_u32p)g.items;
    // the slot-scaled mode's inverse scale (1 otherwise, which changes no bits)
    const float xinv = SC ? rmda_slot_inv(g.xscale) : 1.0f;
    const uint32_t n_slabs = g.n_w / SLAB;
    const uint32_t ntiles = n_slabs / (BN / SLAB);
    const uint32_t n_items = g.n_items != nullptr ? *(const_u32p)g.n_items : g.max_items;
    const task_sched_t sched(n_items, ntiles);
    const uint32_t ntask = sched.ntask;
    if (ntask == 0) {
        return;
    }
    const uint32_t steps = g.k / BK;
    const uint32_t nstage = ntask * steps;

    if (w >= NMW) {
        // ================= issue waves =================
        const uint32_t dw = w - NMW;
        const uint32_t lrow = lane / ACH;  // activation row within one instruction
        const uint32_t lch = lane % ACH;   // its LDS chunk position
        const uint16_t *a_src[A_PER];
        const uint16_t *b_src[B_PER];
        auto setup = [&](uint32_t k) __attribute__((always_inline)) {
            uint32_t nt;
            const uint32_t item = sched.item(k, nt);
            const uint32_t grp = items[item * 4 + 0];
            const uint32_t row0 = items[item * 4 + 1];
            const uint32_t rows = items[item * 4 + 2];
            const bool is_shared = grp == g.shared_group;
            const uint16_t *wg = is_shared ? g.w_shared : g.w + (size_t)grp * g.n_w * g.k;
            const uint32_t rbase = dw * AROWS;
#pragma unroll
            for (uint32_t j = 0; j < A_PER; j += 1) {
                const uint32_t r = rbase + j * ARPI + lrow;
                uint32_t arow;
                if (is_shared) {
                    arow = row0 + (r < rows ? r : 0u) - g.shared_row0;
                } else {
                    const const_u32p rt = (const_u32p)g.rowtok + row0 + rbase + j * ARPI;
                    uint32_t tok[ARPI];
#pragma unroll
                    for (uint32_t c = 0; c < ARPI; c += 1) {
                        tok[c] = rt[c];
                    }
                    uint32_t t = tok[0];
#pragma unroll
                    for (uint32_t c = 1; c < ARPI; c += 1) {
                        t = lrow == c ? tok[c] : t;
                    }
                    arow = r < rows ? t : ((const_u32p)g.rowtok + row0)[0];
                    arow = arow < g.a_rows ? arow : 0u;  // a bad index reads a valid row, never out of bounds
                }
                a_src[j] = g.a + (size_t)arow * g.lda + (lch ^ swz<AK>(r)) * 8;
            }
#pragma unroll
            for (uint32_t j = 0; j < B_PER; j += 1) {
                const uint32_t nbase = (dw * B_PER + j) * RPI;
                const uint32_t slab = nt * (BN / SLAB) + nbase / SLAB;
                const uint32_t nin = nbase % SLAB;
                b_src[j] = wg + (size_t)slab * steps * (SLAB * BK) + nin * BK + lane * 8;
            }
        };
        uint32_t i_task = 0;
        uint32_t i_s = 0;
        uint32_t aslot = 0;
        setup(0);
        auto issue = [&](uint32_t buf) __attribute__((always_inline)) {
            if (i_s == steps) {
                i_task += 1;
                i_s = 0;
                setup(i_task);
            }
            // activation rows first (weights first measured slower at config 3)
            if ((i_s & 1u) == 0) {
                uint8_t *abase = aring + aslot * A_SLOT;
                aslot = aslot + 1 == A_SLOTS ? 0 : aslot + 1;
#pragma unroll
                for (uint32_t j = 0; j < A_PER; j += 1) {
                    __builtin_amdgcn_global_load_lds((const void *)(a_src[j] + (i_s / 2) * AK),
                                                     (lds_void_t *)(abase + (dw * AROWS + j * ARPI) * (AK * 2)),
                                                     16, 0, 0);
                }
            }
            uint8_t *bbase = bring + buf * B_BYTES;
#pragma unroll
            for (uint32_t j = 0; j < B_PER; j += 1) {
                __builtin_amdgcn_global_load_lds((const void *)(b_src[j] + (size_t)i_s * (SLAB * BK)),
                                                 (lds_void_t *)(bbase + (dw * B_PER + j) * RPI * (BK * 2)), 16,
                                                 0, BPOL);
            }
            i_s += 1;
        };
#pragma unroll
        for (uint32_t st = 0; st < AHEAD; st += 1) {
            if (st < nstage) {
                issue(st);
            }
        }
        uint32_t ibuf = AHEAD % STAGES;
        for (uint32_t gs = 0; gs < nstage; gs += 1) {
            // stage gs has landed once only the loads of the `later` stages
            // issued after it remain; their count depends on gs's parity
            const uint32_t later = min(nstage - 1 - gs, AHEAD - 1);
            const bool odd = (gs & 1u) != 0;
            switch (later) {
            case 0: wait_vm<0>(); break;
            case 1:
                if (odd) {
                    wait_vm<LE>();
                } else {
                    wait_vm<LO>();
                }
                break;
            case 2: wait_vm<LE + LO>(); break;
            case 3:
                if (odd) {
                    wait_vm<LE + LO + LE>();
                } else {
                    wait_vm<LO + LE + LO>();
                }
                break;
            default: wait_vm<2 * (LE + LO)>(); break;
            }
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_s_barrier();
            if (gs + AHEAD < nstage) {
                issue(ibuf);
                ibuf = ibuf + 1 == STAGES ? 0 : ibuf + 1;
            }
        }
        return;
    }

    // ================= MFMA waves =================
    const uint32_t wm = w / NB;
    const uint32_t wn = w % NB;
    const uint32_t fr = lane % 16;
    const uint32_t fq = lane / 16;
    // activation fragment of K step half h: chunk 4h + fq of row wm*64 + 16i + fr
    const uint32_t a_row = (wm * 64 + fr) * (AK * 2);
    const uint32_t a_off0 = a_row + ((0u + fq) ^ swz<AK>(fr)) * 16;
    const uint32_t a_off1 = a_row + ((4u + fq) ^ swz<AK>(fr)) * 16;
    const uint32_t b_off = (wn * 64 + fr) * (BK * 2) + (fq ^ swz<BK>(fr)) * 16;
    const uint32_t rq = 4 * fq;
    floatx4_t acc[4][4];
    float hmax_run = 0.0f;  // slot-scaled mode: this lane's largest |SwiGLU| over its tasks
    uint32_t c_row0 = 0;
    uint32_t c_rows = 0;
    uint32_t c_nt = 0;
    uint32_t kc = 0;
    uint32_t ks = 0;
    bool live = false;
    uint32_t nlive = 0;
    uint32_t cbuf = 0;
    uint32_t abuf = 0;
    // the next task's descriptor, read one stage before its first K step
    task_desc_t nx = task_desc(sched, items, 0u);
    for (uint32_t gs = 0; gs < nstage; gs += 1) {
        lds_barrier();
        const uint8_t *bb = bring + cbuf * B_BYTES + b_off;
        const uint8_t *ab = aring + abuf * A_SLOT + ((gs & 1u) != 0 ? a_off1 : a_off0);
        cbuf = cbuf + 1 == STAGES ? 0 : cbuf + 1;
        if ((gs & 1u) != 0) {
            abuf = abuf + 1 == A_SLOTS ? 0 : abuf + 1;
        }
        if (ks == 0) {
            c_row0 = nx.row0;
            c_rows = nx.rows;
            c_nt = nx.nt;
            live = wm * 64 < c_rows;
            nlive = live ? min(4u, (c_rows - wm * 64 + 15) / 16) : 0u;
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
#pragma unroll
                for (int j = 0; j < 4; j += 1) {
                    acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
        // a wave whose rows all lie past the item reads no fragments
        half8_t fa[4], fb[4];
        if (live) {
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
                fa[i] = *reinterpret_cast<const half8_t *>(ab + i * 16 * (AK * 2));
                fb[i] = *reinterpret_cast<const half8_t *>(bb + i * 16 * (BK * 2));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
                fa[i] = half8_t{};
                fb[i] = half8_t{};
            }
        }
        lds_barrier();  // both buffers are in registers: the issue waves may refill them
        if (ks == steps - 1 && kc + 1 < ntask) {
            nx = task_desc(sched, items, kc + 1);
        }
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
            if ((uint32_t)i < nlive) {
#pragma unroll
                for (int j = 0; j < 4; j += 1) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (live && ks == steps - 1) {
            uint16_t *O = reinterpret_cast<uint16_t *>(g.out);
            const uint32_t slab = c_nt * (BN / SLAB) + (wn * 64) / SLAB;
            const uint32_t colbase = slab * (SLAB / 2) + (((wn * 64) % SLAB) / 64) * 32;
#pragma unroll
            for (int i = 0; i < 4; i += 1) {
#pragma unroll
                for (int v = 0; v < 4; v += 1) {
                    const uint32_t rr = wm * 64 + i * 16 + rq + v;
                    if (rr < c_rows) {
#pragma unroll
                        for (int j = 0; j < 2; j += 1) {
                            const float gt = acc[i][j][v] * xinv;
                            const float up = acc[i][j + 2][v] * xinv;
                            const float h = rmda_swiglu_fast(gt, up);
                            swiglu_store<SC, true>(g, O, rmda_hp_index(c_row0 + rr, colbase + j * 16 + fr, g.ldo), h, hmax_run);
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
    if (SC) {
        rmda_wave_amax(g.hp_amax, hmax_run);
    }
}

// Packed slab image: for slab t (128 B rows) and K step ks, 16-byte unit
// (n, p) holds B[slab_row(t, n)][ks*BK + (p ^ swz(n))*8 .. +8], at unit
// index ((t * steps + ks) * 128 + n) * (BK/8) + p.
template <int MODE, int BK>
__global__ __launch_bounds__(256) void pack_kernel(const uint16_t *__restrict__ src, uint16_t *__restrict__ dst,
                                                   uint32_t groups, uint32_t n_w, uint32_t k, uint32_t inter,
                                                   int bf16_in) {
    constexpr uint32_t CH = BK / 8;
    const uint64_t per_group = (uint64_t)n_w * k / 8;  // 16-byte units
    const uint64_t total = per_group * groups;
    const uint32_t steps = k / BK;
    for (uint64_t u = (uint64_t)blockIdx.x * 256 + threadIdx.x; u < total; u += (uint64_t)gridDim.x * 256) {
        const uint64_t gi = u / per_group;
        const uint64_t r = u % per_group;
        const uint32_t p = (uint32_t)(r % CH);
        const uint32_t n = (uint32_t)((r / CH) % SLAB);
        const uint64_t ts = r / (CH * SLAB);
        const uint32_t ks = (uint32_t)(ts % steps);
        const uint32_t t = (uint32_t)(ts / steps);
        const uint32_t row = slab_row<MODE>(t, n, inter);
        const uint32_t col = ks * BK + (p ^ swz<BK>(n)) * 8;
        const uint4 v = *reinterpret_cast<const uint4 *>(src + (gi * n_w + row) * k + col);
        uint4 o = v;
        if (bf16_in) {
            const uint32_t in[4] = {v.x, v.y, v.z, v.w};
            uint32_t out[4];
#pragma unroll
            for (int q = 0; q < 4; q += 1) {
                const float lo = __builtin_bit_cast(float, in[q] << 16);
                const float hi = __builtin_bit_cast(float, in[q] & 0xffff0000u);
                out[q] = (uint32_t)rmda_f2h(lo) | ((uint32_t)rmda_f2h(hi) << 16);
            }
            o = make_uint4(out[0], out[1], out[2], out[3]);
        }
        reinterpret_cast<uint4 *>(dst)[u] = o;
    }
}

// The largest row sum of |w| over `groups` packed F16-mode matrices [n_w][k]
// (the down weights; one thread per weight row, its slab row's 64 bytes per
// K step, so a wave reads whole lines), rows whose sum is not finite left
// out, as float bits: a wave maximum, then one atomicMax per wave.
template <int BK>
__global__ __launch_bounds__(256) void row_abs_kernel(const uint16_t *__restrict__ packed, uint32_t groups,
                                                      uint32_t n_w, uint32_t k, uint32_t *__restrict__ bound) {
    constexpr uint32_t CH = BK / 8;
    const uint32_t steps = k / BK;
    const uint64_t rows = (uint64_t)groups * n_w;
    const uint4 *units = reinterpret_cast<const uint4 *>(packed);
    float m = 0.0f;
    for (uint64_t q = (uint64_t)blockIdx.x * 256 + threadIdx.x; q < rows; q += (uint64_t)gridDim.x * 256) {
        const uint64_t gi = q / n_w;
        const uint32_t r = (uint32_t)(q % n_w);
        // unit (gi, t, ks, n, p) = gi * n_w * k / 8 + ((t * steps + ks) * SLAB + n) * CH + p
        const uint4 *u = units + gi * n_w * k / 8 + ((uint64_t)(r / SLAB) * steps * SLAB + r % SLAB) * CH;
        float sum = 0.0f;
        for (uint32_t ks = 0; ks < steps; ks += 1) {
#pragma unroll
            for (uint32_t p = 0; p < CH; p += 1) {
                const uint4 v = u[(size_t)ks * SLAB * CH + p];
                const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int i = 0; i < 4; i += 1) {
                    sum += fabsf(rmda_h2f((uint16_t)(w4[i] & 0xffffu))) + fabsf(rmda_h2f((uint16_t)(w4[i] >> 16)));
                }
            }
        }
        if (sum <= 3.4028235e38f) {  // false for inf and NaN
            m = fmaxf(m, sum);
        }
    }
    const uint32_t b = rmda_wave_red_u32<true>(__builtin_bit_cast(uint32_t, m));
    if (threadIdx.x % RMDA_WAVE == 0) {
        atomicMax(bound, b);
    }
}

template <int MODE, int BN, int BK, int STAGES, int BPOL, bool SC = false>
hipError_t launch_cfg(hipStream_t s, const rmda_gemm_args_t *a, dim3 grid, bool packed) {
    if (packed) {
        hipLaunchKernelGGL((gemm2_kernel<MODE, BN, BK, STAGES, true, BPOL, SC>), grid, dim3(BM / 64 * BN), 0, s, *a);
    } else {
        hipLaunchKernelGGL((gemm2_kernel<MODE, BN, BK, STAGES, false, BPOL, SC>), grid, dim3(BM / 64 * BN), 0, s, *a);
    }
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_mode(hipStream_t s, const rmda_gemm_args_t *a, const rmda_gemm2_cfg_t &c, bool packed) {
    if (a->max_items == 0) {
        return hipSuccess;
    }
    // persistent: one workgroup per CU, a multiple of the 8 XCDs
    const uint32_t wgs = c.grid >= 8 ? c.grid / 8 * 8 : 8;
    const dim3 grid(wgs);
    // the slot-scaled mode (fp32 SwiGLU output; fp32 rows, or fp16 rows under
    // the weights' bound) has its own instantiations, of the default
    // configurations only
    const bool sc = a->hp32 != nullptr || a->ye32 != nullptr || a->ye_bound != nullptr;
    if (sc) {
        if ((MODE == RMDA_GEMM_SWIGLU) != (a->hp32 != nullptr) ||
            (MODE == RMDA_GEMM_F16) != ((a->ye32 != nullptr) != (a->ye_bound != nullptr)) || a->fc.cnt != nullptr) {
            return hipErrorInvalidValue;
        }
        if (c.spec == 0 || !packed) {
            if (c.stages != 5 || c.bpol != 2) {
                return hipErrorInvalidValue;
            }
            return launch_cfg<MODE, 256, 32, 5, 2, true>(s, a, grid, packed);
        }
        if (c.spec == 7 && MODE == RMDA_GEMM_SWIGLU && a->k % 64 == 0) {
            hipLaunchKernelGGL((gemm4_kernel<5, 2, 4, true>), grid, dim3(16 * RMDA_WAVE), 0, s, *a);
        } else if (c.spec != 4 && MODE == RMDA_GEMM_F16 && a->ye_nt != 0) {
            hipLaunchKernelGGL((gemm3_kernel<MODE, 5, 2, 4, true, false, true, true>), grid, dim3(16 * RMDA_WAVE), 0,
                               s, *a);
        } else if (c.spec != 4) {
            hipLaunchKernelGGL((gemm3_kernel<MODE, 5, 2, 4, true, false, true>), grid, dim3(16 * RMDA_WAVE), 0, s,
                               *a);
        } else {
            hipLaunchKernelGGL((gemm3_kernel<MODE, 5, 2, 4, false, false, true>), grid, dim3(16 * RMDA_WAVE), 0, s,
                               *a);
        }
        return hipGetLastError();
    }
    if (c.spec != 0 && packed) {
        if (c.spec == 7 && MODE == RMDA_GEMM_SWIGLU && a->k % 64 == 0) {
            hipLaunchKernelGGL((gemm4_kernel<5, 2, 4>), grid, dim3(16 * RMDA_WAVE), 0, s, *a);
            return hipGetLastError();
        }
        if (a->fc.cnt != nullptr) {
            if (MODE != RMDA_GEMM_F16 || c.spec == 5 || a->n_w % RMDA_FC_COLS != 0) {
                return hipErrorInvalidValue;
            }
            hipLaunchKernelGGL((gemm3_kernel<RMDA_GEMM_F16, 5, 2, 4, false, true>), grid, dim3(16 * RMDA_WAVE), 0,
                               s, *a);
            return hipGetLastError();
        }
        if (c.spec != 4 && MODE == RMDA_GEMM_F16 && a->ye_nt != 0) {
            hipLaunchKernelGGL((gemm3_kernel<MODE, 5, 2, 4, true, false, false, true>), grid, dim3(16 * RMDA_WAVE), 0,
                               s, *a);
        } else if (c.spec != 4) {
            hipLaunchKernelGGL((gemm3_kernel<MODE, 5, 2, 4, true>), grid, dim3(16 * RMDA_WAVE), 0, s, *a);
        } else {
            hipLaunchKernelGGL((gemm3_kernel<MODE, 5, 2, 4, false>), grid, dim3(16 * RMDA_WAVE), 0, s, *a);
        }
        return hipGetLastError();
    }
    if (a->fc.cnt != nullptr) {
        return hipErrorInvalidValue;  // the folded combine runs on the dedicated-issue kernel only
    }
    if (c.stages == 4) {
        return launch_cfg<MODE, 256, 32, 4, 2>(s, a, grid, packed);
    }
    if (c.bpol == 0) {
        return launch_cfg<MODE, 256, 32, 5, 0>(s, a, grid, packed);
    }
    return launch_cfg<MODE, 256, 32, 5, 2>(s, a, grid, packed);
}

}  // namespace

// Variant 0 is the default: the fastest configuration measured on MI355X at
// the benchmark shapes (packed weights run the dedicated-issue kernel, with
// the second per-stage barrier for both GEMMs, and the layer switches
// gate_up to the activation-ring kernel when experts average 32 rows or
// more; HF-layout weights always run gemm2_kernel).  The others are kept for
// measurement.  LDS per workgroup =
// STAGES * (192 + BN) * BK * 2.
rmda_gemm2_cfg_t rmda_gemm2_variant(int variant) {
    switch (variant) {
    case 1: return {256, 32, 5, 0, 2, 0};  // every MFMA wave issues its share of the loads
    case 2: return {256, 32, 4, 0, 2, 0};  // the same with 4 stages
    case 3: return {256, 32, 5, 0, 0, 0};  // the same without the non-temporal weight hint
    case 4: return {256, 32, 5, 0, 2, 4};  // dedicated issue waves, one barrier per stage
    case 5: return {256, 32, 5, 0, 2, 5};  // the default without the activation-ring switch
    case 7: return {256, 32, 5, 0, 2, 7};  // gate_up with its activation rows in a two-K-step ring
    default: return {256, 32, 5, 0, 2, 6};
    }
}

hipError_t rmda_launch_gemm2(hipStream_t s, const rmda_gemm_args_t *a, rmda_gemm2_cfg_t c, int packed) {
    if (a->k % c.bk != 0 || a->n_w % SLAB != 0) {
        return hipErrorInvalidValue;
    }
    if ((a->n_w / SLAB) % (c.bn / SLAB) != 0) {
        return hipErrorInvalidValue;  // an N tile is two 128-row slabs
    }
    if (a->mode == RMDA_GEMM_SWIGLU) {
        return launch_mode<RMDA_GEMM_SWIGLU>(s, a, c, packed != 0);
    }
    return launch_mode<RMDA_GEMM_F16>(s, a, c, packed != 0);
}

hipError_t rmda_launch_row_abs_max(hipStream_t s, const uint16_t *packed, uint32_t groups, uint32_t n_w, uint32_t k,
                                   int bk, uint32_t *bound) {
    const uint64_t rows = (uint64_t)groups * n_w;
    if (rows == 0) {
        return hipSuccess;
    }
    if (n_w % SLAB != 0 || k % bk != 0 || (bk != 32 && bk != 64)) {
        return hipErrorInvalidValue;
    }
    const dim3 grid((uint32_t)std::min<uint64_t>((rows + 255) / 256, 4096));
    if (bk == 64) {
        hipLaunchKernelGGL(row_abs_kernel<64>, grid, dim3(256), 0, s, packed, groups, n_w, k, bound);
    } else {
        hipLaunchKernelGGL(row_abs_kernel<32>, grid, dim3(256), 0, s, packed, groups, n_w, k, bound);
    }
    return hipGetLastError();
}

hipError_t rmda_launch_pack(hipStream_t s, const uint16_t *src, uint16_t *dst, uint32_t groups, uint32_t n_w,
                            uint32_t k, uint32_t inter, int swiglu, int bk, int bf16_in) {
    const uint64_t units = (uint64_t)groups * n_w * k / 8;
    if (units == 0) {
        return hipSuccess;
    }
    if (n_w % SLAB != 0 || k % bk != 0) {
        return hipErrorInvalidValue;
    }
    uint64_t blocks = (units + 255) / 256;
    if (blocks > 16384) {
        blocks = 16384;
    }
    const dim3 grid((uint32_t)blocks);
    if (swiglu) {
        if (bk == 64) {
            hipLaunchKernelGGL((pack_kernel<RMDA_GEMM_SWIGLU, 64>), grid, dim3(256), 0, s, src, dst, groups, n_w, k,
                               inter, bf16_in);
        } else {
            hipLaunchKernelGGL((pack_kernel<RMDA_GEMM_SWIGLU, 32>), grid, dim3(256), 0, s, src, dst, groups, n_w, k,
                               inter, bf16_in);
        }
    } else {
        if (bk == 64) {
            hipLaunchKernelGGL((pack_kernel<RMDA_GEMM_F16, 64>), grid, dim3(256), 0, s, src, dst, groups, n_w, k,
                               inter, bf16_in);
        } else {
            hipLaunchKernelGGL((pack_kernel<RMDA_GEMM_F16, 32>), grid, dim3(256), 0, s, src, dst, groups, n_w, k,
                               inter, bf16_in);
        }
    }
    return hipGetLastError();
}
