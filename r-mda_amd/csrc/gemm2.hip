// Grouped expert GEMM of the fused layer: weight-streaming design for gfx950.
// Serves the gate_up GEMM (SwiGLU epilogue) and the down GEMM, and packs the
// expert weights into the order it streams them.
//
// Why this shape.  At the benchmark shapes every expert's weight slice is
// needed by ~128 token rows, so the GEMM is bound by streaming the weights
// from HBM (arithmetic intensity ~120 FLOP/B against a ridge of ~312).  Two
// things decide the speed: every weight byte leaves HBM once, and enough
// bytes are in flight to cover HBM latency.
//   * A work item is (group, first row, up to 256 rows): one workgroup owns
//     all rows of an expert (up to 256) for one BN-wide N tile, so each
//     weight tile is read once.  The 256 rows are four 64-row blocks; a block
//     past the item's end loads no A rows and runs no MFMAs (tile height
//     follows the expert's load at 64-row grain).
//   * Operand tiles go straight from global memory into LDS with gfx950's
//     global_load_lds_dwordx4 (no register staging), through a ring of
//     STAGES buffers; while stage s is multiplied, the next STAGES-1 stages
//     are in flight.  Completion is tracked per wave with explicit vmcnt
//     waits (each wave knows how many loads it issued per stage) and a bare
//     s_barrier, so no compiler-inserted full wait drains the pipeline.
//   * LDS rows are BK halves; the 16-byte chunks of row r sit XOR-swizzled
//     (swz below) so MFMA fragment reads are free of bank conflicts.  A DMA
//     instruction writes 64 consecutive 16-byte slots, so the swizzle is
//     applied on the global side: each lane fetches the chunk that belongs
//     at its slot.
//   * Packed weights (rmda_moe_pack_weights) store every 128-row x BK slab
//     in exactly its LDS image order, so each DMA instruction reads one
//     contiguous KiB and a whole stage of B is one contiguous block (the
//     HF [out][in] layout would read BK-wide pieces of 128 rows 4-8 KiB
//     apart).
//   * The grid is renumbered XCD-aware from the real work count read on the
//     device: XCD x gets a contiguous range of (item, N tile) pairs, so the N
//     tiles of one item (which share A rows) meet in one L2 and the 8 XCDs
//     get equal shares whatever the routing.
// MFMA: v_mfma_f32_16x16x32_f16, fp32 accumulate; 8 waves = 4 (M) x 2 (N),
// 64 x BN/2 per wave.
#include "common.h"

namespace {

typedef __attribute__((address_space(3))) void lds_void_t;

constexpr uint32_t BM = RMDA_GEMM2_BM;  // 256 rows per work item
constexpr uint32_t SLAB = 128;          // packed slab height (B rows)
constexpr uint32_t NT = 512;

// chunk swizzle of row r (BK/8 chunks per row): chunk c of row r sits in
// slot c ^ ((r >> 1) & (BK/8 - 1)).  Chosen by measurement on gfx950
// (SQ_LDS_BANK_CONFLICT over this kernel's exact fragment-read sequence):
// zero conflict cycles for BK 32 and 64, where the unswizzled layout loses
// 49% (BK 32) and 74% (BK 64) of LDS cycles to conflicts.  Depends only on
// r mod 16, so it is the same for a slab row and a tile row.
template <int BK>
__device__ __forceinline__ uint32_t swz(uint32_t r) {
    return (r >> 1) & (uint32_t)(BK / 8 - 1);
}

// B row of a group's weight matrix that slab row n of slab `slab` holds.
// SWIGLU slabs interleave 32 gate rows and the 32 matching up rows twice, so
// one wave's accumulators hold gate and up of the same output columns.
template <int MODE>
__device__ __forceinline__ uint32_t slab_row(uint32_t slab, uint32_t n, uint32_t inter) {
    if (MODE == RMDA_GEMM_SWIGLU) {
        const uint32_t bw = n / 64;
        const uint32_t within = n % 64;
        const uint32_t c = slab * 64 + bw * 32 + (within % 32);
        return within < 32 ? c : inter + c;
    }
    return slab * SLAB + n;
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// all LDS reads of this wave done, then the workgroup barrier
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// wait until this wave's loads of the oldest pending stage have landed;
// `after` = later stages already issued (0 .. STAGES-2)
template <int LOADS, int STAGES>
__device__ __forceinline__ void wait_stage(uint32_t after) {
    if constexpr (STAGES >= 4) {
        if (after >= 2) {
            wait_vm<2 * LOADS>();
            return;
        }
    }
    if constexpr (STAGES >= 3) {
        if (after >= 1) {
            wait_vm<LOADS>();
            return;
        }
    }
    wait_vm<0>();
}

template <int MODE, int BN, int BK, int STAGES, bool PACKED>
__global__ __launch_bounds__(512) void gemm2_kernel(rmda_gemm_args_t g) {
    constexpr uint32_t CH = BK / 8;              // 16-byte chunks per row
    constexpr uint32_t RPI = 64 / CH;            // rows per wave-wide DMA instruction
    constexpr uint32_t A_BYTES = BM * BK * 2;
    constexpr uint32_t B_BYTES = BN * BK * 2;
    constexpr uint32_t STAGE_BYTES = A_BYTES + B_BYTES;
    constexpr uint32_t A_INSTR = 32 / RPI;       // per live wave per stage (32 A rows)
    constexpr uint32_t B_INSTR = BN / RPI / 8;   // per wave per stage
    constexpr int LOADS_LIVE = (int)(A_INSTR + B_INSTR);
    constexpr int LOADS_IDLE = (int)B_INSTR;
    constexpr uint32_t WN = BN / 2;              // B rows per wave
    constexpr uint32_t NJ = WN / 16;             // 16-wide MFMA column blocks per wave
    __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE_BYTES];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % RMDA_WAVE;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid / RMDA_WAVE);
    // waves are placed on SIMD w % 4: pairing (wm, wn) as (w / 2, w % 2) puts
    // the two live waves of a 64-row block on different SIMDs and spreads the
    // live blocks of a short item over all four
    const uint32_t wm = w / 2;
    const uint32_t wn = w % 2;

    // ---- work assignment: balanced, XCD-contiguous over the real work ----
    const uint32_t n_slabs = g.n_w / SLAB;
    const uint32_t ntiles = n_slabs / (BN / SLAB);
    const uint32_t n_items = g.n_items != nullptr ? *g.n_items : g.max_items;
    const uint32_t total = n_items * ntiles;
    const uint32_t per = (total + 7) / 8;
    const uint32_t pos = blockIdx.x / 8;
    if (pos >= per) {
        return;
    }
    const uint32_t logical = (blockIdx.x % 8) * per + pos;
    if (logical >= total) {
        return;
    }
    const uint32_t item = logical / ntiles;
    const uint32_t nt = logical % ntiles;
    const uint4 it = reinterpret_cast<const uint4 *>(g.items)[item];
    const uint32_t grp = it.x;
    const uint32_t row0 = it.y;
    const uint32_t rows = it.z;
    const bool is_shared = grp == g.shared_group;
    const uint16_t *wg = is_shared ? g.w_shared : g.w + (size_t)grp * g.n_w * g.k;
    const uint32_t steps = g.k / BK;
    // a wave is live if some row of its 64-row block is (uniform per wave)
    const bool live = wm * 64 < rows;

    // ---- per-lane DMA sources ----
    const uint32_t lrow = lane / CH;   // row within one instruction's block
    const uint32_t lch = lane % CH;    // LDS chunk slot
    // A: wave (wm, wn) loads rows wm*64 + wn*32 + [0, 32); rows past the
    // item's end re-read row 0 of the item
    const uint16_t *a_src[A_INSTR];
    uint32_t a_dst[A_INSTR];
#pragma unroll
    for (uint32_t j = 0; j < A_INSTR; j += 1) {
        const uint32_t rbase = wm * 64 + wn * 32 + j * RPI;
        const uint32_t r = rbase + lrow;
        const uint32_t rr = r < rows ? r : 0u;
        uint32_t arow;
        if (MODE == RMDA_GEMM_SWIGLU) {
            arow = is_shared ? row0 + rr - g.shared_row0 : g.rowtok[row0 + rr];
        } else {
            arow = row0 + rr;
        }
        a_src[j] = g.a + (size_t)arow * g.lda + (lch ^ swz<BK>(r)) * 8;
        a_dst[j] = rbase * (BK * 2);
    }
    // B: wave w loads tile rows (w*B_INSTR + j)*RPI + [0, RPI)
    const uint16_t *b_src[B_INSTR];
#pragma unroll
    for (uint32_t j = 0; j < B_INSTR; j += 1) {
        const uint32_t nbase = (w * B_INSTR + j) * RPI;
        const uint32_t slab = nt * (BN / SLAB) + nbase / SLAB;
        const uint32_t nin = nbase % SLAB;
        if (PACKED) {
            b_src[j] = wg + (size_t)slab * steps * (SLAB * BK) + nin * BK + lane * 8;
        } else {
            const uint32_t n = nin + lrow;
            b_src[j] = wg + (size_t)slab_row<MODE>(slab, n, g.inter) * g.k + (lch ^ swz<BK>(n)) * 8;
        }
    }
    auto issue = [&](uint32_t s, uint32_t buf) {
        uint8_t *base = smem + buf * STAGE_BYTES;
        if (live) {
#pragma unroll
            for (uint32_t j = 0; j < A_INSTR; j += 1) {
                __builtin_amdgcn_global_load_lds((const void *)(a_src[j] + s * BK), (lds_void_t *)(base + a_dst[j]),
                                                 16, 0, 0);
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < B_INSTR; j += 1) {
            const uint16_t *src = PACKED ? b_src[j] + (size_t)s * (SLAB * BK) : b_src[j] + s * BK;
            __builtin_amdgcn_global_load_lds((const void *)src,
                                             (lds_void_t *)(base + A_BYTES + (w * B_INSTR + j) * 1024), 16, 0, 0);
        }
    };

    floatx4_t acc[4][NJ];
#pragma unroll
    for (int i = 0; i < 4; i += 1) {
#pragma unroll
        for (uint32_t j = 0; j < NJ; j += 1) {
            acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        }
    }

    // fragment addresses: lane reads row (block base + lane%16), chunk (kk*4 + lane/16)
    const uint32_t fr = lane % 16;
    const uint32_t fq = lane / 16;
    uint32_t a_off[4][BK / 32];
    uint32_t b_off[NJ][BK / 32];
#pragma unroll
    for (uint32_t kk = 0; kk < BK / 32; kk += 1) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i += 1) {
            const uint32_t ra = wm * 64 + i * 16 + fr;
            a_off[i][kk] = ra * (BK * 2) + (((kk * 4 + fq) ^ swz<BK>(ra)) * 16);
        }
#pragma unroll
        for (uint32_t j = 0; j < NJ; j += 1) {
            const uint32_t rb = wn * WN + j * 16 + fr;
            b_off[j][kk] = A_BYTES + rb * (BK * 2) + (((kk * 4 + fq) ^ swz<BK>(rb)) * 16);
        }
    }

#pragma unroll
    for (uint32_t s = 0; s < STAGES - 1; s += 1) {
        if (s < steps) {
            issue(s, s);
        }
    }
    for (uint32_t s = 0; s < steps; s += 1) {
        const uint32_t left = steps - 1 - s;
        const uint32_t after = left < STAGES - 2 ? left : STAGES - 2;
        if (live) {
            wait_stage<LOADS_LIVE, STAGES>(after);
        } else {
            wait_stage<LOADS_IDLE, STAGES>(after);
        }
        lds_barrier();
        if (s + STAGES - 1 < steps) {
            issue(s + STAGES - 1, (s + STAGES - 1) % STAGES);
        }
        if (live) {
            const uint8_t *base = smem + (s % STAGES) * STAGE_BYTES;
#pragma unroll
            for (uint32_t kk = 0; kk < BK / 32; kk += 1) {
                half8_t af[4];
                half8_t bf[NJ];
#pragma unroll
                for (int i = 0; i < 4; i += 1) {
                    af[i] = *reinterpret_cast<const half8_t *>(base + a_off[i][kk]);
                }
#pragma unroll
                for (uint32_t j = 0; j < NJ; j += 1) {
                    bf[j] = *reinterpret_cast<const half8_t *>(base + b_off[j][kk]);
                }
#pragma unroll
                for (int i = 0; i < 4; i += 1) {
#pragma unroll
                    for (uint32_t j = 0; j < NJ; j += 1) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
                    }
                }
            }
        }
    }
    if (!live) {
        return;
    }

    // epilogue: acc[i][j][v] is C[wm*64 + i*16 + 4*(lane/16) + v][B row wn*WN + j*16 + lane%16]
    const uint32_t rq = 4 * fq;
    uint16_t *O = reinterpret_cast<uint16_t *>(g.out);
    if (MODE == RMDA_GEMM_F16) {
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
#pragma unroll
            for (int v = 0; v < 4; v += 1) {
                const uint32_t rr = wm * 64 + i * 16 + rq + v;
                if (rr < rows) {
#pragma unroll
                    for (uint32_t j = 0; j < NJ; j += 1) {
                        const uint32_t col = nt * BN + wn * WN + j * 16 + fr;
                        O[(size_t)(row0 + rr) * g.ldo + col] = rmda_f2h(acc[i][j][v]);
                    }
                }
            }
        }
    } else {
        // within each 64-row group of B rows, blocks u (gate) and u + 2 (up)
        // hold the same output columns
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
#pragma unroll
            for (int v = 0; v < 4; v += 1) {
                const uint32_t rr = wm * 64 + i * 16 + rq + v;
                if (rr < rows) {
#pragma unroll
                    for (uint32_t gq = 0; gq < NJ / 4; gq += 1) {
#pragma unroll
                        for (uint32_t u = 0; u < 2; u += 1) {
                            const float gt = acc[i][gq * 4 + u][v];
                            const float up = acc[i][gq * 4 + u + 2][v];
                            const float h = gt / (1.0f + __expf(-gt)) * up;
                            const uint32_t bl = wn * WN + gq * 64 + u * 16;  // local B row of the block
                            const uint32_t slab = nt * (BN / SLAB) + bl / SLAB;
                            const uint32_t col = slab * 64 + ((bl % SLAB) / 64) * 32 + u * 16 + fr;
                            O[(size_t)(row0 + rr) * g.ldo + col] = rmda_f2h(h);
                        }
                    }
                }
            }
        }
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

template <int MODE, int BN, int BK, int STAGES>
hipError_t launch_cfg(hipStream_t s, const rmda_gemm_args_t *a, dim3 grid, bool packed) {
    if (packed) {
        hipLaunchKernelGGL((gemm2_kernel<MODE, BN, BK, STAGES, true>), grid, dim3(NT), 0, s, *a);
    } else {
        hipLaunchKernelGGL((gemm2_kernel<MODE, BN, BK, STAGES, false>), grid, dim3(NT), 0, s, *a);
    }
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_mode(hipStream_t s, const rmda_gemm_args_t *a, const rmda_gemm2_cfg_t &c, bool packed) {
    const uint32_t ntiles = a->n_w / SLAB / (c.bn / SLAB);
    uint64_t blocks = (uint64_t)a->max_items * ntiles;
    if (blocks == 0) {
        return hipSuccess;
    }
    blocks = (blocks + 7) / 8 * 8;
    if (blocks > 0x7fffffffull) {
        return hipErrorInvalidValue;
    }
    const dim3 grid((uint32_t)blocks);
    if (c.bn == 256) {
        if (c.bk == 64) {
            return launch_cfg<MODE, 256, 64, 2>(s, a, grid, packed);
        }
        if (c.stages == 4) {
            return launch_cfg<MODE, 256, 32, 4>(s, a, grid, packed);
        }
        return launch_cfg<MODE, 256, 32, 3>(s, a, grid, packed);
    }
    if (c.bk == 64) {
        if (c.stages == 2) {
            return launch_cfg<MODE, 128, 64, 2>(s, a, grid, packed);
        }
        return launch_cfg<MODE, 128, 64, 3>(s, a, grid, packed);
    }
    if (c.stages == 4) {
        return launch_cfg<MODE, 128, 32, 4>(s, a, grid, packed);
    }
    return launch_cfg<MODE, 128, 32, 3>(s, a, grid, packed);
}

}  // namespace

// Variant 0 is the default: the fastest configuration measured on MI355X at
// the benchmark shapes (BN 256, BK 64, two stages: 128 KiB of LDS).
rmda_gemm2_cfg_t rmda_gemm2_variant(int variant) {
    switch (variant) {
    case 1: return {128, 32, 3};
    case 2: return {128, 32, 4};
    case 3: return {256, 32, 3};
    case 4: return {256, 32, 4};
    case 6: return {128, 64, 2};
    case 7: return {128, 64, 3};
    default: return {256, 64, 2};
    }
}

hipError_t rmda_launch_gemm2(hipStream_t s, const rmda_gemm_args_t *a, rmda_gemm2_cfg_t c, int packed) {
    if (a->k % c.bk != 0 || a->n_w % SLAB != 0) {
        return hipErrorInvalidValue;
    }
    if ((a->n_w / SLAB) % (c.bn / SLAB) != 0) {
        c.bn = 128;  // odd slab count: fall back to one slab per tile
    }
    if (a->mode == RMDA_GEMM_SWIGLU) {
        return launch_mode<RMDA_GEMM_SWIGLU>(s, a, c, packed != 0);
    }
    return launch_mode<RMDA_GEMM_F16>(s, a, c, packed != 0);
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
