// Grouped expert GEMM on gfx950 fp16 MFMA (v_mfma_f32_16x16x32_f16), fp32
// accumulate.  One kernel body serves three epilogues:
//   SWIGLU  gate_up of the fused layer: A rows gathered from the token matrix
//           through rowtok (no permuted copy of x is materialised); the tile's
//           B rows pair gate column c with up column inter + c so one thread
//           holds both and writes hp16 = fp16(silu(g) * u) directly
//           (fuses shader/qwen_elem.comp op 0 and the cast);
//   F16     down of the fused layer: A = hp16 rows, fp16 output rows;
//   F32     the reference's matmul_f16_moe (shader/matmul_f16_moe.comp:70-126):
//           128-row tiles mapped to experts by `tiles`, fp32 C scaled by
//           1/(scale(sa)*scale(sb)).
//
// Tile 128 x 128 x 32, 256 threads = 2 x 2 waves of 64 x 64 (4 x 4 MFMA
// tiles of 16 x 16 each, 64 fp32 accumulators per lane).  A and B stage
// through LDS (row pitch 40 halves: conflict-free 16-byte fragment reads),
// double-buffered with a register prefetch of the next K step.
// Work comes from a device-built list (expert, first row, rows); the grid is
// sized for the worst case and idle workgroups exit, so nothing waits on the
// host.  Workgroups are renumbered so consecutive logical tiles (the N tiles
// of one row block, which share A rows) land on the same XCD.
#include "common.h"

namespace {

constexpr uint32_t BM = RMDA_GEMM_BM;
constexpr uint32_t BN = 128;
constexpr uint32_t BK = 32;
constexpr uint32_t PITCH = BK + 8;  // halves
constexpr uint32_t NT = 256;

__device__ __forceinline__ float slot_scale(const uint32_t *amax, uint32_t slot) {
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

template <int MODE>
__global__ __launch_bounds__(256) void gemm_kernel(rmda_gemm_args_t g) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * PITCH];
    __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * PITCH];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % RMDA_WAVE;
    const uint32_t w = tid / RMDA_WAVE;
    const uint32_t wm = w % 2;
    const uint32_t wn = w / 2;

    // XCD-aware renumbering: hardware hands block b to XCD b % 8
    const uint32_t G = gridDim.x;
    const uint32_t per = G / 8;
    const uint32_t logical = (blockIdx.x % 8) * per + blockIdx.x / 8;
    const uint32_t ntiles = (MODE == RMDA_GEMM_SWIGLU) ? g.n_out / 64 : g.n_out / BN;
    const uint32_t item = logical / ntiles;
    const uint32_t nt = logical % ntiles;

    uint32_t grp;
    uint32_t row0;
    uint32_t rows;
    if (MODE == RMDA_GEMM_F32) {
        if (item >= g.max_items) {
            return;
        }
        grp = g.tiles[item];
        if (grp == RMDA_NONE) {
            return;
        }
        row0 = item * BM;
        rows = BM;
    } else {
        const uint32_t n_items = g.n_items != nullptr ? *g.n_items : g.max_items;
        if (item >= n_items) {
            return;
        }
        const uint4 it = reinterpret_cast<const uint4 *>(g.items)[item];
        grp = it.x;
        row0 = it.y;
        rows = it.z;
    }
    const bool is_shared = grp == g.shared_group;
    const uint16_t *wg = is_shared ? g.w_shared : g.w + (size_t)grp * g.n_w * g.k;

    // loader: two 16-byte chunks of A and of B per thread per K step; chunk c
    // covers row (tid + 256c)/4, k offset 8*((tid + 256c)%4)
    const uint32_t lr0 = tid / 4;
    const uint32_t lr1 = lr0 + 64;
    const uint32_t lkc = (tid % 4) * 8;
    auto a_row = [&](uint32_t r) -> uint32_t {
        if (r >= rows) {
            return 0;
        }
        if (MODE == RMDA_GEMM_SWIGLU) {
            const uint32_t sr = row0 + r;
            return is_shared ? sr - g.shared_row0 : g.rowtok[sr];
        }
        return row0 + r;
    };
    auto b_row = [&](uint32_t r) -> uint32_t {
        if (MODE == RMDA_GEMM_SWIGLU) {
            const uint32_t bw = r / 64;
            const uint32_t within = r % 64;
            return within < 32 ? nt * 64 + bw * 32 + within : g.inter + nt * 64 + bw * 32 + (within - 32);
        }
        return nt * BN + r;
    };
    const bool aok0 = lr0 < rows;
    const bool aok1 = lr1 < rows;
    const uint16_t *ap0 = g.a + (size_t)a_row(lr0) * g.lda + lkc;
    const uint16_t *ap1 = g.a + (size_t)a_row(lr1) * g.lda + lkc;
    const uint16_t *bp0 = wg + (size_t)b_row(lr0) * g.k + lkc;
    const uint16_t *bp1 = wg + (size_t)b_row(lr1) * g.k + lkc;
    const uint32_t ls0 = lr0 * PITCH + lkc;
    const uint32_t ls1 = lr1 * PITCH + lkc;

    // Rows past the item's end load row 0 of A (always valid memory) and are
    // zeroed after the load, so every load is an unconditional global load.
    uint4 ra0, ra1, rb0, rb1;
#define GLOAD(k0)                                                                   \
    do {                                                                            \
        ra0 = *reinterpret_cast<const uint4 *>(ap0 + (k0));                        \
        ra1 = *reinterpret_cast<const uint4 *>(ap1 + (k0));                        \
        rb0 = *reinterpret_cast<const uint4 *>(bp0 + (k0));                        \
        rb1 = *reinterpret_cast<const uint4 *>(bp1 + (k0));                        \
        if (!aok0) {                                                                \
            ra0 = make_uint4(0, 0, 0, 0);                                           \
        }                                                                           \
        if (!aok1) {                                                                \
            ra1 = make_uint4(0, 0, 0, 0);                                           \
        }                                                                           \
    } while (0)
#define LSTORE(buf)                                                                 \
    do {                                                                            \
        *reinterpret_cast<uint4 *>(&sA[(buf)][ls0]) = ra0;                          \
        *reinterpret_cast<uint4 *>(&sA[(buf)][ls1]) = ra1;                          \
        *reinterpret_cast<uint4 *>(&sB[(buf)][ls0]) = rb0;                          \
        *reinterpret_cast<uint4 *>(&sB[(buf)][ls1]) = rb1;                          \
    } while (0)

    floatx4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i += 1) {
#pragma unroll
        for (int j = 0; j < 4; j += 1) {
            acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        }
    }

    const uint32_t steps = g.k / BK;
    const uint32_t fr = lane % 16;        // fragment row (A) / column (B)
    const uint32_t fk = (lane / 16) * 8;  // fragment k offset
    GLOAD(0);
    LSTORE(0);
    __syncthreads();
    for (uint32_t s = 0; s < steps; s += 1) {
        const int buf = s & 1;
        if (s + 1 < steps) {
            GLOAD((s + 1) * BK);
        }
        half8_t af[4];
        half8_t bf[4];
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
            af[i] = *reinterpret_cast<const half8_t *>(&sA[buf][(wm * 64 + i * 16 + fr) * PITCH + fk]);
            bf[i] = *reinterpret_cast<const half8_t *>(&sB[buf][(wn * 64 + i * 16 + fr) * PITCH + fk]);
        }
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
#pragma unroll
            for (int j = 0; j < 4; j += 1) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        }
        if (s + 1 < steps) {
            LSTORE(buf ^ 1);
        }
        __syncthreads();
    }

#undef GLOAD
#undef LSTORE
    // epilogue: acc[i][j][v] is C[wm*64 + i*16 + 4*(lane/16) + v][wn*64 + j*16 + lane%16]
    const uint32_t rq = 4 * (lane / 16);
    if (MODE == RMDA_GEMM_F32) {
        const float sc = 1.0f / (slot_scale(g.amax, g.sa) * slot_scale(g.amax, g.sb));
        float *C = reinterpret_cast<float *>(g.out);
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
#pragma unroll
            for (int j = 0; j < 4; j += 1) {
#pragma unroll
                for (int v = 0; v < 4; v += 1) {
                    const uint32_t r = row0 + wm * 64 + i * 16 + rq + v;
                    const uint32_t col = nt * BN + wn * 64 + j * 16 + fr;
                    C[(size_t)r * g.ldo + col] = acc[i][j][v] * sc;
                }
            }
        }
    } else if (MODE == RMDA_GEMM_F16) {
        uint16_t *O = reinterpret_cast<uint16_t *>(g.out);
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
#pragma unroll
            for (int v = 0; v < 4; v += 1) {
                const uint32_t rr = wm * 64 + i * 16 + rq + v;
                if (rr < rows) {
#pragma unroll
                    for (int j = 0; j < 4; j += 1) {
                        const uint32_t col = nt * BN + wn * 64 + j * 16 + fr;
                        O[(size_t)(row0 + rr) * g.ldo + col] = rmda_f2h(acc[i][j][v]);
                    }
                }
            }
        }
    } else {
        uint16_t *O = reinterpret_cast<uint16_t *>(g.out);
#pragma unroll
        for (int i = 0; i < 4; i += 1) {
#pragma unroll
            for (int v = 0; v < 4; v += 1) {
                const uint32_t rr = wm * 64 + i * 16 + rq + v;
                if (rr < rows) {
#pragma unroll
                    for (int j = 0; j < 2; j += 1) {
                        const float gt = acc[i][j][v];
                        const float up = acc[i][j + 2][v];
                        const float h = gt / (1.0f + __expf(-gt)) * up;
                        const uint32_t col = nt * 64 + wn * 32 + j * 16 + fr;
                        O[(size_t)(row0 + rr) * g.ldo + col] = rmda_f2h(h);
                    }
                }
            }
        }
    }
}

}  // namespace

hipError_t rmda_launch_gemm(hipStream_t s, const rmda_gemm_args_t *a) {
    const uint32_t ntiles = (a->mode == RMDA_GEMM_SWIGLU) ? a->n_out / 64 : a->n_out / BN;
    uint64_t blocks = (uint64_t)a->max_items * ntiles;
    if (blocks == 0) {
        return hipSuccess;
    }
    blocks = (blocks + 7) / 8 * 8;
    if (blocks > 0x7fffffffull) {
        return hipErrorInvalidValue;
    }
    const dim3 grid((uint32_t)blocks);
    switch (a->mode) {
    case RMDA_GEMM_SWIGLU:
        hipLaunchKernelGGL(gemm_kernel<RMDA_GEMM_SWIGLU>, grid, dim3(NT), 0, s, *a);
        break;
    case RMDA_GEMM_F16:
        hipLaunchKernelGGL(gemm_kernel<RMDA_GEMM_F16>, grid, dim3(NT), 0, s, *a);
        break;
    default:
        hipLaunchKernelGGL(gemm_kernel<RMDA_GEMM_F32>, grid, dim3(NT), 0, s, *a);
        break;
    }
    return hipGetLastError();
}
