// Router projection: proj[r, c] = x16[r, :] . w[c, :] (+ bias[c]) in fp32.
//
// Replaces the dense fp16 GEMM that fills the reference's `p` buffer
// (src/qwen.c:845 -> :541-570, shader/matmul_f16(_wide).comp).  Routing must
// be bit-exact, so the logits follow one fixed order that the CPU oracle
// replays: d is cut into 8 contiguous chunks of L = d/8; chunk q's partial is
// a sequential fmaf chain over i = qL .. qL+L-1 starting from 0; the eight
// partials are added left to right, then the bias.  Vector fp32 FMA (MFMA's
// internal summation order is not reproducible on a CPU).
//
// Two kernels compute the same bits:
//
// router_sx_kernel (d % 128 == 0; the layer always uses it).  A workgroup
// owns 8 tokens x 64 columns; its 8 waves are the 8 d chunks.  Lane =
// column: each lane streams its own column's weights while the 8 tokens'
// fp16 activations are wave-uniform and arrive through scalar loads into
// SGPRs, so every FMA is one v_fma_mix_f32 (fp16 SGPR operand widened
// exactly, fp32 weight, fp32 accumulator, one rounding: the same value as
// fmaf on the widened operand) and no LDS traffic or barrier sits in the k
// loop.  With packed weights ([d/4][cols padded to 64][4], written once by
// router_pack_kernel) one wave's weight load is 1 KiB contiguous; with HF
// [cols][d] weights each lane reads its own row, which costs the L1 64
// cache-line lookups per wave load and makes that variant about 40% slower.
// Latency is hidden by 16 waves per CU rather than by in-wave prefetch:
// scalar loads return out of order, so the compiler can only wait for all
// of them, and a prefetched batch would be waited for with the current one.
// The 8 chunk partials meet in LDS once at the end.
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


constexpr int SX_BATCH = 8;  // k elements per scalar load (16 bytes per token)

typedef const __attribute__((address_space(4))) uint32_t *const_u32p;

__device__ __forceinline__ float h_lo(uint32_t v) { return rmda_h2f((uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float h_hi(uint32_t v) { return rmda_h2f((uint16_t)(v >> 16)); }

// W_PACKED: w is the packed router layout [d/4][cpad][4] (see
// router_pack_kernel), so lane c's four consecutive k values are 16 bytes
// and one wave's load is 1 KiB contiguous.  Otherwise w is HF [cols][d] and
// every lane reads its own row (64 cache lines per wave load).
//
// CG column groups of 64 per workgroup (blockDim = 512 * CG; wave q works on
// chunk q % 8 of column group q / 8).  FUSE (top-k fused in; CG * 64 >= cols,
// one column slice): the workgroup owns every logit of its RT tokens, keeps
// them in LDS, and its first RT waves route one token each, so the routing
// needs no second launch and no hand-off between workgroups (which on this
// multi-XCD part would need a device-scope fence, i.e. an L2 write-back).
template <int RT, bool W_PACKED, int CG, bool FUSE>
__global__ __launch_bounds__(512 * CG) void router_sx_kernel(const uint16_t *__restrict__ x16,
                                                             const float *__restrict__ w,
                                                             const float *__restrict__ bias,
                                                             float *__restrict__ proj, uint32_t rows,
                                                             uint32_t d, uint32_t cols, uint32_t cpad,
                                                             uint32_t stride, uint32_t nbias,
                                                             uint32_t *zero_words, uint32_t n_zero,
                                                             rmda_route_fuse_t fz) {
    constexpr uint32_t NT = 512 * CG;
    constexpr uint32_t NCOL = RMDA_WAVE * CG;
    __shared__ float red[NQ][RT][NCOL];
    __shared__ float lg[RT][NCOL];

    const uint32_t lane = threadIdx.x % RMDA_WAVE;
    const uint32_t wq = __builtin_amdgcn_readfirstlane(threadIdx.x / RMDA_WAVE);
    const uint32_t q = wq % NQ;   // d chunk
    const uint32_t cg = wq / NQ;  // column group within the workgroup
    if (zero_words != nullptr && blockIdx.x == 0 && blockIdx.y == 0) {
        for (uint32_t i = threadIdx.x; i < n_zero; i += NT) {
            zero_words[i] = 0;
        }
    }
    const uint32_t L = d / NQ;
    const uint32_t nb = L / SX_BATCH;  // even: d % 128 == 0 is a launch condition
    const uint32_t t0 = blockIdx.x * RT;
    const uint32_t c0 = blockIdx.y * NCOL;
    const uint32_t c = c0 + cg * RMDA_WAVE + lane;
    const bool cok = c < cols;
    const float4 *wp;
    size_t wstep;  // float4s between consecutive 4-element groups of k
    if (W_PACKED) {
        wp = reinterpret_cast<const float4 *>(w) + (size_t)(q * L / 4) * cpad + c;
        wstep = cpad;
    } else {
        wp = reinterpret_cast<const float4 *>(w + (size_t)(cok ? c : 0) * d + q * L);
        wstep = 1;
    }
    // token rows past `rows` re-read the last row and are never stored
    const_u32p xr[RT];
#pragma unroll
    for (int t = 0; t < RT; t += 1) {
        const uint32_t tok = t0 + t < rows ? t0 + t : rows - 1;
        xr[t] = (const_u32p)(x16 + (size_t)tok * d + q * L);
    }

    float acc[RT];
#pragma unroll
    for (int t = 0; t < RT; t += 1) {
        acc[t] = 0.0f;
    }
    // two K batches per iteration where the SGPR budget allows it (the fused
    // top-k tail's live values leave room for one)
    constexpr int UNROLL = FUSE ? 1 : 2;
#pragma unroll UNROLL
    for (uint32_t b = 0; b < nb; b += 1) {
        const float4 w0 = wp[(size_t)(2 * b) * wstep];
        const float4 w1 = wp[(size_t)(2 * b + 1) * wstep];
        const float wf[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int t = 0; t < RT; t += 1) {
            const const_u32p xp = xr[t] + b * 4;
            const uint32_t xw[4] = {xp[0], xp[1], xp[2], xp[3]};
#pragma unroll
            for (int j = 0; j < 4; j += 1) {
                acc[t] = __builtin_fmaf(h_lo(xw[j]), wf[2 * j], acc[t]);
                acc[t] = __builtin_fmaf(h_hi(xw[j]), wf[2 * j + 1], acc[t]);
            }
        }
    }

#pragma unroll
    for (int t = 0; t < RT; t += 1) {
        red[q][t][cg * RMDA_WAVE + lane] = acc[t];
    }
    __syncthreads();
    for (uint32_t o = threadIdx.x; o < RT * NCOL; o += NT) {
        const uint32_t t = o / NCOL;
        const uint32_t l = o % NCOL;
        const uint32_t cc = c0 + l;
        float v = red[0][t][l];
#pragma unroll
        for (int qq = 1; qq < NQ; qq += 1) {
            v = v + red[qq][t][l];
        }
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
    // fused top-k (fz.experts <= NCOL): wave t routes token t0 + t from LDS
    __syncthreads();
    const uint32_t t = t0 + wq;
    if (wq < (uint32_t)RT && t < rows) {
        uint32_t *ir = fz.idx + (size_t)t * fz.topk;
        float *wr = fz.wt + (size_t)t * fz.topk;
        rmda_route_row<CG, false>(&lg[wq][0], fz.experts, fz.topk, ir, wr, nullptr);
    }
}

// HF router weights [cols][d] -> packed [d/4][cpad][4], zero columns past
// `cols`.  One thread per packed float; a one-time load-time reorder.
__global__ __launch_bounds__(256) void router_pack_kernel(const float *__restrict__ w, float *__restrict__ out,
                                                          uint32_t cols, uint32_t cpad, uint32_t d) {
    const size_t n = (size_t)d * cpad;
    for (size_t o = (size_t)blockIdx.x * 256 + threadIdx.x; o < n; o += (size_t)gridDim.x * 256) {
        const uint32_t j = (uint32_t)(o % 4);
        const uint32_t c = (uint32_t)((o / 4) % cpad);
        const uint32_t i4 = (uint32_t)(o / (4 * (size_t)cpad));
        out[o] = c < cols ? w[(size_t)c * d + i4 * 4 + j] : 0.0f;
    }
}

}  // namespace

uint32_t rmda_router_cpad(uint32_t cols) { return (cols + RMDA_WAVE - 1) / RMDA_WAVE * RMDA_WAVE; }

namespace {

template <int CG, bool FUSE>
void launch_sx(hipStream_t s, dim3 grid, bool w_packed, const uint16_t *x16, const float *w, const float *bias,
               float *proj, uint32_t rows, uint32_t d, uint32_t cols, uint32_t cpad, uint32_t stride,
               uint32_t nbias, uint32_t *zero_words, uint32_t n_zero, const rmda_route_fuse_t &fz) {
    constexpr int RT = RMDA_ROUTE_GROUP;
    if (w_packed) {
        hipLaunchKernelGGL((router_sx_kernel<RT, true, CG, FUSE>), grid, dim3(512 * CG), 0, s, x16, w, bias, proj, rows,
                           d, cols, cpad, stride, nbias, zero_words, n_zero, fz);
    } else {
        hipLaunchKernelGGL((router_sx_kernel<RT, false, CG, FUSE>), grid, dim3(512 * CG), 0, s, x16, w, bias, proj, rows,
                           d, cols, cpad, stride, nbias, zero_words, n_zero, fz);
    }
}

}  // namespace

hipError_t rmda_launch_router(hipStream_t s, const uint16_t *x16, const float *w, int w_packed, const float *bias,
                              float *proj, uint32_t rows, uint32_t d, uint32_t cols, uint32_t stride,
                              uint32_t nbias, uint32_t *zero_words, uint32_t n_zero,
                              const rmda_route_fuse_t *fuse) {
    constexpr uint32_t RT = RMDA_ROUTE_GROUP;
    const bool sx = d % 128 == 0 && rows > 0;
    if ((w_packed || fuse != nullptr) && !sx) {
        return hipErrorInvalidValue;
    }
    if (fuse != nullptr && (fuse->experts > cols || cols > rmda_route_fuse_max_cols())) {
        return hipErrorInvalidValue;
    }
    if (sx) {
        const uint32_t cpad = rmda_router_cpad(cols);
        rmda_route_fuse_t fz{};
        if (fuse != nullptr) {
            fz = *fuse;
        }
        const uint32_t gx = (rows + RT - 1) / RT;
        if (fuse != nullptr && cols > RMDA_WAVE) {
            launch_sx<2, true>(s, dim3(gx, 1), w_packed, x16, w, bias, proj, rows, d, cols, cpad, stride, nbias,
                               zero_words, n_zero, fz);
        } else if (fuse != nullptr) {
            launch_sx<1, true>(s, dim3(gx, 1), w_packed, x16, w, bias, proj, rows, d, cols, cpad, stride, nbias,
                               zero_words, n_zero, fz);
        } else {
            launch_sx<1, false>(s, dim3(gx, (cols + RMDA_WAVE - 1) / RMDA_WAVE), w_packed, x16, w, bias, proj, rows,
                                d, cols, cpad, stride, nbias, zero_words, n_zero, fz);
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

uint32_t rmda_route_fuse_max_cols() { return 2 * RMDA_WAVE; }

hipError_t rmda_launch_router_pack(hipStream_t s, const float *w, float *out, uint32_t cols, uint32_t d) {
    const uint32_t cpad = rmda_router_cpad(cols);
    const size_t n = (size_t)d * cpad;
    const uint32_t blocks = (uint32_t)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    hipLaunchKernelGGL(router_pack_kernel, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, s, w, out, cols, cpad, d);
    return hipGetLastError();
}
