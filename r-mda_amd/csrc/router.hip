// Router projection: proj[r, c] = x16[r, :] . w[c, :] (+ bias[c]) in fp32.
//
// Replaces the dense fp16 GEMM that fills the reference's `p` buffer
// (src/qwen.c:845 -> :541-570, shader/matmul_f16(_wide).comp).  Routing must
// be bit-exact, so the logits follow one fixed order that the CPU oracle
// replays: d is cut into 8 contiguous chunks of L = d/8; chunk q's partial is
// a sequential fmaf chain over i = qL .. qL+L-1 starting from 0; the eight
// partials are added left to right, then the bias.
//
// Work split: a workgroup owns a 16-token x 32-column output tile (512
// workgroups at T=2048, E=128: two or three resident per CU, so global-load
// latency hides behind other workgroups' FMAs).  Its 256 threads are 8 chunk
// groups x 32 threads; each thread keeps 4 tokens x 4 columns of one chunk's
// partials in registers (16 independent fmaf chains) and walks its chunk in
// steps of 16 through LDS, double-buffered; within a wave the x reads are
// 8-way broadcasts.  The eight partials then meet in LDS and are summed in
// chunk order.  Vector fp32 FMA (MFMA's internal summation order is not
// reproducible on a CPU).
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

__global__ __launch_bounds__(256) void router_kernel(const uint16_t *__restrict__ x16,
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

}  // namespace

hipError_t rmda_launch_router(hipStream_t s, const uint16_t *x16, const float *w, const float *bias,
                              float *proj, uint32_t rows, uint32_t d, uint32_t cols, uint32_t stride,
                              uint32_t nbias, uint32_t *zero_words, uint32_t n_zero) {
    dim3 grid((rows + TM - 1) / TM, (cols + TC - 1) / TC);
    if (rows == 0) {
        grid.x = 1;  // still run block (0,0) for the zero fill
    }
    hipLaunchKernelGGL(router_kernel, grid, dim3(256), 0, s, x16, w, bias, proj, rows, d, cols, stride,
                       nbias, zero_words, n_zero);
    return hipGetLastError();
}
