// Weighted gather-sum of expert outputs back to token order.
//
// combine_ref_kernel restates shader/moe_combine.comp:26-40 (fp32 expert
// rows `y`, shared-expert term, hyper-connection streams h += acc * 2 *
// sigmoid(inj / hc)), plus a plain fp16 output mode.  One thread per output
// element, like the reference.
//
// combine32_kernel is its bandwidth version for the drop-in entry points
// (d % 4 == 0; combine_ref_kernel remains for other d).
//
// combine16_kernel is the fused layer's version: fp16 expert rows, fp16
// output and/or the hyper-connection streams, one workgroup per token.  The token's topk (slot, weight) pairs are
// read once into LDS; each thread then handles 8 consecutive columns with
// 16-byte loads of every selected row, accumulating in fp32 in j order (the
// reference's order, :32-34) before the shared-expert term (:35).
#include "common.h"

namespace {

__device__ __forceinline__ float sigmoidf(float v) {
    return rmda_sigmoidf(v);
}

__global__ __launch_bounds__(256) void combine_ref_kernel(rmda_pc_moe_combine_t pc,
                                                          const float *__restrict__ wt,
                                                          const uint32_t *__restrict__ slot,
                                                          const float *__restrict__ y,
                                                          const float *__restrict__ proj,
                                                          const float *__restrict__ sh,
                                                          const float *__restrict__ inj,
                                                          float *__restrict__ h,
                                                          uint16_t *__restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)pc.rows * pc.d) {
        return;
    }
    const uint32_t r = (uint32_t)(i / pc.d);
    const uint32_t c = (uint32_t)(i % pc.d);
    float acc = 0.0f;
    for (uint32_t j = 0; j < pc.topk; j += 1) {
        const uint32_t s = slot[(size_t)r * pc.topk + j];
        if (s != RMDA_NONE) {
            acc += wt[(size_t)r * pc.topk + j] * y[(size_t)s * pc.d + c];
        }
    }
    if (sh != nullptr) {
        acc += sigmoidf(proj[(size_t)r * pc.pstride + pc.sg_off]) * sh[i];
    }
    if (out != nullptr) {
        out[i] = rmda_f2h(acc);
        return;
    }
    for (uint32_t s = 0; s < pc.hc; s += 1) {
        const float gte = sigmoidf(inj[(size_t)r * pc.inj_stride + pc.inj_off + s] / (float)pc.hc);
        h[(size_t)r * pc.hc * pc.d + (size_t)s * pc.d + c] += acc * 2.0f * gte;
    }
}

// The drop-in combine (rmda_moe_combine / _plain) at bandwidth: the same
// arithmetic as combine_ref_kernel per element (fp32 y rows, acc += wt*y in
// j order, then the shared term, then the hc streams or the fp16 output), but
// one workgroup per token: the token's slots, weights and stream gates are
// read once into LDS and each thread moves 4 consecutive columns with 16-byte
// loads and stores.  Needs d % 4 == 0.
template <bool HC>
__global__ __launch_bounds__(256) void combine32_kernel(rmda_pc_moe_combine_t pc,
                                                        const float *__restrict__ wt,
                                                        const uint32_t *__restrict__ slot,
                                                        const float *__restrict__ y,
                                                        const float *__restrict__ proj,
                                                        const float *__restrict__ sh,
                                                        const float *__restrict__ inj,
                                                        float *__restrict__ h,
                                                        uint16_t *__restrict__ out) {
    __shared__ uint32_t s_slot[RMDA_MAX_TOPK];
    __shared__ float s_wt[RMDA_MAX_TOPK];
    __shared__ float s_g[RMDA_MAX_HC];
    __shared__ float s_sg;
    const uint32_t r = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    if (tid < pc.topk) {
        s_slot[tid] = slot[(size_t)r * pc.topk + tid];
        s_wt[tid] = wt[(size_t)r * pc.topk + tid];
    }
    if (tid == 0 && sh != nullptr) {
        s_sg = sigmoidf(proj[(size_t)r * pc.pstride + pc.sg_off]);
    }
    if (HC && tid < pc.hc) {
        s_g[tid] = sigmoidf(inj[(size_t)r * pc.inj_stride + pc.inj_off + tid] / (float)pc.hc);
    }
    __syncthreads();
    const uint32_t d4 = pc.d / 4;
    for (uint32_t c = tid; c < d4; c += 256) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (uint32_t j = 0; j < pc.topk; j += 1) {
            const uint32_t s = s_slot[j];
            if (s == RMDA_NONE) {
                continue;
            }
            const float wj = s_wt[j];
            const float4 v = reinterpret_cast<const float4 *>(y + (size_t)s * pc.d)[c];
            acc.x += wj * v.x;
            acc.y += wj * v.y;
            acc.z += wj * v.z;
            acc.w += wj * v.w;
        }
        if (sh != nullptr) {
            const float4 v = reinterpret_cast<const float4 *>(sh + (size_t)r * pc.d)[c];
            acc.x += s_sg * v.x;
            acc.y += s_sg * v.y;
            acc.z += s_sg * v.z;
            acc.w += s_sg * v.w;
        }
        if (out != nullptr) {
            uint2 o;
            o.x = (uint32_t)rmda_f2h(acc.x) | ((uint32_t)rmda_f2h(acc.y) << 16);
            o.y = (uint32_t)rmda_f2h(acc.z) | ((uint32_t)rmda_f2h(acc.w) << 16);
            reinterpret_cast<uint2 *>(out + (size_t)r * pc.d)[c] = o;
        }
        if (HC) {
            for (uint32_t st = 0; st < pc.hc; st += 1) {
                float4 *hp = reinterpret_cast<float4 *>(h + ((size_t)r * pc.hc + st) * pc.d) + c;
                const float g = s_g[st];
                float4 a = *hp;
                a.x += acc.x * 2.0f * g;
                a.y += acc.y * 2.0f * g;
                a.z += acc.z * 2.0f * g;
                a.w += acc.w * 2.0f * g;
                *hp = a;
            }
        }
    }
}

// One 16-byte slice of an expert row, read past the caches' normal retention:
// every expert row is read by exactly one token's workgroup, once.
typedef unsigned int rmda_u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 rmda_stream_load16(const uint4 *p) {
    const rmda_u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const rmda_u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// HC: the hyper-connection epilogue of shader/moe_combine.comp:36-38 in place
// of (or besides) the fp16 output: h[r][s][c] += acc * 2 * sigmoid(inj / hc).
template <bool HC>
__global__ __launch_bounds__(256) void combine16_kernel(const float *__restrict__ wt,
                                                        const uint32_t *__restrict__ slot,
                                                        const uint16_t *__restrict__ y,
                                                        const float *__restrict__ proj,
                                                        uint32_t pstride, uint32_t sg_off,
                                                        uint32_t shared_row0, int has_shared,
                                                        uint16_t *__restrict__ out, uint32_t d,
                                                        uint32_t topk, rmda_hc_t hcp,
                                                        const uint32_t *__restrict__ run_if,
                                                        const uint32_t *__restrict__ yscale,
                                                        const uint32_t *__restrict__ ybound) {
    if (run_if != nullptr && *run_if == 0) {
        return;  // the down GEMM folded the combine in
    }
    // the slot-scaled mode's rows stand for y * f, f a power of two: taken
    // into the weights, which gives the same products bit for bit
    const float f = ybound != nullptr ? rmda_slot_inv(yscale) / rmda_ye_mul(ybound) : 1.0f;
    __shared__ uint32_t s_slot[RMDA_MAX_TOPK + 1];
    __shared__ float s_wt[RMDA_MAX_TOPK + 1];
    __shared__ float s_g[RMDA_MAX_HC];
    const uint32_t r = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    if (tid < topk) {
        s_slot[tid] = slot[(size_t)r * topk + tid];
        s_wt[tid] = wt[(size_t)r * topk + tid] * f;
    }
    if (tid == 0 && has_shared) {
        s_slot[RMDA_MAX_TOPK] = shared_row0 + r;
        s_wt[RMDA_MAX_TOPK] = sigmoidf(proj[(size_t)r * pstride + sg_off]) * f;
    }
    if (HC && tid < hcp.hc) {
        s_g[tid] = 2.0f * sigmoidf(hcp.inj[(size_t)r * hcp.inj_stride + hcp.inj_off + tid] / (float)hcp.hc);
    }
    __syncthreads();
    const uint32_t d8 = d / 8;
    for (uint32_t c = tid; c < d8; c += 256) {
        float acc[8];
#pragma unroll
        for (int v = 0; v < 8; v += 1) {
            acc[v] = 0.0f;
        }
        for (uint32_t j = 0; j < topk; j += 1) {
            const uint32_t s = s_slot[j];
            if (s == RMDA_NONE) {
                continue;
            }
            rmda_comb_acc8(acc, s_wt[j], rmda_stream_load16(reinterpret_cast<const uint4 *>(y + (size_t)s * d) + c));
        }
        if (has_shared) {
            rmda_comb_acc8(acc, s_wt[RMDA_MAX_TOPK],
                           rmda_stream_load16(reinterpret_cast<const uint4 *>(y + (size_t)s_slot[RMDA_MAX_TOPK] * d) + c));
        }
        if (out != nullptr) {
            reinterpret_cast<uint4 *>(out + (size_t)r * d)[c] = rmda_pack8_f16(acc);
        }
        if (HC) {
            for (uint32_t st = 0; st < hcp.hc; st += 1) {
                rmda_hc_acc8(hcp.h + ((size_t)r * hcp.hc + st) * d + (size_t)c * 8, acc, s_g[st]);
            }
        }
    }
}

}  // namespace

hipError_t rmda_launch_combine(hipStream_t s, const rmda_pc_moe_combine_t *pc, const float *wt,
                               const uint32_t *slot, const float *y, const float *proj,
                               const float *sh, const float *inj, float *h, uint16_t *out) {
    const uint64_t n = (uint64_t)pc->rows * pc->d;
    if (n == 0) {
        return hipSuccess;
    }
    // the vector kernel reads y, sh and h as float4 and writes out as 8-byte
    // words; other alignments take the per-element kernel
    const auto al = [](const void *q, uintptr_t a) { return (reinterpret_cast<uintptr_t>(q) & (a - 1)) == 0; };
    const bool vec_ok = al(y, 16) && al(sh, 16) && al(h, 16) && al(out, 8);
    if (pc->d % 4 == 0 && pc->topk <= RMDA_MAX_TOPK && pc->hc <= RMDA_MAX_HC && vec_ok) {
        // the streams when h is given, the fp16 output when out is (both
        // for the fused layer's slot-scaled mode)
        if (h == nullptr || pc->hc == 0) {
            hipLaunchKernelGGL(combine32_kernel<false>, dim3(pc->rows), dim3(256), 0, s, *pc, wt, slot, y, proj, sh,
                               inj, nullptr, out);
        } else {
            hipLaunchKernelGGL(combine32_kernel<true>, dim3(pc->rows), dim3(256), 0, s, *pc, wt, slot, y, proj, sh,
                               inj, h, out);
        }
        return hipGetLastError();
    }
    hipLaunchKernelGGL(combine_ref_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, *pc, wt, slot,
                       y, proj, sh, inj, h, out);
    return hipGetLastError();
}

hipError_t rmda_launch_combine16(hipStream_t s, const float *wt, const uint32_t *slot,
                                 const uint16_t *y, const float *proj, uint32_t pstride,
                                 uint32_t sg_off, uint32_t shared_row0, int has_shared,
                                 uint16_t *out, uint32_t rows, uint32_t d, uint32_t topk,
                                 const rmda_hc_t *hc, const uint32_t *run_if, const uint32_t *yscale,
                                 const uint32_t *ybound) {
    if (rows == 0) {
        return hipSuccess;
    }
    if (hc != nullptr && hc->h != nullptr) {
        hipLaunchKernelGGL(combine16_kernel<true>, dim3(rows), dim3(256), 0, s, wt, slot, y, proj, pstride, sg_off,
                           shared_row0, has_shared, out, d, topk, *hc, run_if, yscale, ybound);
    } else {
        hipLaunchKernelGGL(combine16_kernel<false>, dim3(rows), dim3(256), 0, s, wt, slot, y, proj, pstride,
                           sg_off, shared_row0, has_shared, out, d, topk, rmda_hc_t{}, run_if, yscale, ybound);
    }
    return hipGetLastError();
}
