// Elementwise helpers of the MoE path and the synthetic-input generator.
//   elem_kernel    shader/qwen_elem.comp:20-31 (op 0 SwiGLU, op 1 silu(g*scale))
//   absmax_kernel  shader/absmax.comp:13-31 (grid-stride max |x|, LDS tree,
//                  atomicMax on the float bits; values are non-negative)
//   cast_kernel    shader/cast_f16.comp:20-35 (power-of-two slot scale, RNE)
//   bf16_kernel    shader/qwen_bf16.comp:9-15 (two bf16 -> two fp16 in place)
//   fill_kernel    counter hash -> standardised Irwin-Hall(4) -> fp16/fp32
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void elem_kernel(rmda_pc_qwen_elem_t pc, const float *__restrict__ a,
                                                   float *__restrict__ y) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)pc.rows * pc.n) {
        return;
    }
    const uint32_t r = (uint32_t)(i / pc.n);
    const uint32_t c = (uint32_t)(i % pc.n);
    const float g = a[(size_t)r * pc.astride + pc.ao + c];
    if (pc.op == 0) {
        y[i] = g / (1.0f + expf(-g)) * a[(size_t)r * pc.astride + pc.bo + c];
    } else {
        const float v = g * pc.scale;
        y[i] = v / (1.0f + expf(-v));
    }
}

// elem op 0 (SwiGLU) and the absmax of its output in one pass, for the
// qwen.c recording, where the absmax pass re-read all of y: y is the same
// expression per element as elem_kernel's, and amax[slot] the same fmaxf of
// fabsf (NaN skipped) as absmax_kernel's, reduced per block and merged by
// one atomicMax per block (a grid of at most 1024 blocks, as absmax's).
__global__ __launch_bounds__(256) void elem_absmax_kernel(rmda_pc_qwen_elem_t pc, const float *__restrict__ a,
                                                          float *__restrict__ y, uint32_t *__restrict__ amax,
                                                          uint32_t slot) {
    __shared__ float red[256];
    const uint32_t tid = threadIdx.x;
    const uint64_t n = (uint64_t)pc.rows * pc.n;
    float m = 0.0f;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + tid; i < n; i += (uint64_t)gridDim.x * 256) {
        const uint32_t r = (uint32_t)(i / pc.n);
        const uint32_t c = (uint32_t)(i % pc.n);
        const float g = a[(size_t)r * pc.astride + pc.ao + c];
        const float v = g / (1.0f + expf(-g)) * a[(size_t)r * pc.astride + pc.bo + c];
        y[i] = v;
        m = fmaxf(m, fabsf(v));
    }
    red[tid] = m;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (tid < s) {
            red[tid] = fmaxf(red[tid], red[tid + s]);
        }
        __syncthreads();
    }
    if (tid == 0) {
        atomicMax(&amax[slot], __builtin_bit_cast(uint32_t, red[0]));
    }
}

__global__ __launch_bounds__(256) void absmax_kernel(const float *__restrict__ x, uint32_t n,
                                                     uint32_t *__restrict__ amax, uint32_t slot) {
    __shared__ float red[256];
    const uint32_t tid = threadIdx.x;
    float m = 0.0f;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + tid; i < n; i += (uint64_t)gridDim.x * 256) {
        m = fmaxf(m, fabsf(x[i]));
    }
    red[tid] = m;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (tid < s) {
            red[tid] = fmaxf(red[tid], red[tid + s]);
        }
        __syncthreads();
    }
    if (tid == 0) {
        atomicMax(&amax[slot], __builtin_bit_cast(uint32_t, red[0]));
    }
}

__device__ __forceinline__ float cast_scale(const uint32_t *amax, uint32_t slot) {
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

__global__ __launch_bounds__(256) void cast_kernel(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                   uint32_t n, const uint32_t *__restrict__ amax,
                                                   uint32_t slot) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) {
        return;
    }
    dst[i] = rmda_f2h(src[i] * cast_scale(amax, slot));
}

__global__ __launch_bounds__(256) void bf16_kernel(uint32_t *__restrict__ w, uint32_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) {
        return;
    }
    const uint32_t u = w[i];
    const float lo = __builtin_bit_cast(float, u << 16);
    const float hi = __builtin_bit_cast(float, u & 0xffff0000u);
    w[i] = (uint32_t)rmda_f2h(lo) | ((uint32_t)rmda_f2h(hi) << 16);
}

__device__ __forceinline__ uint64_t mix64(uint64_t x) {
    const uint64_t a = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    const uint64_t b = (a ^ (a >> 27)) * 0x94d049bb133111ebull;
    return b ^ (b >> 31);
}

// Same definition as the host generator: SplitMix64 finaliser applied to
// (stream, key, index); four 16-bit uniforms summed exactly; minus 2, times
// sqrt(3) and std, each a single IEEE rounding.
__global__ __launch_bounds__(256) void fill_kernel(void *dst, uint64_t n, int f16, uint64_t stream,
                                                   uint64_t seed, float std) {
    const uint64_t k = mix64(mix64(stream + 0x9e3779b97f4a7c15ull) ^ seed);
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
        const uint64_t h = mix64(k ^ i);
        const int32_t s = 2 * (int32_t)(h & 0xffffu) + 2 * (int32_t)((h >> 16) & 0xffffu) +
                          2 * (int32_t)((h >> 32) & 0xffffu) + 2 * (int32_t)((h >> 48) & 0xffffu) + 4;
        const float z = (float)(s - 262144) * 7.62939453125e-06f;
        const float v = __fmul_rn(__fmul_rn(z, 1.7320508075688772f), std);
        if (f16) {
            reinterpret_cast<uint16_t *>(dst)[i] = rmda_f2h(v);
        } else {
            reinterpret_cast<float *>(dst)[i] = v;
        }
    }
}

}  // namespace

hipError_t rmda_launch_elem(hipStream_t s, const rmda_pc_qwen_elem_t *pc, const float *a, float *y) {
    const uint64_t n = (uint64_t)pc->rows * pc->n;
    if (n == 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(elem_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, *pc, a, y);
    return hipGetLastError();
}

hipError_t rmda_launch_elem_absmax(hipStream_t s, const rmda_pc_qwen_elem_t *pc, const float *a, float *y,
                                   uint32_t *amax, uint32_t slot) {
    const uint64_t n = (uint64_t)pc->rows * pc->n;
    if (n == 0) {
        return hipSuccess;
    }
    const uint64_t blocks = (n + 255) / 256 > 1024 ? 1024 : (n + 255) / 256;
    hipLaunchKernelGGL(elem_absmax_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, *pc, a, y, amax, slot);
    return hipGetLastError();
}

hipError_t rmda_launch_absmax(hipStream_t s, const rmda_pc_absmax_t *pc, const float *x, uint32_t *amax) {
    uint32_t blocks = (pc->n + 255) / 256;
    blocks = blocks < 1 ? 1 : (blocks > 1024 ? 1024 : blocks);
    hipLaunchKernelGGL(absmax_kernel, dim3(blocks), dim3(256), 0, s, x, pc->n, amax, pc->slot);
    return hipGetLastError();
}

hipError_t rmda_launch_cast(hipStream_t s, const rmda_pc_cast_t *pc, const float *src, uint16_t *dst,
                            const uint32_t *amax) {
    if (pc->n == 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(cast_kernel, dim3((pc->n + 255) / 256), dim3(256), 0, s, src, dst, pc->n, amax, pc->slot);
    return hipGetLastError();
}

hipError_t rmda_launch_bf16(hipStream_t s, uint32_t n, uint32_t *w) {
    if (n == 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(bf16_kernel, dim3((n + 255) / 256), dim3(256), 0, s, w, n);
    return hipGetLastError();
}

hipError_t rmda_launch_fill_normal(hipStream_t s, void *dst, size_t n, int f16, uint64_t stream,
                                   uint64_t seed, float std) {
    if (n == 0) {
        return hipSuccess;
    }
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 8192) {
        blocks = 8192;
    }
    hipLaunchKernelGGL(fill_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, dst, (uint64_t)n, f16, stream,
                       seed, std);
    return hipGetLastError();
}
