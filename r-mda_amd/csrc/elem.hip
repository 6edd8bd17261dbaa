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
        y[i] = rmda_swiglu(g, a[(size_t)r * pc.astride + pc.bo + c]);
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
        const float v = rmda_swiglu(g, a[(size_t)r * pc.astride + pc.bo + c]);
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

// 16-byte versions of elem_kernel, elem_absmax_kernel, absmax_kernel and
// cast_kernel, for rows of whole float4s (n, astride, ao, bo multiples of 4,
// buffers 16-byte aligned): the same expression per element, four elements
// per lane, a block per (column range, row stride) so no index needs a
// division.  The absmax kernels reduce per block and merge with one
// atomicMax per block (at most 1024 blocks; absmax4_kernel, which keeps four
// loads in flight per thread, at most 256).
__device__ __forceinline__ float silu_scaled1(float g, float scale) {
    const float v = g * scale;
    return v / (1.0f + expf(-v));
}

__device__ __forceinline__ void block_absmax(float m, uint32_t *amax, uint32_t slot) {
    __shared__ float red[256];
    const uint32_t tid = threadIdx.x;
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

__device__ __forceinline__ bool row_live(const rmda_rowmask_t &mk, uint32_t r) {
    const uint32_t e = mk.tiles[r / mk.tile];
    return e != RMDA_NONE && r - mk.off[e] < mk.count[e];
}

template <bool ABS, bool MASK>
__global__ __launch_bounds__(256) void elem4_kernel(rmda_pc_qwen_elem_t pc, const float *__restrict__ a,
                                                    float *__restrict__ y, uint32_t *__restrict__ amax,
                                                    uint32_t slot, rmda_rowmask_t mk) {
    const uint32_t n4 = pc.n / 4;
    float m = 0.0f;
    for (uint32_t r = blockIdx.y; r < pc.rows; r += gridDim.y) {
        if (MASK && !row_live(mk, r)) {
            continue;
        }
        const float4 *ga = reinterpret_cast<const float4 *>(a + (size_t)r * pc.astride + pc.ao);
        const float4 *ua = reinterpret_cast<const float4 *>(a + (size_t)r * pc.astride + pc.bo);
        float4 *yr = reinterpret_cast<float4 *>(y + (size_t)r * pc.n);
        for (uint32_t c = blockIdx.x * 256 + threadIdx.x; c < n4; c += gridDim.x * 256) {
            const float4 g = ga[c];
            float4 v;
            if (pc.op == 0) {
                const float4 u = ua[c];
                v = make_float4(rmda_swiglu(g.x, u.x), rmda_swiglu(g.y, u.y), rmda_swiglu(g.z, u.z),
                                rmda_swiglu(g.w, u.w));
            } else {
                v = make_float4(silu_scaled1(g.x, pc.scale), silu_scaled1(g.y, pc.scale),
                                silu_scaled1(g.z, pc.scale), silu_scaled1(g.w, pc.scale));
            }
            yr[c] = v;
            if (ABS) {
                m = fmaxf(m, fabsf(v.x));
                m = fmaxf(m, fabsf(v.y));
                m = fmaxf(m, fabsf(v.z));
                m = fmaxf(m, fabsf(v.w));
            }
        }
    }
    if (ABS) {
        block_absmax(m, amax, slot);
    }
}

// four loads in flight per thread; the maximum does not depend on the order
// the values are taken in.  At most 256 blocks: each block ends in one
// device atomicMax on the one slot word, and those serialise (1024 blocks:
// config 3's 16.8 MB took 15 us)
__global__ __launch_bounds__(256) void absmax4_kernel(const float4 *__restrict__ x, uint32_t n4,
                                                      uint32_t *__restrict__ amax, uint32_t slot) {
    constexpr uint32_t U = 4;
    const uint32_t st = gridDim.x * 256;
    float m = 0.0f;
    auto take = [&](const float4 &v) {
        m = fmaxf(m, fabsf(v.x));
        m = fmaxf(m, fabsf(v.y));
        m = fmaxf(m, fabsf(v.z));
        m = fmaxf(m, fabsf(v.w));
    };
    uint32_t i = blockIdx.x * 256 + threadIdx.x;
    for (; (uint64_t)i + (U - 1) * (uint64_t)st < n4; i += U * st) {
        float4 v[U];
#pragma unroll
        for (uint32_t u = 0; u < U; u += 1) {
            v[u] = x[i + u * st];
        }
#pragma unroll
        for (uint32_t u = 0; u < U; u += 1) {
            take(v[u]);
        }
    }
    for (; i < n4; i += st) {
        take(x[i]);
    }
    block_absmax(m, amax, slot);
}

template <bool MASK>
__global__ __launch_bounds__(256) void cast4r_kernel(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                     uint32_t rows, uint32_t n, const uint32_t *__restrict__ amax,
                                                     uint32_t slot, rmda_rowmask_t mk) {
    const uint32_t n4 = n / 4;
    const float sc = cast_scale(amax, slot);
    for (uint32_t r = blockIdx.y; r < rows; r += gridDim.y) {
        if (MASK && !row_live(mk, r)) {
            continue;
        }
        const float4 *sr = reinterpret_cast<const float4 *>(src + (size_t)r * n);
        uint2 *dr = reinterpret_cast<uint2 *>(dst + (size_t)r * n);
        for (uint32_t c = blockIdx.x * 256 + threadIdx.x; c < n4; c += gridDim.x * 256) {
            const float4 v = sr[c];
            dr[c] = make_uint2((uint32_t)rmda_f2h(v.x * sc) | ((uint32_t)rmda_f2h(v.y * sc) << 16),
                               (uint32_t)rmda_f2h(v.z * sc) | ((uint32_t)rmda_f2h(v.w * sc) << 16));
        }
    }
}

// The masked cast by tile: blocks (b, 0 .. gridDim.y - 1) take tile b of
// the mask's row tiles, read its expert's offset and count once, and cast
// the tile's live rows [max(lo, off), min(lo + tile, off + count))
// (row_live's rows) between them, with four loads in flight per thread.
// The row-strided cast4r_kernel<true> re-read the mask for every row, a
// chain of dependent loads per row.
__global__ __launch_bounds__(256) void cast4t_kernel(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                     uint32_t rows, uint32_t n, const uint32_t *__restrict__ amax,
                                                     uint32_t slot, rmda_rowmask_t mk) {
    const uint32_t e = mk.tiles[blockIdx.x];
    if (e == RMDA_NONE) {
        return;
    }
    const uint64_t lo = (uint64_t)blockIdx.x * mk.tile;
    const uint64_t off = mk.off[e];
    const uint64_t r0 = lo > off ? lo : off;
    uint64_t r1 = off + mk.count[e];
    r1 = r1 < lo + mk.tile ? r1 : lo + mk.tile;
    r1 = r1 < rows ? r1 : rows;
    if (r0 >= r1) {
        return;
    }
    const uint32_t n4 = n / 4;
    const uint32_t total = (uint32_t)(r1 - r0) * n4;  // float4s of the live rows, contiguous
    const float4 *sr = reinterpret_cast<const float4 *>(src + r0 * n);
    uint2 *dr = reinterpret_cast<uint2 *>(dst + r0 * n);
    const float sc = cast_scale(amax, slot);
    auto cvt = [&](const float4 &v) {
        return make_uint2((uint32_t)rmda_f2h(v.x * sc) | ((uint32_t)rmda_f2h(v.y * sc) << 16),
                          (uint32_t)rmda_f2h(v.z * sc) | ((uint32_t)rmda_f2h(v.w * sc) << 16));
    };
    constexpr uint32_t U = 4;
    const uint32_t st = gridDim.y * 256;
    uint32_t i = blockIdx.y * 256 + threadIdx.x;
    for (; i + (U - 1) * st < total; i += U * st) {
        float4 v[U];
#pragma unroll
        for (uint32_t u = 0; u < U; u += 1) {
            v[u] = sr[i + u * st];
        }
#pragma unroll
        for (uint32_t u = 0; u < U; u += 1) {
            dr[i + u * st] = cvt(v[u]);
        }
    }
    for (; i < total; i += st) {
        dr[i] = cvt(sr[i]);
    }
}

__global__ __launch_bounds__(256) void cast4_kernel(const float4 *__restrict__ src, uint2 *__restrict__ dst,
                                                    uint32_t n4, const uint32_t *__restrict__ amax, uint32_t slot) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) {
        return;
    }
    const float sc = cast_scale(amax, slot);
    const float4 v = src[i];
    dst[i] = make_uint2((uint32_t)rmda_f2h(v.x * sc) | ((uint32_t)rmda_f2h(v.y * sc) << 16),
                        (uint32_t)rmda_f2h(v.z * sc) | ((uint32_t)rmda_f2h(v.w * sc) << 16));
}

bool aligned16(const void *p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

bool elem_vec_ok(const rmda_pc_qwen_elem_t *pc, const float *a, const float *y) {
    return pc->n % 4 == 0 && pc->astride % 4 == 0 && pc->ao % 4 == 0 && (pc->op != 0 || pc->bo % 4 == 0) &&
           aligned16(a) && aligned16(y);
}

dim3 elem_grid(const rmda_pc_qwen_elem_t *pc) {
    const uint32_t gx = (pc->n / 4 + 255) / 256;
    uint32_t gy = 1024 / (gx > 1024 ? 1024 : gx);
    gy = gy > pc->rows ? pc->rows : gy;
    return dim3(gx > 1024 ? 1024 : gx, gy < 1 ? 1 : gy);
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
    if (elem_vec_ok(pc, a, y)) {
        hipLaunchKernelGGL((elem4_kernel<false, false>), elem_grid(pc), dim3(256), 0, s, *pc, a, y, nullptr, 0u,
                           rmda_rowmask_t{});
        return hipGetLastError();
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
    if (pc->op == 0 && elem_vec_ok(pc, a, y)) {
        hipLaunchKernelGGL((elem4_kernel<true, false>), elem_grid(pc), dim3(256), 0, s, *pc, a, y, amax, slot,
                           rmda_rowmask_t{});
        return hipGetLastError();
    }
    const uint64_t blocks = (n + 255) / 256 > 1024 ? 1024 : (n + 255) / 256;
    hipLaunchKernelGGL(elem_absmax_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, *pc, a, y, amax, slot);
    return hipGetLastError();
}

hipError_t rmda_launch_elem_absmax_rows(hipStream_t s, const rmda_pc_qwen_elem_t *pc, const float *a, float *y,
                                        uint32_t *amax, uint32_t slot, const rmda_rowmask_t *mask) {
    if (pc->rows == 0 || pc->n == 0) {
        return hipSuccess;
    }
    if (pc->op != 0 || !elem_vec_ok(pc, a, y) || mask == nullptr) {
        return rmda_launch_elem_absmax(s, pc, a, y, amax, slot);
    }
    hipLaunchKernelGGL((elem4_kernel<true, true>), elem_grid(pc), dim3(256), 0, s, *pc, a, y, amax, slot, *mask);
    return hipGetLastError();
}

hipError_t rmda_launch_cast_rows(hipStream_t s, uint32_t rows, uint32_t n, const float *src, uint16_t *dst,
                                 const uint32_t *amax, uint32_t slot, const rmda_rowmask_t *mask) {
    if (rows == 0 || n == 0) {
        return hipSuccess;
    }
    if (n % 4 != 0 || !aligned16(src) || (reinterpret_cast<uintptr_t>(dst) & 7u) != 0 || mask == nullptr) {
        const rmda_pc_cast_t pc{rows * n, slot};
        return rmda_launch_cast(s, &pc, src, dst, amax);
    }
    if (mask->tile > 0 && (uint64_t)rows * n < (1ull << 32)) {
        // blocks per row tile of the mask: about 16 float4 per thread when the tile is full
        const uint32_t nt = (rows + mask->tile - 1) / mask->tile;
        const uint32_t per = (mask->tile * (n / 4) + 4095) / 4096;
        hipLaunchKernelGGL(cast4t_kernel, dim3(nt, per > 16 ? 16 : per), dim3(256), 0, s, src, dst, rows, n, amax,
                           slot, *mask);
        return hipGetLastError();
    }
    rmda_pc_qwen_elem_t shape{};
    shape.rows = rows;
    shape.n = n;
    hipLaunchKernelGGL((cast4r_kernel<true>), elem_grid(&shape), dim3(256), 0, s, src, dst, rows, n, amax, slot, *mask);
    return hipGetLastError();
}

hipError_t rmda_launch_absmax(hipStream_t s, const rmda_pc_absmax_t *pc, const float *x, uint32_t *amax) {
    if (pc->n % 4 == 0 && pc->n > 0 && aligned16(x)) {
        uint32_t b4 = (pc->n / 4 + 255) / 256;
        b4 = b4 > 256 ? 256 : b4;
        hipLaunchKernelGGL(absmax4_kernel, dim3(b4), dim3(256), 0, s, reinterpret_cast<const float4 *>(x), pc->n / 4,
                           amax, pc->slot);
        return hipGetLastError();
    }
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
    if (pc->n % 4 == 0 && aligned16(src) && (reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
        hipLaunchKernelGGL(cast4_kernel, dim3((pc->n / 4 + 255) / 256), dim3(256), 0, s,
                           reinterpret_cast<const float4 *>(src), reinterpret_cast<uint2 *>(dst), pc->n / 4, amax,
                           pc->slot);
        return hipGetLastError();
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

// ---- the fused layer's fp32-activation (slot-scaled) mode ----

namespace {

// float bits of the largest fabsf over the values a thread saw, per block
__device__ __forceinline__ uint32_t block_max_bits(float m) {
    __shared__ float red[256];
    const uint32_t tid = threadIdx.x;
    red[tid] = m;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (tid < s) {
            red[tid] = fmaxf(red[tid], red[tid + s]);
        }
        __syncthreads();
    }
    return __builtin_bit_cast(uint32_t, red[0]);
}

// the cast_f16.comp scale of an absmax value (cast_scale without the slot)
__device__ __forceinline__ float amax_scale(uint32_t u) {
    const float a = __builtin_bit_cast(float, u);
    if (!(a > 0.0f) || __builtin_isinf(a)) {
        return 1.0f;
    }
    return ldexpf(1.0f, 141 - (int)((u >> 23) & 0xffu));
}

__device__ __forceinline__ uint2 cast4(const float4 &v, float sc) {
    return make_uint2((uint32_t)rmda_f2h(v.x * sc) | ((uint32_t)rmda_f2h(v.y * sc) << 16),
                      (uint32_t)rmda_f2h(v.z * sc) | ((uint32_t)rmda_f2h(v.w * sc) << 16));
}

// absmax.comp over x, one part per block (no slot word to clear first)
__global__ __launch_bounds__(256) void x_absmax_kernel(const float4 *__restrict__ x, size_t n4,
                                                       uint32_t *__restrict__ part) {
    // four loads in flight per thread (the maximum does not depend on the order)
    constexpr uint32_t U = 4;
    const size_t st = (size_t)gridDim.x * 256;
    float m = 0.0f;
    auto take = [&](const float4 &v) {
        m = fmaxf(m, fabsf(v.x));
        m = fmaxf(m, fabsf(v.y));
        m = fmaxf(m, fabsf(v.z));
        m = fmaxf(m, fabsf(v.w));
    };
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + (U - 1) * st < n4; i += U * st) {
        float4 v[U];
#pragma unroll
        for (uint32_t u = 0; u < U; u += 1) {
            v[u] = x[i + u * st];
        }
#pragma unroll
        for (uint32_t u = 0; u < U; u += 1) {
            take(v[u]);
        }
    }
    for (; i < n4; i += st) {
        take(x[i]);
    }
    const uint32_t r = block_max_bits(m);
    if (threadIdx.x == 0) {
        part[blockIdx.x] = r;
    }
}

// every block folds the parts (the values are non-negative, so their bit
// patterns order as the values do), then cast_f16.comp over its share
__global__ __launch_bounds__(256) void x_cast_kernel(const float4 *__restrict__ x, size_t n4,
                                                     const uint32_t *__restrict__ part, uint2 *__restrict__ x16,
                                                     uint32_t *__restrict__ x_slot, uint32_t *__restrict__ hp_parts) {
    __shared__ uint32_t s_amax;
    if (threadIdx.x < RMDA_WAVE) {
        uint32_t m = 0;
        for (uint32_t i = threadIdx.x; i < RMDA_XCAST_PARTS; i += RMDA_WAVE) {
            m = max(m, part[i]);
        }
        m = rmda_wave_red_u32<true>(m);
        if (threadIdx.x == 0) {
            s_amax = m;
        }
    }
    __syncthreads();
    const uint32_t amax = s_amax;
    if (blockIdx.x == 0) {
        if (threadIdx.x == 0) {
            *x_slot = amax;
        }
        if (threadIdx.x < RMDA_AMAX_PARTS) {
            hp_parts[threadIdx.x * RMDA_AMAX_STRIDE] = 0u;
        }
    }
    const float sc = amax_scale(amax);
    constexpr uint32_t U = 4;
    const size_t st = (size_t)gridDim.x * 256;
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + (U - 1) * st < n4; i += U * st) {
        float4 v[U];
#pragma unroll
        for (uint32_t u = 0; u < U; u += 1) {
            v[u] = x[i + u * st];
        }
#pragma unroll
        for (uint32_t u = 0; u < U; u += 1) {
            x16[i + u * st] = cast4(v[u], sc);
        }
    }
    for (; i < n4; i += st) {
        x16[i] = cast4(x[i], sc);
    }
}

// every block folds the GEMM's partial absmax words, block 0 stores the fold
// to the slot the down GEMM reads; the blocked hp: 16-row groups are
// contiguous runs of 16 * inter values
__global__ __launch_bounds__(256) void hp_cast_kernel(const float4 *__restrict__ hp32, uint2 *__restrict__ hp16,
                                                      const uint32_t *__restrict__ hp_parts,
                                                      uint32_t *__restrict__ slot, const uint32_t *__restrict__ off,
                                                      const uint32_t *__restrict__ count, uint32_t experts,
                                                      uint32_t inter, uint32_t sh_row0, uint32_t sh_rows) {
    static_assert(RMDA_AMAX_PARTS == RMDA_WAVE, "one partial word per lane");
    __shared__ uint32_t s_amax;
    if (threadIdx.x < RMDA_WAVE) {
        const uint32_t m = rmda_wave_red_u32<true>(hp_parts[threadIdx.x * RMDA_AMAX_STRIDE]);
        if (threadIdx.x == 0) {
            s_amax = m;
            if (blockIdx.x == 0) {
                *slot = m;
            }
        }
    }
    __syncthreads();
    const uint32_t routed_end = off[experts - 1] + (count[experts - 1] + 15u) / 16u * 16u;
    const size_t n_r = (size_t)routed_end * inter / 4;
    const size_t s0 = (size_t)sh_row0 * inter / 4;
    const size_t n_s = (size_t)((sh_rows + 15u) / 16u * 16u) * inter / 4;
    const float sc = amax_scale(s_amax);
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n_r + n_s; i += (size_t)gridDim.x * 256) {
        const size_t j = i < n_r ? i : s0 + (i - n_r);
        hp16[j] = cast4(hp32[j], sc);
    }
}

}  // namespace

hipError_t rmda_launch_x_absmax(hipStream_t s, const float *x, size_t n, uint32_t *part) {
    hipLaunchKernelGGL(x_absmax_kernel, dim3(RMDA_XCAST_PARTS), dim3(256), 0, s,
                       reinterpret_cast<const float4 *>(x), n / 4, part);
    return hipGetLastError();
}

hipError_t rmda_launch_x_cast(hipStream_t s, const float *x, size_t n, const uint32_t *part, uint16_t *x16,
                              uint32_t *x_slot, uint32_t *hp_parts) {
    hipLaunchKernelGGL(x_cast_kernel, dim3(RMDA_XCAST_PARTS), dim3(256), 0, s, reinterpret_cast<const float4 *>(x),
                       n / 4, part, reinterpret_cast<uint2 *>(x16), x_slot, hp_parts);
    return hipGetLastError();
}

hipError_t rmda_launch_hp_cast(hipStream_t s, const float *hp32, uint16_t *hp16, const uint32_t *hp_parts,
                               uint32_t *slot, const uint32_t *off, const uint32_t *count, uint32_t experts,
                               uint32_t inter, uint32_t sh_row0, uint32_t sh_rows) {
    hipLaunchKernelGGL(hp_cast_kernel, dim3(1024), dim3(256), 0, s, reinterpret_cast<const float4 *>(hp32),
                       reinterpret_cast<uint2 *>(hp16), hp_parts, slot, off, count, experts, inter, sh_row0,
                       sh_rows);
    return hipGetLastError();
}
