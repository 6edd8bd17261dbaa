// Top-k gating: the wave64 redesign of shader/moe_route.comp.
//
// Reference semantics (shader/moe_route.comp:20-61): per row, topk rounds;
// each round takes the largest untaken logit by strict '>' from -3.0e38, so
// the lowest expert index wins ties and NaN / values <= -3e38 are never
// taken; idx is emitted in selection (descending) order; lane 0 sums
// z = sum_k exp(l_k - l_0) in selection order and writes wt_k = exp(l_k-l_0)/z;
// count[e] += 1 per selection.
//
// Here one wave owns one row.  Lane l holds columns l, l+64, ... (coalesced;
// up to 8 per lane for 512 experts) instead of the reference's 16 contiguous
// columns on 32 lanes.  A round is one lane-local scan plus one wave-wide
// max over a 64-bit key (order-preserving float bits << 32 | ~column), which
// yields the largest value and, among equal values, the lowest column in a
// single reduction.  Only columns < experts are read (the reference reads
// 512 columns regardless).
#include "common.h"

namespace {

constexpr int MAXV = RMDA_MAX_EXPERTS / RMDA_WAVE;  // values per lane

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        uint32_t lo = __shfl_xor((uint32_t)v, m);
        uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m);
        uint64_t o = ((uint64_t)hi << 32) | lo;
        v = o > v ? o : v;
    }
    return v;
}

template <int NV>
__global__ __launch_bounds__(256) void route_kernel(const float *__restrict__ proj,
                                                    uint32_t *__restrict__ idx,
                                                    float *__restrict__ wt,
                                                    uint32_t *__restrict__ count, uint32_t rows,
                                                    uint32_t experts, uint32_t topk,
                                                    uint32_t stride) {
    const uint32_t lane = threadIdx.x % RMDA_WAVE;
    const uint32_t r = blockIdx.x * 4 + threadIdx.x / RMDA_WAVE;
    if (r >= rows) {
        return;
    }
    const float *l = proj + (size_t)r * stride;
    float v[NV];
#pragma unroll
    for (int j = 0; j < NV; j += 1) {
        const uint32_t c = lane + RMDA_WAVE * j;
        v[j] = c < experts ? l[c] : -3.0e38f;  // -3e38 is never selectable
    }
    uint32_t taken = 0;
    // z and the per-lane output are built round by round (lane k keeps round
    // k's selection), so no per-round arrays are needed; z still accumulates
    // in selection order like the reference (:52-55).
    float sv0 = 0.0f;
    float z = 0.0f;
    uint32_t my_sel = RMDA_NONE;
    float my_val = 0.0f;
    for (uint32_t k = 0; k < topk; k += 1) {
        float lb = -3.0e38f;
        int lv = -1;
#pragma unroll
        for (int j = 0; j < NV; j += 1) {
            if (((taken >> j) & 1u) == 0 && v[j] > lb) {
                lb = v[j];
                lv = j;
            }
        }
        uint64_t key = 0;
        if (lv >= 0) {
            key = ((uint64_t)rmda_float_key(lb) << 32) | (uint32_t)(~(lane + RMDA_WAVE * (uint32_t)lv));
        }
        key = wave_max_u64(key);
        uint32_t col = RMDA_NONE;
        float val = -3.0e38f;
        if (key != 0) {
            col = ~(uint32_t)key;
            val = rmda_key_float((uint32_t)(key >> 32));
            if (col % RMDA_WAVE == lane) {
                taken |= 1u << (col / RMDA_WAVE);
            }
        }
        if (k == 0) {
            sv0 = val;
        }
        z = z + expf(val - sv0);
        if (lane == k) {
            my_sel = col;
            my_val = val;
        }
    }
    if (lane < topk) {
        idx[(size_t)r * topk + lane] = my_sel;
        wt[(size_t)r * topk + lane] = expf(my_val - sv0) / z;
        if (count != nullptr && my_sel != RMDA_NONE) {
            atomicAdd(&count[my_sel], 1u);
        }
    }
}

}  // namespace

hipError_t rmda_launch_route(hipStream_t s, const float *proj, uint32_t *idx, float *wt,
                             uint32_t *count, uint32_t rows, uint32_t experts, uint32_t topk,
                             uint32_t stride) {
    if (rows == 0) {
        return hipSuccess;
    }
    dim3 grid((rows + 3) / 4);
    const uint32_t nv = (experts + RMDA_WAVE - 1) / RMDA_WAVE;
    if (nv <= 1) {
        hipLaunchKernelGGL(route_kernel<1>, grid, dim3(256), 0, s, proj, idx, wt, count, rows, experts, topk, stride);
    } else if (nv <= 2) {
        hipLaunchKernelGGL(route_kernel<2>, grid, dim3(256), 0, s, proj, idx, wt, count, rows, experts, topk, stride);
    } else if (nv <= 4) {
        hipLaunchKernelGGL(route_kernel<4>, grid, dim3(256), 0, s, proj, idx, wt, count, rows, experts, topk, stride);
    } else {
        hipLaunchKernelGGL(route_kernel<MAXV>, grid, dim3(256), 0, s, proj, idx, wt, count, rows, experts, topk, stride);
    }
    return hipGetLastError();
}
