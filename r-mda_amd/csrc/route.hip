// Top-k gating: the wave64 redesign of shader/moe_route.comp.
//
// Reference semantics (shader/moe_route.comp:20-61): per row, topk rounds;
// each round takes the largest untaken logit by strict '>' from -3.0e38, so
// the lowest expert index wins ties and NaN / values <= -3e38 are never
// taken; idx is emitted in selection (descending) order; lane 0 sums
// z = sum_k exp(l_k - l_0) in selection order and writes wt_k = exp(l_k-l_0)/z;
// count[e] += 1 per selection.
//
// Here one wave owns one row (rmda_route_row in common.h).  Lane l holds
// columns l, l+64, ... (coalesced; up to 8 per lane for 512 experts) instead
// of the reference's 16 contiguous columns on 32 lanes.  A round is one
// lane-local scan, one wave-wide max of the order-preserving float key,
// which yields the largest value, and the lowest column holding it: read
// from the one lane that holds the maximum or, when several lanes tie, a
// wave-wide min over their columns.  Only columns < experts are read (the
// reference reads 512 columns regardless).
#include "common.h"

namespace {

constexpr int MAXV = RMDA_MAX_EXPERTS / RMDA_WAVE;  // values per lane

template <int NV>
__global__ __launch_bounds__(256) void route_kernel(const float *__restrict__ proj,
                                                    uint32_t *__restrict__ idx,
                                                    float *__restrict__ wt,
                                                    uint32_t *__restrict__ count, uint32_t rows,
                                                    uint32_t experts, uint32_t topk,
                                                    uint32_t stride) {
    const uint32_t r = blockIdx.x * 4 + threadIdx.x / RMDA_WAVE;
    if (r >= rows) {
        return;
    }
    rmda_route_row<NV, false>(proj + (size_t)r * stride, experts, topk, idx + (size_t)r * topk,
                              wt + (size_t)r * topk, count);
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
