// Stable permutation into expert-contiguous rows: the deterministic redesign
// of shader/moe_scatter.comp.
//
// slot[pr] = boff[pr / RMDA_RANK_BLOCK][e] + lrank[pr] with boff and lrank from
// rank_kernel, which equals off[e] + (number of pr' < pr with idx[pr'] == e):
// what the reference's atomicAdd(fill[e]) gives when its workgroups run in
// pr order (shader/moe_scatter.comp:22-27), with no atomics at all.
//
// Two variants:
//  - map only (fused layer): one thread per pair writes slot and the inverse
//    map rowtok[slot] = token, which the gate_up GEMM gathers through;
//  - copy (drop-in rmda_moe_scatter): one wave per token reads the token's
//    row once (16-byte chunks, coalesced) and writes it to each of its topk
//    slots.  The reference reads the row once per pair (:29-32).
#include "common.h"

namespace {

__device__ __forceinline__ uint32_t pair_slot(const uint32_t *idx, const uint32_t *lrank,
                                              const uint32_t *boff, uint32_t pr,
                                              uint32_t experts) {
    const uint32_t e = idx[pr];
    if (e >= experts) {
        return RMDA_NONE;
    }
    return boff[(size_t)(pr / RMDA_RANK_BLOCK) * experts + e] + lrank[pr];
}

__global__ __launch_bounds__(256) void permute_map_kernel(const uint32_t *__restrict__ idx,
                                                          const uint32_t *__restrict__ lrank,
                                                          const uint32_t *__restrict__ boff,
                                                          uint32_t npairs, uint32_t topk,
                                                          uint32_t experts,
                                                          uint32_t *__restrict__ slot,
                                                          uint32_t *__restrict__ rowtok) {
    const uint32_t pr = blockIdx.x * 256 + threadIdx.x;
    if (pr >= npairs) {
        return;
    }
    const uint32_t s = pair_slot(idx, lrank, boff, pr, experts);
    slot[pr] = s;
    if (rowtok != nullptr && s != RMDA_NONE) {
        rowtok[s] = pr / topk;
    }
}

__global__ __launch_bounds__(256) void permute_copy_kernel(const uint32_t *__restrict__ idx,
                                                           const uint32_t *__restrict__ lrank,
                                                           const uint32_t *__restrict__ boff,
                                                           uint32_t rows, uint32_t topk,
                                                           uint32_t experts,
                                                           uint32_t *__restrict__ slot,
                                                           const uint4 *__restrict__ x16,
                                                           uint4 *__restrict__ xp, uint32_t d8) {
    const uint32_t lane = threadIdx.x % RMDA_WAVE;
    const uint32_t r = blockIdx.x * 4 + threadIdx.x / RMDA_WAVE;
    if (r >= rows) {
        return;
    }
    uint32_t mine = RMDA_NONE;
    if (lane < topk) {
        const uint32_t pr = r * topk + lane;
        mine = pair_slot(idx, lrank, boff, pr, experts);
        slot[pr] = mine;
    }
    const uint4 *src = x16 + (size_t)r * d8;
    // every lane runs every iteration so the slot broadcasts see all lanes
    for (uint32_t c0 = 0; c0 < d8; c0 += RMDA_WAVE) {
        const uint32_t c = c0 + lane;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (c < d8) {
            v = src[c];
        }
        for (uint32_t j = 0; j < topk; j += 1) {
            const uint32_t s = __shfl(mine, j);
            if (s != RMDA_NONE && c < d8) {
                xp[(size_t)s * d8 + c] = v;
            }
        }
    }
}

}  // namespace

hipError_t rmda_launch_permute(hipStream_t s, const uint32_t *idx, const uint32_t *lrank,
                               const uint32_t *boff, uint32_t npairs, uint32_t topk,
                               uint32_t experts, uint32_t *slot, uint32_t *rowtok,
                               const uint16_t *x16, uint16_t *xp, uint32_t d8) {
    if (npairs == 0) {
        return hipSuccess;
    }
    if (xp == nullptr) {
        hipLaunchKernelGGL(permute_map_kernel, dim3((npairs + 255) / 256), dim3(256), 0, s, idx, lrank,
                           boff, npairs, topk, experts, slot, rowtok);
    } else {
        const uint32_t rows = npairs / topk;
        hipLaunchKernelGGL(permute_copy_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, idx, lrank, boff,
                           rows, topk, experts, slot, reinterpret_cast<const uint4 *>(x16),
                           reinterpret_cast<uint4 *>(xp), d8);
    }
    return hipGetLastError();
}
