// Stable permutation into expert-contiguous rows: the deterministic redesign
// of shader/moe_scatter.comp.
//
// slot[pr] = boff[pr / RMDA_RANK_BLOCK][e] + lrank[pr] with boff and lrank from
// rank_kernel, which equals off[e] + (number of pr' < pr with idx[pr'] == e):
// what the reference's atomicAdd(fill[e]) gives when its workgroups run in
// pr order (shader/moe_scatter.comp:22-27), with no atomics at all.
//
// Three kernels:
//  - map only (fused layer): one thread per pair writes slot and the inverse
//    map rowtok[slot] = token, which the gate_up GEMM gathers through;
//  - copy (drop-in rmda_moe_scatter above RMDA_SCATTER1_MAX_PAIRS pairs):
//    one wave per token reads the token's row once (16-byte chunks,
//    coalesced) and writes it to each of its topk slots.  The reference
//    reads the row once per pair (:29-32);
//  - scatter1 (drop-in rmda_moe_scatter up to that bound): the same copy with
//    the ranks computed in the same launch (below), so no rank kernel runs.
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

// Row copy of the permutation: lanes 0..topk-1 of `mine` name the xp rows
// that receive token row `src` (d8 16-byte chunks).  Each lane loads
// CP_BATCH chunks before storing any, so a wave keeps CP_BATCH loads in
// flight instead of waiting out one load per 64 chunks.
constexpr uint32_t CP_BATCH = 4;

__device__ __forceinline__ void load_batch(const uint4 *__restrict__ src, uint32_t c0, uint32_t d8,
                                           uint32_t lane, bool live, uint4 (&v)[CP_BATCH]) {
#pragma unroll
    for (uint32_t u = 0; u < CP_BATCH; u += 1) {
        const uint32_t c = c0 + u * RMDA_WAVE + lane;
        v[u] = (live && c < d8) ? src[c] : make_uint4(0, 0, 0, 0);
    }
}

// every lane runs every round so the slot broadcasts see all lanes
__device__ __forceinline__ void store_batch(uint4 *__restrict__ xp, uint32_t mine, uint32_t topk, uint32_t c0,
                                            uint32_t d8, uint32_t lane, const uint4 (&v)[CP_BATCH]) {
    for (uint32_t j = 0; j < topk; j += 1) {
        const uint32_t s = __shfl(mine, j);
        if (s != RMDA_NONE) {
#pragma unroll
            for (uint32_t u = 0; u < CP_BATCH; u += 1) {
                const uint32_t c = c0 + u * RMDA_WAVE + lane;
                if (c < d8) {
                    xp[(size_t)s * d8 + c] = v[u];
                }
            }
        }
    }
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
    for (uint32_t c0 = 0; c0 < d8; c0 += CP_BATCH * RMDA_WAVE) {
        uint4 v[CP_BATCH];
        load_batch(src, c0, d8, lane, true, v);
        store_batch(xp, mine, topk, c0, d8, lane, v);
    }
}

// The drop-in scatter in one launch, for up to RMDA_SCATTER1_MAX_PAIRS pairs.
// Block b owns tokens [4b, 4b+4), i.e. pairs [p0, p0 + 4*topk) with
// p0 = 4b*topk, and computes everything it needs itself:
//   1. an LDS histogram of idx[0, p0): pair pr's rank among the pairs of its
//      expert is that count plus the number of earlier pairs of its own block
//      with the same expert (a wave-0 compare over at most 64 pairs);
//   2. slot = off[e] + rank, as the two-kernel path (rank, then permute);
//   3. each wave copies one token's row to its k slots (the row's first
//      chunks are loaded before the count, so their latency is hidden).
// Nothing passes between blocks, so no block waits on another.  The
// histogram costs O(p0) L2 reads per block, O(npairs^2) in all, which is why
// the size is bounded: at BASELINE config 3 (16 K pairs) it is 16 MB of L2
// reads, and blocks with short prefixes are already copying while the later
// ones count.  The last block adds its own pairs and writes `fill` (the
// per-expert counts).
template <bool VEC>
__global__ __launch_bounds__(256) void scatter1_kernel(const uint32_t *__restrict__ idx,
                                                       const uint32_t *__restrict__ off,
                                                       uint32_t *__restrict__ fill, uint32_t rows,
                                                       uint32_t topk, uint32_t experts,
                                                       uint32_t *__restrict__ slot,
                                                       const uint4 *__restrict__ x16,
                                                       uint4 *__restrict__ xp, uint32_t d8) {
    __shared__ uint32_t hist[RMDA_MAX_EXPERTS];
    __shared__ uint32_t sslot[4 * RMDA_MAX_TOPK];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % RMDA_WAVE;
    const uint32_t w = tid / RMDA_WAVE;
    const uint32_t npairs = rows * topk;
    const uint32_t p0 = blockIdx.x * 4 * topk;  // a multiple of 4
    const uint32_t bp = min(4 * topk, npairs - p0);
    // this wave's token row: its first chunks are loaded now and land while
    // the block counts
    const uint32_t r = blockIdx.x * 4 + w;
    const bool live = r < rows;
    const uint4 *src = x16 + (size_t)(live ? r : 0) * d8;
    uint4 v0[CP_BATCH];
    load_batch(src, 0, d8, lane, live, v0);
    for (uint32_t e = tid; e < experts; e += 256) {
        hist[e] = 0;
    }
    __syncthreads();
    if (VEC) {
        // four 16-byte loads in flight per thread, then their 16 counts
        const uint4 *iv = reinterpret_cast<const uint4 *>(idx);
        const uint32_t n4 = p0 / 4;
        for (uint32_t i = tid; i < n4; i += 1024) {
            uint4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u += 1) {
                const uint32_t j = i + u * 256;
                v[u] = j < n4 ? iv[j] : make_uint4(RMDA_NONE, RMDA_NONE, RMDA_NONE, RMDA_NONE);
            }
#pragma unroll
            for (int u = 0; u < 4; u += 1) {
                const uint32_t q[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (int t = 0; t < 4; t += 1) {
                    if (q[t] < experts) {
                        atomicAdd(&hist[q[t]], 1u);
                    }
                }
            }
        }
    } else {
        for (uint32_t i = tid; i < p0; i += 256) {
            const uint32_t e = idx[i];
            if (e < experts) {
                atomicAdd(&hist[e], 1u);
            }
        }
    }
    __syncthreads();
    uint32_t e = RMDA_NONE;
    if (w == 0) {
        if (lane < bp) {
            e = idx[p0 + lane];
            e = e < experts ? e : RMDA_NONE;
        }
        uint32_t rk = 0;
        for (uint32_t j = 0; j < bp; j += 1) {
            const uint32_t ej = (uint32_t)__builtin_amdgcn_readlane((int)e, (int)j);
            rk += (j < lane && ej == e) ? 1u : 0u;
        }
        if (lane < bp) {
            const uint32_t s = e != RMDA_NONE ? off[e] + hist[e] + rk : RMDA_NONE;
            slot[p0 + lane] = s;
            sslot[lane] = s;
        }
    }
    __syncthreads();
    if (blockIdx.x == gridDim.x - 1) {
        // the last block's prefix plus its own pairs: every pair counted
        if (w == 0 && e != RMDA_NONE) {
            atomicAdd(&hist[e], 1u);
        }
        __syncthreads();
        for (uint32_t c = tid; c < experts; c += 256) {
            fill[c] = hist[c];
        }
    }
    if (!live) {
        return;
    }
    const uint32_t mine = lane < topk ? sslot[w * topk + lane] : RMDA_NONE;
    store_batch(xp, mine, topk, 0, d8, lane, v0);
    for (uint32_t c0 = CP_BATCH * RMDA_WAVE; c0 < d8; c0 += CP_BATCH * RMDA_WAVE) {
        uint4 v[CP_BATCH];
        load_batch(src, c0, d8, lane, true, v);
        store_batch(xp, mine, topk, c0, d8, lane, v);
    }
}

}  // namespace

hipError_t rmda_launch_scatter1(hipStream_t s, const uint32_t *idx, const uint32_t *off, uint32_t *fill,
                                uint32_t rows, uint32_t topk, uint32_t experts, uint32_t *slot,
                                const uint16_t *x16, uint16_t *xp, uint32_t d8) {
    if (rows == 0) {
        return hipSuccess;
    }
    const dim3 grid((rows + 3) / 4);
    const uint4 *xs = reinterpret_cast<const uint4 *>(x16);
    uint4 *xd = reinterpret_cast<uint4 *>(xp);
    if ((reinterpret_cast<uintptr_t>(idx) & 15u) == 0) {
        hipLaunchKernelGGL(scatter1_kernel<true>, grid, dim3(256), 0, s, idx, off, fill, rows, topk, experts, slot,
                           xs, xd, d8);
    } else {
        hipLaunchKernelGGL(scatter1_kernel<false>, grid, dim3(256), 0, s, idx, off, fill, rows, topk, experts,
                           slot, xs, xd, d8);
    }
    return hipGetLastError();
}

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
