// Expert offsets (moe_scan) and the deterministic ranking behind the stable
// permutation (the order moe_scatter's atomics would give if the pairs ran
// one after another).
//
// rank_kernel: pairs are cut into blocks of RMDA_RANK_BLOCK.  A workgroup of
// NT threads walks its block NT pairs at a time; each wave ORs a 64-bit lane
// mask per expert in LDS, so a pair's rank among equal experts in its block
// is (running count) + (masks of lower waves) + popcount(own mask & lanes
// below).  The block's per-expert totals go to hist[b][e].  The last block to
// finish (atomic ticket) converts hist into per-block base offsets, writes
// off/count, and builds the grouped-GEMM work list, so the whole ranking is
// one launch with no host round trip and no atomic-order dependence.
// Two shortcuts skip the hand-off: a single block's counts are the totals,
// and with count_all (up to RMDA_RANK_ALL_MAX pairs) every block also counts
// the pairs before and after its own in LDS, which gives it the totals and
// its own bases.  In both cases the blocks write slot and rowtok themselves
// (no permutation launch), and block 0 alone writes the shared outputs.
#include "common.h"

namespace {

constexpr uint32_t NT0 = 256;  // threads of the helper kernels and of a single-block rank launch

__global__ __launch_bounds__(256) void zero_kernel(uint32_t *p, size_t n, uint32_t value) {
    for (size_t i = blockIdx.x * (size_t)NT0 + threadIdx.x; i < n; i += (size_t)gridDim.x * NT0) {
        p[i] = value;
    }
}

// Exclusive scan of one value per thread over an NT-thread block.
template <uint32_t NT>
__device__ uint32_t block_exscan(uint32_t v, uint32_t *sbuf, uint32_t *total) {
    const uint32_t lane = threadIdx.x % RMDA_WAVE;
    const uint32_t w = threadIdx.x / RMDA_WAVE;
    // inclusive wave scan in registers: DPP row_shr 1, 2, 4, 8 within each
    // 16-lane row (lanes shifted in from outside the row add 0), then
    // row_bcast 15 and 31 carry the row totals upward
    uint32_t x = v;
    x += __builtin_amdgcn_update_dpp(0u, x, 0x111, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, 0x112, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, 0x114, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, 0x118, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, 0x142, 0xA, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, 0x143, 0xC, 0xF, false);
    if (lane == RMDA_WAVE - 1) {
        sbuf[w] = x;
    }
    __syncthreads();
    uint32_t base = 0;
    uint32_t tot = 0;
    for (uint32_t i = 0; i < NT / RMDA_WAVE; i += 1) {
        base += i < w ? sbuf[i] : 0u;
        tot += sbuf[i];
    }
    __syncthreads();
    *total = tot;
    return base + x - v;
}

// block_exscan of v, and in the same pass (one pair of barriers) the block
// totals of u1 and u2; sbuf holds 3 * NT / 64 words.
template <uint32_t NT>
__device__ uint32_t block_exscan3(uint32_t v, uint32_t u1, uint32_t u2, uint32_t *sbuf, uint32_t *total,
                                  uint32_t *total1, uint32_t *total2) {
    constexpr uint32_t NW = NT / RMDA_WAVE;
    const uint32_t lane = threadIdx.x % RMDA_WAVE;
    const uint32_t w = threadIdx.x / RMDA_WAVE;
    uint32_t x[3] = {v, u1, u2};
#pragma unroll
    for (uint32_t j = 0; j < 3; j += 1) {
        x[j] += __builtin_amdgcn_update_dpp(0u, x[j], 0x111, 0xF, 0xF, false);
        x[j] += __builtin_amdgcn_update_dpp(0u, x[j], 0x112, 0xF, 0xF, false);
        x[j] += __builtin_amdgcn_update_dpp(0u, x[j], 0x114, 0xF, 0xF, false);
        x[j] += __builtin_amdgcn_update_dpp(0u, x[j], 0x118, 0xF, 0xF, false);
        x[j] += __builtin_amdgcn_update_dpp(0u, x[j], 0x142, 0xA, 0xF, false);
        x[j] += __builtin_amdgcn_update_dpp(0u, x[j], 0x143, 0xC, 0xF, false);
    }
    if (lane == RMDA_WAVE - 1) {
        sbuf[w] = x[0];
        sbuf[NW + w] = x[1];
        sbuf[2 * NW + w] = x[2];
    }
    __syncthreads();
    uint32_t base = 0;
    uint32_t t[3] = {0u, 0u, 0u};
    for (uint32_t i = 0; i < NW; i += 1) {
        base += i < w ? sbuf[i] : 0u;
        t[0] += sbuf[i];
        t[1] += sbuf[NW + i];
        t[2] += sbuf[2 * NW + i];
    }
    __syncthreads();
    *total = t[0];
    *total1 = t[1];
    *total2 = t[2];
    return base + x[0] - v;
}

// shader/moe_scan.comp:14-37, one thread per expert (experts <= 512).
// tiles[t] is written once per t: the owner is found by binary search over
// the inclusive padded prefix instead of relying on a pre-fill.
__global__ __launch_bounds__(512) void scan_kernel(const uint32_t *__restrict__ count,
                                                   uint32_t *__restrict__ off,
                                                   uint32_t *__restrict__ tiles,
                                                   uint32_t n_tiles, uint32_t experts,
                                                   uint32_t tile) {
    __shared__ uint32_t s[512];
    const uint32_t e = threadIdx.x;
    uint32_t p = 0;
    if (e < experts) {
        p = (count[e] + tile - 1u) / tile * tile;
    }
    s[e] = p;
    __syncthreads();
    for (uint32_t dd = 1; dd < 512; dd <<= 1) {
        uint32_t v = s[e];
        if (e >= dd) {
            v += s[e - dd];
        }
        __syncthreads();
        s[e] = v;
        __syncthreads();
    }
    if (e < experts) {
        off[e] = s[e] - p;
    }
    for (uint32_t t = e; t < n_tiles; t += 512) {
        // first expert whose inclusive end exceeds t*tile
        const uint64_t row = (uint64_t)t * tile;
        uint32_t lo = 0;
        uint32_t hi = experts;
        while (lo < hi) {
            uint32_t mid = (lo + hi) / 2;
            if ((uint64_t)s[mid] > row) {
                hi = mid;
            } else {
                lo = mid + 1;
            }
        }
        tiles[t] = lo < experts ? lo : RMDA_NONE;
    }
}

// Upper bound on the polls of a rank block that waits for the routing
// blocks of its launch (each poll is one device-scope load and a short
// sleep, so about a second in all): a safety net that lets every wave exit
// even if the ticket never completed; it is never reached in a correct run.
constexpr uint32_t kRouteWaitPolls = 1u << 20;

// NV > 0: the top-k folded in (rmda_rank_args_t::route_proj), NV logits per
// lane: one block per NT / 64 rows routes; the blocks that take the last
// nb tickets (nb = the rank blocks of npairs) then rank.
template <uint32_t NT, int NV>
__global__ __launch_bounds__(NT) void rank_kernel(rmda_rank_args_t a) {
    __shared__ unsigned long long msk[NT / RMDA_WAVE][RMDA_MAX_EXPERTS];
    __shared__ uint32_t run[RMDA_MAX_EXPERTS];
    __shared__ uint32_t sbuf[3 * NT / RMDA_WAVE];  // block scans (block_exscan3 uses all three rows)
    __shared__ uint32_t s_last;
    __shared__ uint32_t cls_n[RMDA_ITEM_CLASSES];  // work-list items per 16-row class
    __shared__ uint32_t cls_b[RMDA_ITEM_CLASSES];
    __shared__ uint32_t sh_slot[2];
    __shared__ uint32_t pre[RMDA_MAX_EXPERTS];   // count_all: pairs before this block
    __shared__ uint32_t post[RMDA_MAX_EXPERTS];  // count_all: pairs after it
    // count_all counts pre and post into CS copies of each, lane l adding to
    // copy l % CS, and then sums the copies.  A wave's lanes hold
    // consecutive pairs, so under skewed routing (one expert in the same
    // top-k slot of most tokens) half of a wave's lanes add to the same
    // expert, and the LDS serialises adds to one word.  A row of CW words
    // (one spare) puts copy s of expert e in its own bank.
    constexpr uint32_t CS = NT >= 1024 || NV > 0 ? 8u : 1u;  // the launches that may count_all
    constexpr uint32_t CW = RMDA_MAX_EXPERTS + 1u;
    __shared__ uint32_t hcopy[2 * CS * CW];  // [pre, post][CS][CW]
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid % RMDA_WAVE;
    const uint32_t w = tid / RMDA_WAVE;
    const uint32_t E = a.experts;
    // routed: rank blocks are dealt by ticket below; otherwise one per workgroup
    const uint32_t nb = NV > 0 ? (a.npairs + RMDA_RANK_BLOCK - 1u) / RMDA_RANK_BLOCK : gridDim.x;
    uint32_t b = NV > 0 ? 0u : blockIdx.x;
    // every block counts every pair itself: no hand-off, and each block
    // writes its own slots (see rmda_rank_args_t::count_all)
    const bool all = a.count_all != 0 && nb > 1;
    // this kernel writes the slots itself (below), so lrank is not needed
    const bool self_slots = a.slot != nullptr && (nb == 1 || all);

    for (uint32_t e = tid; e < E; e += NT) {
        run[e] = 0;
        pre[e] = 0;
        post[e] = 0;
    }
    if (all) {
        for (uint32_t i = tid; i < 2 * CS * CW; i += NT) {
            hcopy[i] = 0u;
        }
    }
    // Top-k folded in: block r's wave w routes row (NT/64)*r + w as
    // route_kernel does, storing its experts with device-scope stores.  Each
    // block then takes a ticket (a zero word the router kernel cleared at the
    // start of the call) with a device-scope release increment, so its idx
    // stores happen before the ticket.  The blocks that draw the last nb
    // tickets become rank blocks nb-1 ... 0 in ticket order and wait until
    // every block has drawn one (the one that drew the last ticket needs no
    // wait); a device-scope acquire fence then makes every block's idx visible
    // to this block's loads, and they rank as the nb blocks of an unrouted
    // launch do.  The other blocks leave.  At most nb blocks ever wait, and a
    // waiting block drew its ticket after routing, so the blocks still to
    // route can always be scheduled (the device holds far more than nb of
    // these workgroups at once): no co-residency of the whole grid is needed.
    if constexpr (NV > 0) {
        const uint32_t t = blockIdx.x * (NT / RMDA_WAVE) + w;
        if (t < a.route_rows) {
            float v[NV];
            rmda_route_load<NV, false>(a.route_proj + (size_t)t * a.route_stride, E, v);
            rmda_route_select<NV, true>(v, a.topk, a.route_idx + (size_t)t * a.topk, a.route_wt + (size_t)t * a.topk,
                                        nullptr, nullptr);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const uint32_t G = gridDim.x;
        if (tid == 0) {
            const uint32_t tk = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            if (tk + nb >= G) {
                if (tk + 1u < G) {
                    for (uint32_t n = 0;
                         __hip_atomic_load(a.done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < G && n < kRouteWaitPolls;
                         n += 1) {
                        __builtin_amdgcn_s_sleep(2);
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            }
            s_last = tk;
        }
        __syncthreads();
        if (s_last + nb < G) {
            return;
        }
        b = G - 1u - s_last;
    }
    // a pair's expert: written by other blocks of this launch when it routed
    auto pair_expert = [&](uint32_t pr) -> uint32_t {
        if constexpr (NV > 0) {
            return rmda_load_agent(&a.idx[pr]);
        } else {
            return a.idx[pr];
        }
    };
    // Folded combine: preset each token's arrival counters to the number of
    // rows it sends through the down GEMM.  Block b takes the tokens whose
    // first pair lies in its own 1024 pairs (so their idx words are mostly the
    // ones this block loads below); a token with no rows at all gets the zero
    // output row the combine would have written.
    if (a.fc_cnt != nullptr) {
        const uint32_t K = a.topk;
        const uint32_t t_lo = (b * RMDA_RANK_BLOCK + K - 1) / K;
        const uint32_t t_hi = min(((b + 1) * RMDA_RANK_BLOCK + K - 1) / K, a.fc_rows);
        for (uint32_t t = t_lo + tid; t < t_hi; t += NT) {
            uint32_t n = a.fc_shared;
            for (uint32_t j = 0; j < K; j += 1) {
                n += pair_expert(t * K + j) < E ? 1u : 0u;
            }
            uint4 *c4 = reinterpret_cast<uint4 *>(a.fc_cnt + (size_t)t * a.fc_nblk);
            for (uint32_t q = 0; q < a.fc_nblk / 4; q += 1) {
                c4[q] = make_uint4(n, n, n, n);
            }
            if (n == 0 && a.fc_zero_out != nullptr) {
                uint4 *o4 = reinterpret_cast<uint4 *>(a.fc_zero_out + (size_t)t * a.fc_d);
                for (uint32_t q = 0; q < a.fc_d / 8; q += 1) {
                    o4[q] = make_uint4(0u, 0u, 0u, 0u);
                }
            }
        }
    }
    // count_all: the other blocks' pairs as 16-byte words, CB per thread per
    // batch; the first batch is issued now and lands during the ranking
    // below (idx was written on other XCDs, so these loads miss L2)
    constexpr uint32_t CB = 16;
    const uint4 *iv = reinterpret_cast<const uint4 *>(a.idx);
    const uint32_t n4 = a.npairs / 4;
    const uint32_t own_lo = b * (RMDA_RANK_BLOCK / 4);
    const uint32_t own_hi = own_lo + RMDA_RANK_BLOCK / 4;
    uint4 cv[CB];
    auto count_load = [&](uint32_t i0) {
#pragma unroll
        for (uint32_t u = 0; u < CB; u += 1) {
            const uint32_t j = i0 + u * NT;
            cv[u] = (j < n4 && (j < own_lo || j >= own_hi)) ? iv[j]
                                                           : make_uint4(RMDA_NONE, RMDA_NONE, RMDA_NONE, RMDA_NONE);
        }
    };
    auto count_add = [&](uint32_t i0) {
#pragma unroll
        for (uint32_t u = 0; u < CB; u += 1) {
            uint32_t *h = hcopy + ((i0 + u * NT < own_lo ? 0u : CS) + lane % CS) * CW;
            const uint32_t q[4] = {cv[u].x, cv[u].y, cv[u].z, cv[u].w};
#pragma unroll
            for (uint32_t t = 0; t < 4; t += 1) {
                if (q[t] < E) {
                    atomicAdd(&h[q[t]], 1u);
                }
            }
        }
    };
    if (all) {
        count_load(tid);
    }
    const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (RMDA_WAVE - lane));
    // all of the thread's experts are loaded up front: one memory round trip
    // for the block instead of one per 256 pairs
    constexpr uint32_t ITS = RMDA_RANK_BLOCK / NT;
    uint32_t ev[ITS];
    uint32_t lr[ITS];  // local ranks, kept for the single-block permutation
#pragma unroll
    for (uint32_t it = 0; it < ITS; it += 1) {
        const uint32_t pr = b * RMDA_RANK_BLOCK + it * NT + tid;
        ev[it] = pr < a.npairs ? pair_expert(pr) : RMDA_NONE;
    }
#pragma unroll
    for (uint32_t it = 0; it < ITS; it += 1) {
        for (uint32_t e = lane; e < E; e += RMDA_WAVE) {
            msk[w][e] = 0ull;
        }
        __syncthreads();
        const uint32_t pr = b * RMDA_RANK_BLOCK + it * NT + tid;
        const uint32_t e = ev[it] < E ? ev[it] : RMDA_NONE;
        if (e != RMDA_NONE) {
            atomicOr(&msk[w][e], 1ull << lane);
        }
        __syncthreads();
        if (e != RMDA_NONE) {
            uint32_t r = run[e];
            for (uint32_t ww = 0; ww < w; ww += 1) {
                r += __popcll(msk[ww][e]);
            }
            r += __popcll(msk[w][e] & below);
            if (!self_slots) {
                a.lrank[pr] = r;  // for the permutation kernel
            }
            lr[it] = r;
        }
        __syncthreads();
        for (uint32_t e2 = tid; e2 < E; e2 += NT) {
            uint32_t add = 0;
            for (uint32_t ww = 0; ww < NT / RMDA_WAVE; ww += 1) {
                add += __popcll(msk[ww][e2]);
            }
            run[e2] += add;
        }
        __syncthreads();
    }
    // Hand-off: the last block to arrive finalises.  Every wave stores its
    // share of the block totals with device-scope atomic stores and waits for
    // them (vmcnt(0)) before the workgroup barrier; thread 0 then takes the
    // ticket with a device-scope acquire-release increment, which releases
    // the block's totals to the last block and, in the last block, acquires
    // all of them before its device-scope loads read them.
    // A single block needs no hand-off: its own counts (run[]) are the totals.
    if (all) {
        count_add(tid);
        for (uint32_t i0 = tid + CB * NT; i0 < n4; i0 += CB * NT) {
            count_load(i0);
            count_add(i0);
        }
        // the last npairs % 4 pairs (past the 16-byte words) are the last
        // block's own, i.e. after every other block
        if (b + 1 < nb && tid < a.npairs - 4 * n4) {
            const uint32_t e = a.idx[4 * n4 + tid];
            if (e < E) {
                atomicAdd(&hcopy[(CS + lane % CS) * CW + e], 1u);
            }
        }
        __syncthreads();
        // thread i < E sums pre[i], thread E + i post[i]
        for (uint32_t i = tid; i < 2 * E; i += NT) {
            const uint32_t hi = i >= E ? 1u : 0u;
            const uint32_t e = i - hi * E;
            uint32_t n = 0;
#pragma unroll
            for (uint32_t c = 0; c < CS; c += 1) {
                n += hcopy[(hi * CS + c) * CW + e];
            }
            (hi != 0 ? post : pre)[e] = n;
        }
        __syncthreads();
    } else if (nb > 1) {
        for (uint32_t e = tid; e < E; e += NT) {
            __hip_atomic_store(&a.hist[(size_t)b * E + e], run[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            // the increment wraps the ticket back to 0 on the last block
            s_last = __builtin_amdgcn_atomic_inc32(a.done, nb - 1, __ATOMIC_ACQ_REL, "agent") == nb - 1;
        }
        __syncthreads();
        if (!s_last) {
            return;
        }
    }

    // Each thread owns experts e0 = 2t and e0+1.  Pass 1: column totals of
    // hist over blocks (other blocks' words read at device scope, RB blocks
    // of both experts in flight at a time instead of one dependent round trip
    // per block).  Padded widths and offsets follow from one block-wide scan.
    // Pass 2: hist[b][e] <- off[e] + sum_{b'<b} hist[b'][e], from the values
    // pass 1 kept when nb <= RB, else reloaded RB blocks at a time.
    constexpr uint32_t RB = 16;
    const uint32_t e0 = 2 * tid;
    const bool own0 = e0 < E;
    const bool own1 = e0 + 1 < E;
    uint32_t h0[RB], h1[RB];
    auto load_batch = [&](uint32_t bb0) {
#pragma unroll
        for (uint32_t u = 0; u < RB; u += 1) {
            const bool in = bb0 + u < nb;
            h0[u] = in && own0 ? rmda_load_agent(&a.hist[(size_t)(bb0 + u) * E + e0]) : 0u;
            h1[u] = in && own1 ? rmda_load_agent(&a.hist[(size_t)(bb0 + u) * E + e0 + 1]) : 0u;
        }
    };
    uint32_t c0 = 0;
    uint32_t c1 = 0;
    if (nb == 1 || all) {
#pragma unroll
        for (uint32_t u = 0; u < RB; u += 1) {
            h0[u] = 0u;
            h1[u] = 0u;
        }
        h0[0] = own0 ? pre[e0] + run[e0] + post[e0] : 0u;
        h1[0] = own1 ? pre[e0 + 1] + run[e0 + 1] + post[e0 + 1] : 0u;
        c0 = h0[0];
        c1 = h1[0];
    } else {
        for (uint32_t bb0 = 0; bb0 < nb; bb0 += RB) {
            load_batch(bb0);
#pragma unroll
            for (uint32_t u = 0; u < RB; u += 1) {
                c0 += h0[u];
                c1 += h1[u];
            }
        }
    }
    const uint32_t p0 = (c0 + a.tile - 1u) / a.tile * a.tile;
    const uint32_t p1 = (c1 + a.tile - 1u) / a.tile * a.tile;
    // offsets, and with them the two totals the tile choice below needs
    // (all rows; rows of experts with at least hot_min rows)
    const uint32_t hm = a.hot_min;
    uint32_t total = 0;
    uint32_t rows_all = 0;
    uint32_t rows_hot = 0;
    const uint32_t base = block_exscan3<NT>(p0 + p1, c0 + c1, (c0 >= hm ? c0 : 0u) + (c1 >= hm ? c1 : 0u), sbuf,
                                            &total, &rows_all, &rows_hot);
    uint32_t o0 = base;
    uint32_t o1 = base + p0;
    if (a.off_in != nullptr) {
        o0 = own0 ? a.off_in[e0] : 0u;
        o1 = own1 ? a.off_in[e0 + 1] : 0u;
    }
    const bool lead = !all || b == 0;  // the block that writes the shared outputs
    if (own0 && lead) {
        if (a.off != nullptr) {
            a.off[e0] = o0;
        }
        if (a.count != nullptr) {
            a.count[e0] = c0;
        }
    }
    if (own1 && lead) {
        if (a.off != nullptr) {
            a.off[e0 + 1] = o1;
        }
        if (a.count != nullptr) {
            a.count[e0 + 1] = c1;
        }
    }
    if (self_slots) {
        // The block knows its pairs' bases: it writes the permutation itself,
        // slot = off[e] + pairs of e before the block + local rank, and the
        // row -> token map, so the separate permutation launch is not needed.
        // run[] (this block's counts, no longer needed) now holds the bases.
        __syncthreads();
        if (own0) {
            run[e0] = o0 + pre[e0];
        }
        if (own1) {
            run[e0 + 1] = o1 + pre[e0 + 1];
        }
        __syncthreads();
#pragma unroll
        for (uint32_t it = 0; it < ITS; it += 1) {
            const uint32_t pr = b * RMDA_RANK_BLOCK + it * NT + tid;
            if (pr < a.npairs) {
                const uint32_t e = ev[it];
                const uint32_t sl = e < E ? run[e] + lr[it] : RMDA_NONE;
                a.slot[pr] = sl;
                if (a.rowtok != nullptr && sl != RMDA_NONE) {
                    a.rowtok[sl] = pr / a.topk;
                }
            }
        }
    }
    if (all && b != 0) {
        return;  // block 0 writes the work list
    }
    uint32_t acc0 = o0;
    uint32_t acc1 = o1;
    for (uint32_t bb0 = 0; bb0 < nb && !all; bb0 += RB) {
        if (nb > RB) {
            load_batch(bb0);
        }
#pragma unroll
        for (uint32_t u = 0; u < RB; u += 1) {
            if (bb0 + u < nb) {
                if (own0) {
                    a.hist[(size_t)(bb0 + u) * E + e0] = acc0;
                }
                if (own1) {
                    a.hist[(size_t)(bb0 + u) * E + e0 + 1] = acc1;
                }
            }
            acc0 += h0[u];
            acc1 += h1[u];
        }
    }
    if (a.items == nullptr) {
        return;
    }
    // Tile choice by expert load: when the experts with at least hot_min rows
    // (and the shared group, if it has that many) hold half the rows or more,
    // the list is cut into bm_hot-row items for the compute tile and
    // *n_items is 0; otherwise it is cut into bm-row items for the
    // weight-streaming tile and *n_items_hot is 0.  Each GEMM kernel reads its
    // own count, so the other one finds no work.
    uint32_t bm = a.bm;
    bool hot = false;
    if (a.n_items_hot != nullptr) {
        rows_all += a.shared_rows;
        rows_hot += a.shared_rows >= hm ? a.shared_rows : 0u;
        const bool hot_auto = hm > 0 && rows_hot > 0 && 2ull * rows_hot >= rows_all;
        hot = a.force == 2u ? true : a.force == 1u ? false : hot_auto;
        bm = hot ? a.bm_hot : a.bm;
        if (a.hint_out != nullptr && tid == 0) {
            __hip_atomic_store(a.hint_out, hot_auto ? 2u : 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        if (tid == 0) {
            *(hot ? a.n_items : a.n_items_hot) = 0u;
        }
    }
    uint32_t *const n_out = hot ? a.n_items_hot : a.n_items;
    if (hot) {
        // The compute tile's list is in expert order (an expert's items
        // adjacent, the shared group last), not sorted by rows: its default
        // schedule (task_sched_t) deals whole items to the XCDs in snake
        // order, and a compute-tile task costs about the same whatever its
        // rows (the weight slab's fill dominates; sorting by rows measured no
        // better).  The alternative schedule (chunk_sched_t) deals contiguous
        // runs of this order to each XCD, so that one XCD's CUs share an
        // expert's weight tiles in their L2.
        const uint32_t ni0 = (c0 + bm - 1u) / bm;
        const uint32_t ni1 = (c1 + bm - 1u) / bm;
        uint32_t n_routed = 0;
        const uint32_t base0 = block_exscan<NT>(ni0 + ni1, sbuf, &n_routed);
        uint4 *hitems = reinterpret_cast<uint4 *>(a.items);
        for (uint32_t j = 0; j < 2; j += 1) {
            const uint32_t c = j == 0 ? c0 : c1;
            const uint32_t o = j == 0 ? o0 : o1;
            const uint32_t b0 = j == 0 ? base0 : base0 + ni0;
            const uint32_t ni = j == 0 ? ni0 : ni1;
            for (uint32_t i = 0; i < ni; i += 1) {
                hitems[b0 + i] = make_uint4(e0 + j, o + i * bm, min(bm, c - i * bm), 0u);
            }
        }
        const uint32_t ns = (a.shared_rows + bm - 1u) / bm;
        for (uint32_t i = tid; i < ns; i += NT) {
            hitems[n_routed + i] = make_uint4(E, a.shared_row0 + i * bm, min(bm, a.shared_rows - i * bm), 0u);
        }
        if (tid == 0) {
            *n_out = n_routed + ns;
        }
        return;
    }
    // Grouped-GEMM work list: ceil(count/bm) items per expert plus the shared
    // group's, sorted by row count, largest first, in 16-row classes (the
    // GEMMs deal the list out in that order to balance their workgroups).
    // Each item takes a slot in its class with an LDS atomic, so the order
    // inside a class varies from run to run; an item's result does not.
    const uint32_t ncls = (bm + 15u) / 16u;
    if (tid < RMDA_ITEM_CLASSES) {
        cls_n[tid] = 0;
    }
    __syncthreads();
    uint32_t nfull[2], last_cls[2], slot_full[2], slot_last[2];
    for (uint32_t j = 0; j < 2; j += 1) {
        const uint32_t c = j == 0 ? c0 : c1;
        const uint32_t ni = (c + bm - 1u) / bm;
        nfull[j] = ni > 0 ? ni - 1u : 0u;
        last_cls[j] = ni > 0 ? (c - nfull[j] * bm + 15u) / 16u : 0u;
        slot_full[j] = nfull[j] > 0 ? atomicAdd(&cls_n[ncls - 1u], nfull[j]) : 0u;
        slot_last[j] = ni > 0 ? atomicAdd(&cls_n[last_cls[j] - 1u], 1u) : 0u;
    }
    const uint32_t ns = (a.shared_rows + bm - 1u) / bm;
    if (tid == 0 && ns > 0) {
        sh_slot[0] = ns > 1 ? atomicAdd(&cls_n[ncls - 1u], ns - 1u) : 0u;
        sh_slot[1] = atomicAdd(&cls_n[(a.shared_rows - (ns - 1u) * bm + 15u) / 16u - 1u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t base = 0;
        for (uint32_t c = ncls; c-- > 0;) {
            cls_b[c] = base;
            base += cls_n[c];
        }
        *n_out = base;
    }
    __syncthreads();
    uint4 *items = reinterpret_cast<uint4 *>(a.items);
    for (uint32_t j = 0; j < 2; j += 1) {
        const uint32_t e = e0 + j;
        const uint32_t c = j == 0 ? c0 : c1;
        const uint32_t o = j == 0 ? o0 : o1;
        for (uint32_t i = 0; i < nfull[j]; i += 1) {
            items[cls_b[ncls - 1u] + slot_full[j] + i] = make_uint4(e, o + i * bm, bm, 0u);
        }
        if (last_cls[j] > 0) {
            const uint32_t i = nfull[j];
            items[cls_b[last_cls[j] - 1u] + slot_last[j]] = make_uint4(e, o + i * bm, c - i * bm, 0u);
        }
    }
    if (ns > 0) {
        for (uint32_t i = tid; i + 1u < ns; i += NT) {
            items[cls_b[ncls - 1u] + sh_slot[0] + i] = make_uint4(E, a.shared_row0 + i * bm, bm, 0u);
        }
        if (tid == 0) {
            const uint32_t i = ns - 1u;
            const uint32_t rows = a.shared_rows - i * bm;
            items[cls_b[(rows + 15u) / 16u - 1u] + sh_slot[1]] = make_uint4(E, a.shared_row0 + i * bm, rows, 0u);
        }
    }
}

// count[e] = number of idx[0, npairs) equal to e, for up to
// RMDA_COUNT1_MAX_PAIRS pairs: one 1024-thread block, an LDS histogram, no
// hand-off between blocks.  Four 16-byte loads per thread in flight when idx
// is 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(1024) void count_kernel(const uint32_t *__restrict__ idx, uint32_t npairs,
                                                     uint32_t experts, uint32_t *__restrict__ count) {
    // CS copies of the histogram, lane l adding to copy l % CS (rows of CW
    // words, one spare so that the copies of one expert sit in different
    // banks): under skewed routing many lanes of a wave hold the same expert,
    // and the LDS serialises adds to one word
    constexpr uint32_t CS = 8;
    constexpr uint32_t CW = RMDA_MAX_EXPERTS + 1u;
    __shared__ uint32_t hc[CS * CW];
    const uint32_t tid = threadIdx.x;
    uint32_t *const h = hc + (tid % RMDA_WAVE % CS) * CW;
    for (uint32_t i = tid; i < CS * CW; i += 1024) {
        hc[i] = 0;
    }
    __syncthreads();
    uint32_t done = 0;
    if (VEC) {
        const uint4 *iv = reinterpret_cast<const uint4 *>(idx);
        const uint32_t n4 = npairs / 4;
        for (uint32_t i = tid; i < n4; i += 4 * 1024) {
            uint4 v[4];
#pragma unroll
            for (uint32_t u = 0; u < 4; u += 1) {
                const uint32_t j = i + u * 1024;
                v[u] = j < n4 ? iv[j] : make_uint4(RMDA_NONE, RMDA_NONE, RMDA_NONE, RMDA_NONE);
            }
#pragma unroll
            for (uint32_t u = 0; u < 4; u += 1) {
                const uint32_t q[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (uint32_t t = 0; t < 4; t += 1) {
                    if (q[t] < experts) {
                        atomicAdd(&h[q[t]], 1u);
                    }
                }
            }
        }
        done = 4 * n4;
    }
    for (uint32_t i = done + tid; i < npairs; i += 1024) {
        const uint32_t e = idx[i];
        if (e < experts) {
            atomicAdd(&h[e], 1u);
        }
    }
    __syncthreads();
    for (uint32_t e = tid; e < experts; e += 1024) {
        uint32_t n = 0;
#pragma unroll
        for (uint32_t c = 0; c < CS; c += 1) {
            n += hc[c * CW + e];
        }
        count[e] = n;
    }
}

}  // namespace

hipError_t rmda_launch_count(hipStream_t s, const uint32_t *idx, uint32_t npairs, uint32_t experts,
                             uint32_t *count) {
    if ((reinterpret_cast<uintptr_t>(idx) & 15u) == 0) {
        hipLaunchKernelGGL(count_kernel<true>, dim3(1), dim3(1024), 0, s, idx, npairs, experts, count);
    } else {
        hipLaunchKernelGGL(count_kernel<false>, dim3(1), dim3(1024), 0, s, idx, npairs, experts, count);
    }
    return hipGetLastError();
}

hipError_t rmda_launch_zero(hipStream_t s, uint32_t *p, size_t n, uint32_t value) {
    if (n == 0) {
        return hipSuccess;
    }
    size_t blocks = (n + NT0 - 1) / NT0;
    if (blocks > 1024) {
        blocks = 1024;
    }
    hipLaunchKernelGGL(zero_kernel, dim3((uint32_t)blocks), dim3(NT0), 0, s, p, n, value);
    return hipGetLastError();
}

hipError_t rmda_launch_scan(hipStream_t s, const uint32_t *count, uint32_t *off, uint32_t *tiles,
                            uint32_t n_tiles, uint32_t experts, uint32_t tile) {
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(512), 0, s, count, off, tiles, n_tiles, experts, tile);
    return hipGetLastError();
}

// the routed rank launch: one block per NTR / 64 rows routes; the last
// blocks to finish rank (rank_kernel, NV > 0)
template <uint32_t NTR>
void launch_routed(hipStream_t s, const rmda_rank_args_t *a, uint32_t nv) {
    const dim3 g1((a->route_rows + NTR / RMDA_WAVE - 1) / (NTR / RMDA_WAVE)), b1(NTR);
    if (nv <= 1) {
        hipLaunchKernelGGL((rank_kernel<NTR, 1>), g1, b1, 0, s, *a);
    } else if (nv <= 2) {
        hipLaunchKernelGGL((rank_kernel<NTR, 2>), g1, b1, 0, s, *a);
    } else if (nv <= 4) {
        hipLaunchKernelGGL((rank_kernel<NTR, 4>), g1, b1, 0, s, *a);
    } else {
        hipLaunchKernelGGL((rank_kernel<NTR, RMDA_MAX_EXPERTS / RMDA_WAVE>), g1, b1, 0, s, *a);
    }
}

hipError_t rmda_launch_rank(hipStream_t s, const rmda_rank_args_t *a) {
    uint32_t nb = (a->npairs + RMDA_RANK_BLOCK - 1) / RMDA_RANK_BLOCK;
    if (nb == 0) {
        nb = 1;  // one block still finalises (zero counts, empty work list)
    }
    // one block (up to 1024 pairs): 256 threads; several blocks: 1024, one
    // thread per pair, so each block ranks its pairs in one pass and spreads
    // the per-expert finishing work over four times the threads (BASELINE
    // config 5, 20 blocks over 512 experts: rank 15.5 -> 10.2 us; config 3
    // 7.6 -> 7.35 us; one block is 0.15 us slower with 1024)
    if (a->route_proj != nullptr) {
        // top-k folded in: one block per 8 rows (16 with several rank
        // blocks) routes, the last nb to finish rank (one rank block, decode:
        // 8-wave blocks took 7.16-7.19 us, 4-wave ones 7.45-7.65 and 16-wave
        // ones 8.8-9.1, their last block then routing as well as ranking the
        // most; several: 16-wave blocks, config 3 rank 15.4 -> 14.5 us,
        // config 5 25.4 -> 23.0 us against 8-wave ones).  Several rank blocks need
        // count_all (each counts every pair, so none waits for another's
        // totals) and write the permutation themselves.
        const bool multi_ok = a->count_all != 0 && a->slot != nullptr && a->npairs <= RMDA_RANK_ALL_MAX &&
                              (reinterpret_cast<uintptr_t>(a->idx) & 15u) == 0;
        if ((nb != 1 && !multi_ok) || a->experts > RMDA_MAX_EXPERTS || a->topk == 0 || a->done == nullptr ||
            a->route_idx != a->idx || (uint64_t)a->route_rows * a->topk != a->npairs) {
            return hipErrorInvalidValue;
        }
        const uint32_t nv = (a->experts + RMDA_WAVE - 1) / RMDA_WAVE;
        if (nb == 1) {
            launch_routed<512>(s, a, nv);
        } else {
            // several rank blocks rank faster with one thread per pair, as
            // the unrouted launch does
            launch_routed<1024>(s, a, nv);
        }
        return hipGetLastError();
    }
    if (nb > 1) {
        hipLaunchKernelGGL((rank_kernel<1024, 0>), dim3(nb), dim3(1024), 0, s, *a);
    } else {
        hipLaunchKernelGGL((rank_kernel<NT0, 0>), dim3(nb), dim3(NT0), 0, s, *a);
    }
    return hipGetLastError();
}
