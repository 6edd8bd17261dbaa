// Scheduling and synchronisation helpers shared by the persistent grouped
// GEMM kernels (gemm2.hip: the weight-streaming tile; gemm_hot.hip: the
// compute tile for experts that receive many rows).  gfx950 only.
#pragma once

#include "common.h"

namespace rmda_gemm {

typedef __attribute__((address_space(3))) void lds_void_t;

// chunk swizzle of row r (BK/8 chunks per row): chunk c of row r sits in
// slot c ^ ((r >> 1) & (BK/8 - 1)).  Chosen by measurement on gfx950
// (SQ_LDS_BANK_CONFLICT over this kernel's exact fragment-read sequence):
// zero conflict cycles for BK 32 and 64, where the unswizzled layout loses
// 49% (BK 32) and 74% (BK 64) of LDS cycles to conflicts.  Depends only on
// r mod 16, so it is the same for a slab row and a tile row.
template <int BK>
__device__ __forceinline__ uint32_t swz(uint32_t r) {
    return (r >> 1) & (uint32_t)(BK / 8 - 1);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// all LDS reads of this wave done, then the workgroup barrier
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// wait until this wave's loads of the oldest pending stage have landed:
// `after` later stages (0 .. 4) of L loads each may stay in flight
template <int L>
__device__ __forceinline__ void wait_after(uint32_t after) {
    switch (after) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<L>(); break;
    case 2: wait_vm<2 * L>(); break;
    case 3: wait_vm<3 * L>(); break;
    default: wait_vm<4 * L>(); break;
    }
}

// `loads` is one of the four per-wave stage sizes (uniform per wave)
template <int LA, int LB_HI, int LB_LO>
__device__ __forceinline__ void wait_stage(bool live, bool b_hi, uint32_t after) {
    if (live) {
        if (b_hi) {
            wait_after<LA + LB_HI>(after);
        } else {
            wait_after<LA + LB_LO>(after);
        }
    } else {
        if (b_hi) {
            wait_after<LB_HI>(after);
        } else {
            wait_after<LB_LO>(after);
        }
    }
}

// Task schedule of a persistent launch: grid = 8 * S workgroups, workgroup b
// on XCD b % 8.  The work list comes sorted by rows, largest first.
//   * Item i goes to XCD snake(i / 8, i % 8, 8): the XCDs' shares balance,
//     and the N tiles of one item (which share A rows) meet in one L2.
//   * An XCD's tasks (its items in list order, N tiles innermost, so in
//     falling cost) are dealt to its S workgroups round by round.  Rounds
//     alternate direction so that pairs of rounds cancel; an odd number (>= 3)
//     of full rounds starts with three rounds whose positions add up to
//     3(S-1)/2 +- 1/2 for every workgroup.
__device__ __forceinline__ uint32_t snake(uint32_t round, uint32_t pos, uint32_t width) {
    return (round & 1u) != 0 ? width - 1u - pos : pos;
}

struct task_sched_t {
    uint32_t xcd, wg, S, ntiles, full, ntask;
    __device__ __forceinline__ task_sched_t(uint32_t n_items, uint32_t nt) {
        xcd = blockIdx.x % 8u;
        wg = blockIdx.x / 8u;
        S = gridDim.x / 8u;
        ntiles = nt;
        const uint32_t rounds = n_items / 8u;
        const uint32_t n_x = rounds + (snake(rounds, xcd, 8u) < n_items % 8u ? 1u : 0u);
        const uint32_t total = n_x * nt;
        full = total / S;
        ntask = full + (pos(full) < total % S ? 1u : 0u);
    }
    // this workgroup's position in round q
    __device__ __forceinline__ uint32_t pos(uint32_t q) const {
        if (q < 3u && full >= 3u && (full & 1u) != 0 && (S & 1u) == 0) {
            const uint32_t h = S / 2u;
            return q == 0u ? wg : q == 1u ? (wg + h) % S : (wg < h ? S - 2u - 2u * wg : 2u * S - 1u - 2u * wg);
        }
        return snake(q, wg, S);
    }
    // work-list item of this workgroup's q-th task, and its N tile
    __device__ __forceinline__ uint32_t item(uint32_t q, uint32_t &nt) const {
        const uint32_t t = q * S + pos(q);
        const uint32_t k = t / ntiles;
        nt = t - k * ntiles;
        return 8u * k + snake(k, xcd, 8u);
    }
};

// Contiguous schedule: round q's tasks [q*G, (q+1)*G) in list order (item
// major, N tile minor) are cut into eight runs of G/8, one per XCD, so the
// CUs of an XCD work on adjacent items, i.e. on the same expert's weight
// tiles and neighbouring row blocks, and share both through their L2.
struct chunk_sched_t {
    uint32_t G, pos, ntiles, ntask;
    __device__ __forceinline__ chunk_sched_t(uint32_t n_items, uint32_t nt) {
        G = gridDim.x;
        pos = (blockIdx.x % 8u) * (G / 8u) + blockIdx.x / 8u;
        ntiles = nt;
        const uint32_t total = n_items * nt;
        ntask = total / G + (pos < total % G ? 1u : 0u);
    }
    __device__ __forceinline__ uint32_t item(uint32_t q, uint32_t &nt) const {
        const uint32_t t = q * G + pos;
        const uint32_t k = t / ntiles;
        nt = t - k * ntiles;
        return k;
    }
};

typedef const __attribute__((address_space(4))) uint32_t *const_u32p;

// One SwiGLU output of the gate_up epilogue: fp16 into hp, or in the
// slot-scaled mode (SC, a template parameter of every GEMM kernel, so the
// default epilogue carries no test of it) fp32 into hp32 with its magnitude
// into the lane's running maximum over its tasks (rmda_wave_amax merges it at
// the kernel's end).
// Both tiles store through this, so they stay bitwise equal in either mode.
// NT: a non-temporal store, which keeps the outputs from displacing the
// gathered activation rows that the item's other N tiles read from L2 next.
// The streaming tile takes it (measured on MI355X: gate_up at config 3
// 150.4 -> 139.1 us, config 5 413.8 -> 383.9 us, the teacher's shape 603 ->
// 586 us); the compute tile does not (config 4: 109.3 -> 112.6 us, and its
// down GEMM then reads hp from HBM).
template <bool SC, bool NT>
__device__ __forceinline__ void swiglu_store(const rmda_gemm_args_t &g, uint16_t *O, size_t hi, float h,
                                             float &hmax) {
    if constexpr (SC) {
        if constexpr (NT) {
            __builtin_nontemporal_store(h, &g.hp32[hi]);
        } else {
            g.hp32[hi] = h;
        }
        hmax = fmaxf(hmax, fabsf(h));
    } else if constexpr (NT) {
        __builtin_nontemporal_store(rmda_f2h(h), &O[hi]);
    } else {
        O[hi] = rmda_f2h(h);
    }
}

// The down epilogue's multiplier: 1, or in the slot-scaled mode the inverse
// hp slot scale (fp32 rows) or rmda_ye_mul of the packed weights' bound
// (fp16 rows).
template <bool SC, int MODE>
__device__ __forceinline__ float down_mul(const rmda_gemm_args_t &g) {
    if constexpr (SC && MODE == RMDA_GEMM_F16) {
        return g.ye32 != nullptr ? rmda_slot_inv(g.yscale) : rmda_ye_mul(g.ye_bound);
    }
    return 1.0f;
}

// One output of the down epilogue, already multiplied by down_mul: fp16
// into ye (non-temporal with NT: a compile-time choice, since a runtime
// branch between two stores of the same value to the same address is
// folded into one plain store), or fp32 into ye32 in the slot-scaled mode's
// fp32-row variant.
template <bool SC, bool NT = false>
__device__ __forceinline__ void down_store(const rmda_gemm_args_t &g, uint16_t *O, size_t i, float y) {
    if (SC && g.ye32 != nullptr) {
        g.ye32[i] = y;
    } else if constexpr (NT) {
        __builtin_nontemporal_store(rmda_f2h(y), &O[i]);
    } else {
        O[i] = rmda_f2h(y);
    }
}

}  // namespace rmda_gemm
