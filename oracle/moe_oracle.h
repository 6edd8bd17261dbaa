/*
 * moe_oracle.h - CPU oracle for the MoE feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline; the product path (librmda_moe.so) never links or
 * calls it.
 *
 * A single-file C restatement of the reference's moe_* shader semantics
 * (shader/moe_route.comp, moe_scan.comp, moe_scatter.comp,
 * matmul_f16_moe.comp, moe_combine.comp, qwen_elem.comp, absmax.comp,
 * cast_f16.comp, qwen_bf16.comp) and of the orchestration in
 * src/qwen.c:770-907, generalised to any experts <= 512 and any padding.
 * The argument structs are the ones in include/rmda_moe.h (same layout as
 * src/pc.h).
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/rmda_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 <-> fp32, round to nearest even, subnormals kept, NaN quietened. */
float orc_h2f(uint16_t h);
uint16_t orc_f2h(float f);
void orc_h2f_n(const uint16_t *src, float *dst, size_t n);
void orc_f2h_n(const float *src, uint16_t *dst, size_t n);

/* Counter hash and the synthetic-input generator (same definition as the
 * library's rmda_moe_fill_normal_*). */
uint64_t orc_hash_u64(uint64_t stream, uint64_t key, uint64_t i);
float orc_normal(uint64_t stream, uint64_t key, uint64_t i, float std);
void orc_fill_normal_f16(uint16_t *dst, size_t n, uint64_t stream, uint64_t seed, float std);
void orc_fill_normal_f32(float *dst, size_t n, uint64_t stream, uint64_t seed, float std);

/* Router projection in the library's canonical fp32 order (8 contiguous
 * chunks of d, each a sequential fmaf chain from 0, chunk sums added left to
 * right, then the bias). */
void orc_router(const rmda_moe_router_t *pc, const uint16_t *x16, const float *w,
                const float *bias, float *proj, int threads);
/* orc_router with each chunk sum multiplied by post before the bias */
void orc_router_scaled(const rmda_moe_router_t *pc, const uint16_t *x16, const float *w,
                       const float *bias, float post, float *proj, int threads);

/* shader/moe_route.comp, generalised (only columns < experts are read). */
void orc_moe_route(const rmda_pc_moe_route_t *pc, const float *proj, uint32_t *idx,
                   float *wt, uint32_t *count);
/* shader/moe_scan.comp; tiles[0..n_tiles) fully written (RMDA_NONE = unused). */
void orc_moe_scan(const rmda_pc_moe_scan_t *pc, const uint32_t *count, uint32_t *off,
                  uint32_t *tiles, uint32_t n_tiles);
/* shader/moe_scatter.comp run sequentially in pr order: the canonical stable
 * permutation.  fill is in/out like the reference (caller zeroes it). */
void orc_moe_scatter(const rmda_pc_moe_scatter_t *pc, const uint32_t *idx,
                     const uint32_t *off, uint32_t *fill, const uint16_t *x16,
                     uint16_t *xp, uint32_t *slot);
/* shader/matmul_f16_moe.comp: per 128-row tile, fixed-order fp32 accumulate. */
void orc_moe_mm(const rmda_pc_moe_mm_t *pc, const uint16_t *a, const uint16_t *b,
                float *c, const uint32_t *amax, const uint32_t *tiles, int threads);
/* shader/moe_combine.comp (sh may be NULL: no shared term). */
void orc_moe_combine(const rmda_pc_moe_combine_t *pc, const float *wt, const uint32_t *slot,
                     const float *y, const float *proj, const float *sh, const float *inj,
                     float *h);
void orc_moe_combine_plain(const rmda_pc_moe_combine_t *pc, const float *wt,
                           const uint32_t *slot, const float *y, const float *proj,
                           const float *sh, float *out);
/* shader/qwen_elem.comp, absmax.comp, cast_f16.comp, qwen_bf16.comp */
void orc_qwen_elem(const rmda_pc_qwen_elem_t *pc, const float *a, float *y);
void orc_absmax(const rmda_pc_absmax_t *pc, const float *x, uint32_t *amax);
void orc_cast_f16(const rmda_pc_cast_t *pc, const float *src, uint16_t *dst, const uint32_t *amax);
float orc_slot_scale(const uint32_t *amax, uint32_t slot);
void orc_qwen_bf16(const rmda_pc_qwen_bf16_t *pc, uint32_t *w);

/* The whole layer in the reference's order (src/qwen.c:838-907), plain
 * output mode (out[r,c] = combine accumulator, fp32).
 *   tile:       segment padding P (128 = reference, 1 = compact)
 *   hp_scale:   1 = absmax + power-of-two fp16 cast of hp and the shared hs
 *               as the reference does (src/qwen.c:858-877), 0 = plain fp16 cast
 *   x_scale:    1 = absmax + cast of x before the GEMMs (src/qwen.c:844), 0 = none
 *   rows_sel:   if non-NULL, only these n_sel tokens get an output row
 *               (routing, scan and permutation still cover every token; the
 *               expert GEMMs run only for the selected tokens' pairs); out is
 *               then n_sel x d.
 * Intermediates (each may be NULL): proj [rows][proj_stride], idx, wt, slot
 * [rows*topk], count, off [experts].  Returns 0, or -1 on a bad shape. */
typedef struct orc_layer_t {
    rmda_moe_shape_t shape;
    uint32_t tile;
    int hp_scale;
    int x_scale;
    int threads;
    const uint16_t *x;
    const float *w_router;
    const float *bias;
    const uint16_t *w_gate_up;
    const uint16_t *w_down;
    const uint16_t *w_sh_gate_up;
    const uint16_t *w_sh_down;
    const uint32_t *rows_sel;
    uint32_t n_sel;
    float *out;
    float *proj;
    uint32_t *idx;
    float *wt;
    uint32_t *slot;
    uint32_t *count;
    uint32_t *off;
    /* nonzero: round every expert output row (ye) to fp16 before the
     * combine, as the fused GPU layer stores it (the reference keeps fp32) */
    int ye16;
    /* or NULL: wall-clock ms of the layer's stages, in the order
     * router, route, scan, scatter, gate_up (+SwiGLU, cast), down, shared
     * expert, combine (ORC_LAYER_STAGES) */
    double *stage_ms;
    /* or NULL: fp32 activations in place of x (x may then be NULL), cast to
     * fp16 with a slot scale for the router and the GEMMs as the reference
     * casts its fp32 chunk (src/qwen.c:517-539, :844); the router divides the
     * scale out before the bias */
    const float *x32;
} orc_layer_t;
#define ORC_LAYER_STAGES 8

int orc_moe_layer(const orc_layer_t *L);
uint32_t orc_proj_stride(const rmda_moe_shape_t *s);

#ifdef __cplusplus
}
#endif

#endif
