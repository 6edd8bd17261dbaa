/* The boundary's argument structs against the reference's push-constant
 * structs (src/pc.h:85-93,107-118,315-323,369-404): every struct the C-ABI
 * takes in place of an mda_pc_*_t has the same size, and each field the same
 * offset and type, so a qwen.c shim passes `&pc` through unchanged.
 * Compiled (not run) by tests/test_cpu_c_abi.py with gcc -std=c17 against
 * the reference tree's own header, when that tree is present. */
#include <stddef.h>

#include "pc.h"
#include "rmda_moe.h"

#define SAME_TYPE(a, b) _Generic((a), __typeof__(b): 1, default: 0)

/* mda_pc_moe_route_t */
_Static_assert(sizeof(rmda_pc_moe_route_t) == sizeof(mda_pc_moe_route_t), "moe_route: size");
_Static_assert(offsetof(rmda_pc_moe_route_t, rows) == offsetof(mda_pc_moe_route_t, rows), "moe_route.rows: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_route_t *)0)->rows, ((mda_pc_moe_route_t *)0)->rows), "moe_route.rows: type");
_Static_assert(offsetof(rmda_pc_moe_route_t, experts) == offsetof(mda_pc_moe_route_t, experts), "moe_route.experts: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_route_t *)0)->experts, ((mda_pc_moe_route_t *)0)->experts), "moe_route.experts: type");
_Static_assert(offsetof(rmda_pc_moe_route_t, topk) == offsetof(mda_pc_moe_route_t, topk), "moe_route.topk: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_route_t *)0)->topk, ((mda_pc_moe_route_t *)0)->topk), "moe_route.topk: type");
_Static_assert(offsetof(rmda_pc_moe_route_t, stride) == offsetof(mda_pc_moe_route_t, stride), "moe_route.stride: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_route_t *)0)->stride, ((mda_pc_moe_route_t *)0)->stride), "moe_route.stride: type");
/* mda_pc_moe_scan_t */
_Static_assert(sizeof(rmda_pc_moe_scan_t) == sizeof(mda_pc_moe_scan_t), "moe_scan: size");
_Static_assert(offsetof(rmda_pc_moe_scan_t, experts) == offsetof(mda_pc_moe_scan_t, experts), "moe_scan.experts: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_scan_t *)0)->experts, ((mda_pc_moe_scan_t *)0)->experts), "moe_scan.experts: type");
_Static_assert(offsetof(rmda_pc_moe_scan_t, tile) == offsetof(mda_pc_moe_scan_t, tile), "moe_scan.tile: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_scan_t *)0)->tile, ((mda_pc_moe_scan_t *)0)->tile), "moe_scan.tile: type");
/* mda_pc_moe_scatter_t */
_Static_assert(sizeof(rmda_pc_moe_scatter_t) == sizeof(mda_pc_moe_scatter_t), "moe_scatter: size");
_Static_assert(offsetof(rmda_pc_moe_scatter_t, rows) == offsetof(mda_pc_moe_scatter_t, rows), "moe_scatter.rows: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_scatter_t *)0)->rows, ((mda_pc_moe_scatter_t *)0)->rows), "moe_scatter.rows: type");
_Static_assert(offsetof(rmda_pc_moe_scatter_t, topk) == offsetof(mda_pc_moe_scatter_t, topk), "moe_scatter.topk: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_scatter_t *)0)->topk, ((mda_pc_moe_scatter_t *)0)->topk), "moe_scatter.topk: type");
_Static_assert(offsetof(rmda_pc_moe_scatter_t, d8) == offsetof(mda_pc_moe_scatter_t, d8), "moe_scatter.d8: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_scatter_t *)0)->d8, ((mda_pc_moe_scatter_t *)0)->d8), "moe_scatter.d8: type");
/* mda_pc_moe_mm_t */
_Static_assert(sizeof(rmda_pc_moe_mm_t) == sizeof(mda_pc_moe_mm_t), "moe_mm: size");
_Static_assert(offsetof(rmda_pc_moe_mm_t, m) == offsetof(mda_pc_moe_mm_t, m), "moe_mm.m: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_mm_t *)0)->m, ((mda_pc_moe_mm_t *)0)->m), "moe_mm.m: type");
_Static_assert(offsetof(rmda_pc_moe_mm_t, n) == offsetof(mda_pc_moe_mm_t, n), "moe_mm.n: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_mm_t *)0)->n, ((mda_pc_moe_mm_t *)0)->n), "moe_mm.n: type");
_Static_assert(offsetof(rmda_pc_moe_mm_t, k) == offsetof(mda_pc_moe_mm_t, k), "moe_mm.k: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_mm_t *)0)->k, ((mda_pc_moe_mm_t *)0)->k), "moe_mm.k: type");
_Static_assert(offsetof(rmda_pc_moe_mm_t, sa) == offsetof(mda_pc_moe_mm_t, sa), "moe_mm.sa: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_mm_t *)0)->sa, ((mda_pc_moe_mm_t *)0)->sa), "moe_mm.sa: type");
_Static_assert(offsetof(rmda_pc_moe_mm_t, sb) == offsetof(mda_pc_moe_mm_t, sb), "moe_mm.sb: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_mm_t *)0)->sb, ((mda_pc_moe_mm_t *)0)->sb), "moe_mm.sb: type");
/* mda_pc_moe_combine_t */
_Static_assert(sizeof(rmda_pc_moe_combine_t) == sizeof(mda_pc_moe_combine_t), "moe_combine: size");
_Static_assert(offsetof(rmda_pc_moe_combine_t, rows) == offsetof(mda_pc_moe_combine_t, rows), "moe_combine.rows: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_combine_t *)0)->rows, ((mda_pc_moe_combine_t *)0)->rows), "moe_combine.rows: type");
_Static_assert(offsetof(rmda_pc_moe_combine_t, d) == offsetof(mda_pc_moe_combine_t, d), "moe_combine.d: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_combine_t *)0)->d, ((mda_pc_moe_combine_t *)0)->d), "moe_combine.d: type");
_Static_assert(offsetof(rmda_pc_moe_combine_t, topk) == offsetof(mda_pc_moe_combine_t, topk), "moe_combine.topk: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_combine_t *)0)->topk, ((mda_pc_moe_combine_t *)0)->topk), "moe_combine.topk: type");
_Static_assert(offsetof(rmda_pc_moe_combine_t, pstride) == offsetof(mda_pc_moe_combine_t, pstride), "moe_combine.pstride: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_combine_t *)0)->pstride, ((mda_pc_moe_combine_t *)0)->pstride), "moe_combine.pstride: type");
_Static_assert(offsetof(rmda_pc_moe_combine_t, sg_off) == offsetof(mda_pc_moe_combine_t, sg_off), "moe_combine.sg_off: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_combine_t *)0)->sg_off, ((mda_pc_moe_combine_t *)0)->sg_off), "moe_combine.sg_off: type");
_Static_assert(offsetof(rmda_pc_moe_combine_t, inj_stride) == offsetof(mda_pc_moe_combine_t, inj_stride), "moe_combine.inj_stride: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_combine_t *)0)->inj_stride, ((mda_pc_moe_combine_t *)0)->inj_stride), "moe_combine.inj_stride: type");
_Static_assert(offsetof(rmda_pc_moe_combine_t, inj_off) == offsetof(mda_pc_moe_combine_t, inj_off), "moe_combine.inj_off: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_combine_t *)0)->inj_off, ((mda_pc_moe_combine_t *)0)->inj_off), "moe_combine.inj_off: type");
_Static_assert(offsetof(rmda_pc_moe_combine_t, hc) == offsetof(mda_pc_moe_combine_t, hc), "moe_combine.hc: offset");
_Static_assert(SAME_TYPE(((rmda_pc_moe_combine_t *)0)->hc, ((mda_pc_moe_combine_t *)0)->hc), "moe_combine.hc: type");
/* mda_pc_qwen_elem_t */
_Static_assert(sizeof(rmda_pc_qwen_elem_t) == sizeof(mda_pc_qwen_elem_t), "qwen_elem: size");
_Static_assert(offsetof(rmda_pc_qwen_elem_t, rows) == offsetof(mda_pc_qwen_elem_t, rows), "qwen_elem.rows: offset");
_Static_assert(SAME_TYPE(((rmda_pc_qwen_elem_t *)0)->rows, ((mda_pc_qwen_elem_t *)0)->rows), "qwen_elem.rows: type");
_Static_assert(offsetof(rmda_pc_qwen_elem_t, n) == offsetof(mda_pc_qwen_elem_t, n), "qwen_elem.n: offset");
_Static_assert(SAME_TYPE(((rmda_pc_qwen_elem_t *)0)->n, ((mda_pc_qwen_elem_t *)0)->n), "qwen_elem.n: type");
_Static_assert(offsetof(rmda_pc_qwen_elem_t, astride) == offsetof(mda_pc_qwen_elem_t, astride), "qwen_elem.astride: offset");
_Static_assert(SAME_TYPE(((rmda_pc_qwen_elem_t *)0)->astride, ((mda_pc_qwen_elem_t *)0)->astride), "qwen_elem.astride: type");
_Static_assert(offsetof(rmda_pc_qwen_elem_t, ao) == offsetof(mda_pc_qwen_elem_t, ao), "qwen_elem.ao: offset");
_Static_assert(SAME_TYPE(((rmda_pc_qwen_elem_t *)0)->ao, ((mda_pc_qwen_elem_t *)0)->ao), "qwen_elem.ao: type");
_Static_assert(offsetof(rmda_pc_qwen_elem_t, bo) == offsetof(mda_pc_qwen_elem_t, bo), "qwen_elem.bo: offset");
_Static_assert(SAME_TYPE(((rmda_pc_qwen_elem_t *)0)->bo, ((mda_pc_qwen_elem_t *)0)->bo), "qwen_elem.bo: type");
_Static_assert(offsetof(rmda_pc_qwen_elem_t, op) == offsetof(mda_pc_qwen_elem_t, op), "qwen_elem.op: offset");
_Static_assert(SAME_TYPE(((rmda_pc_qwen_elem_t *)0)->op, ((mda_pc_qwen_elem_t *)0)->op), "qwen_elem.op: type");
_Static_assert(offsetof(rmda_pc_qwen_elem_t, scale) == offsetof(mda_pc_qwen_elem_t, scale), "qwen_elem.scale: offset");
_Static_assert(SAME_TYPE(((rmda_pc_qwen_elem_t *)0)->scale, ((mda_pc_qwen_elem_t *)0)->scale), "qwen_elem.scale: type");
/* mda_pc_absmax_t */
_Static_assert(sizeof(rmda_pc_absmax_t) == sizeof(mda_pc_absmax_t), "absmax: size");
_Static_assert(offsetof(rmda_pc_absmax_t, n) == offsetof(mda_pc_absmax_t, n), "absmax.n: offset");
_Static_assert(SAME_TYPE(((rmda_pc_absmax_t *)0)->n, ((mda_pc_absmax_t *)0)->n), "absmax.n: type");
_Static_assert(offsetof(rmda_pc_absmax_t, slot) == offsetof(mda_pc_absmax_t, slot), "absmax.slot: offset");
_Static_assert(SAME_TYPE(((rmda_pc_absmax_t *)0)->slot, ((mda_pc_absmax_t *)0)->slot), "absmax.slot: type");
/* mda_pc_cast_t */
_Static_assert(sizeof(rmda_pc_cast_t) == sizeof(mda_pc_cast_t), "cast: size");
_Static_assert(offsetof(rmda_pc_cast_t, n) == offsetof(mda_pc_cast_t, n), "cast.n: offset");
_Static_assert(SAME_TYPE(((rmda_pc_cast_t *)0)->n, ((mda_pc_cast_t *)0)->n), "cast.n: type");
_Static_assert(offsetof(rmda_pc_cast_t, slot) == offsetof(mda_pc_cast_t, slot), "cast.slot: offset");
_Static_assert(SAME_TYPE(((rmda_pc_cast_t *)0)->slot, ((mda_pc_cast_t *)0)->slot), "cast.slot: type");
/* mda_pc_qwen_bf16_t */
_Static_assert(sizeof(rmda_pc_qwen_bf16_t) == sizeof(mda_pc_qwen_bf16_t), "qwen_bf16: size");
_Static_assert(offsetof(rmda_pc_qwen_bf16_t, n) == offsetof(mda_pc_qwen_bf16_t, n), "qwen_bf16.n: offset");
_Static_assert(SAME_TYPE(((rmda_pc_qwen_bf16_t *)0)->n, ((mda_pc_qwen_bf16_t *)0)->n), "qwen_bf16.n: type");

int rmda_abi_layout_checked;
