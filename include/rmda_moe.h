/*
 * rmda_moe.h - C ABI of the MI355X (gfx950) MoE feed-forward path.
 *
 * This library replaces the Vulkan dispatch of R-MDA's MoE teacher layer
 * (reference: src/qwen.c:770-907 issuing mda_vkc_run, src/vkc.c:771-789) with
 * hand-written HIP kernels.  Every entry point is plain C: device pointers,
 * sizes and the reference's own argument structs (field for field the
 * push-constant structs of src/pc.h), no C++ or torch types.
 *
 * Conventions shared by every entry point
 *   - Pointers are device pointers (hipMalloc'd or equivalent) unless stated.
 *   - Calls are enqueue-only on the context's stream; nothing reads results
 *     back to the host, so no device->host synchronisation happens inside a
 *     call (the reference's layer is one GPU-resident command buffer,
 *     src/qwen.c:1074-1076).  rmda_moe_sync() is the "flush".
 *   - Return value: RMDA_OK (0) or a negative RMDA_ERR_* code.  The first
 *     failure is also kept as a sticky error in the context and every later
 *     call returns RMDA_ERR_STICKY without enqueueing work, mirroring the
 *     reference's sticky c->fail (src/vkc.c:15-20, :771-789).  Nothing calls
 *     exit().
 *   - One context = one host thread at a time (the reference records from a
 *     single thread, src/qwen.c:1069-1078).
 *   - Hot calls never allocate device memory.  The context owns a small
 *     fixed-capacity scratch area allocated once in rmda_moe_ctx_create();
 *     the fused layer uses a caller-provided workspace.
 */
#ifndef RMDA_MOE_H
#define RMDA_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version of this header's binary interface.  It changes whenever a struct
 * the caller passes in or the library fills grows or changes layout (no
 * counterpart in the reference, which links its kernels statically).  A
 * caller checks rmda_moe_abi_version() == RMDA_MOE_ABI_VERSION once at load
 * time; on a mismatch it was built against another header and must be
 * rebuilt, since the library may read or write past its structs.
 *   1  the first release;
 *   2  rmda_moe_ws_layout_t gained items / n_items / n_items_hot and
 *      rmda_qwen_moe_layout_t gained hp / hp16 / tiles;
 *   3  rmda_moe_layer_args_t gained x32 (fp32 activations with a slot
 *      scale). */
#define RMDA_MOE_ABI_VERSION 3

/* Same value as MDA_PC_NO_SLOT (src/pc.h:6): "no fp16 scale slot". */
#define RMDA_NO_SLOT 0xffffffffu
/* Sentinel for an unused tile / a pair with no selectable expert. */
#define RMDA_NONE 0xffffffffu

/* Reference limits kept by the drop-in kernels. */
#define RMDA_MAX_EXPERTS 512u /* moe_scan runs 512 lanes, shader/moe_scan.comp:2 */
#define RMDA_MAX_TOPK 16u     /* MAXK, shader/moe_route.comp:18 */
#define RMDA_MM_TILE 128u     /* TILE, shader/matmul_f16_moe.comp:16; MDA_QWEN_TILE src/qwen.h:14 */

/* Scratch capacity of a context: routed pairs (rows * topk) per call of
 * rmda_moe_scatter.  Larger calls fail with RMDA_ERR_CAPACITY. */
#define RMDA_CTX_MAX_PAIRS (1u << 21)

enum {
    RMDA_OK = 0,
    RMDA_ERR_ARG = -1,       /* null pointer or invalid flag */
    RMDA_ERR_SHAPE = -2,     /* shape violates a kernel's requirement */
    RMDA_ERR_CAPACITY = -3,  /* beyond a documented maximum */
    RMDA_ERR_HIP = -4,       /* a HIP runtime call failed */
    RMDA_ERR_STICKY = -5,    /* an earlier call failed; context is poisoned */
    RMDA_ERR_WORKSPACE = -6, /* caller workspace missing or too small */
    RMDA_ERR_DEVICE = -7     /* no usable gfx950 device */
};

/* ---- argument structs: identical layout to the reference push constants ---- */

/* src/pc.h:369-374 */
typedef struct rmda_pc_moe_route_t {
    uint32_t rows;
    uint32_t experts;
    uint32_t topk;
    uint32_t stride;
} rmda_pc_moe_route_t;

/* src/pc.h:376-379 */
typedef struct rmda_pc_moe_scan_t {
    uint32_t experts;
    uint32_t tile;
} rmda_pc_moe_scan_t;

/* src/pc.h:381-385 */
typedef struct rmda_pc_moe_scatter_t {
    uint32_t rows;
    uint32_t topk;
    uint32_t d8;
} rmda_pc_moe_scatter_t;

/* src/pc.h:387-393 */
typedef struct rmda_pc_moe_mm_t {
    uint32_t m;
    uint32_t n;
    uint32_t k;
    uint32_t sa;
    uint32_t sb;
} rmda_pc_moe_mm_t;

/* src/pc.h:395-404 */
typedef struct rmda_pc_moe_combine_t {
    uint32_t rows;
    uint32_t d;
    uint32_t topk;
    uint32_t pstride;
    uint32_t sg_off;
    uint32_t inj_stride;
    uint32_t inj_off;
    uint32_t hc;
} rmda_pc_moe_combine_t;

/* src/pc.h:315-323 */
typedef struct rmda_pc_qwen_elem_t {
    uint32_t rows;
    uint32_t n;
    uint32_t astride;
    uint32_t ao;
    uint32_t bo;
    uint32_t op;
    float scale;
} rmda_pc_qwen_elem_t;

/* src/pc.h:85-88 */
typedef struct rmda_pc_absmax_t {
    uint32_t n;
    uint32_t slot;
} rmda_pc_absmax_t;

/* src/pc.h:90-93 */
typedef struct rmda_pc_cast_t {
    uint32_t n;
    uint32_t slot;
} rmda_pc_cast_t;

/* shader/qwen_bf16.comp:5-7 */
typedef struct rmda_pc_qwen_bf16_t {
    uint32_t n;
} rmda_pc_qwen_bf16_t;

/* ---- context ---- */

typedef struct rmda_moe_ctx rmda_moe_ctx_t;

/* Create a context on HIP device `device` issuing work on `stream`
 * (a hipStream_t; NULL = the device's null stream).  Allocates the context's
 * fixed scratch.  Fails with RMDA_ERR_DEVICE unless the device is gfx950. */
int rmda_moe_ctx_create(rmda_moe_ctx_t **out, int device, void *stream);
void rmda_moe_ctx_destroy(rmda_moe_ctx_t *ctx);
int rmda_moe_set_stream(rmda_moe_ctx_t *ctx, void *stream);
/* Load buckets of the fused layer's grouped GEMMs (no counterpart in the
 * reference, whose matmul_f16_moe has one 128 x 128 tile): an expert that
 * receives at least `rows` rows in a call is hot, and when hot experts (and
 * the shared expert, if it has that many rows) hold at least half of the
 * call's rows, both GEMMs run the compute tile (256-row items, 8 waves of
 * 128 x 64) instead of the weight-streaming tile (192-row items).  Either
 * tile gives bitwise the same output.  Packed weights only; 0 disables the
 * compute tile; the default is 256. */
int rmda_moe_set_hot_rows(rmda_moe_ctx_t *ctx, uint32_t rows);
/* Which grouped-GEMM tile launches (no counterpart in the reference).  The
 * choice is made on the device, from the call's routing, after the host has
 * enqueued the GEMM launches, so:
 *   RMDA_TILE_AUTO      launches both tiles every call; the one whose list
 *                       the rank kernel left empty exits at once (about
 *                       4 us per launch on MI355X);
 *   RMDA_TILE_ADAPTIVE  (default) launches only the tile that the
 *                       context's previous call on the same packed weights
 *                       and row count chose (the rank kernel reports its
 *                       choice to a host-visible word of a 64-entry table
 *                       keyed by those two) and makes the rank kernel cut
 *                       its list for that tile; the first call of a key
 *                       (and of a key whose entry another key took since),
 *                       and every call after rmda_moe_set_hot_rows or this
 *                       function, runs as AUTO until its choice lands;
 *   RMDA_TILE_STREAM / RMDA_TILE_HOT  always that tile.
 * Every policy gives bitwise the same output; calls with rows < hot rows
 * (no expert can be hot) and HF-layout weights launch the streaming tile
 * only. */
enum { RMDA_TILE_ADAPTIVE = 0, RMDA_TILE_AUTO = 1, RMDA_TILE_STREAM = 2, RMDA_TILE_HOT = 3 };
int rmda_moe_set_tile_policy(rmda_moe_ctx_t *ctx, int policy);
/* Route inside the rank launch for calls of more than one rank block of
 * 1024 (token, expert) pairs, up to 65536 pairs: the
 * launches before gate_up are then the router and one rank launch, in which
 * one workgroup per 16 tokens selects the top-k as moe_route does
 * (shader/moe_route.comp:20-61, dispatched at src/qwen.c:799-811) and the
 * workgroups that finish last rank the pairs, after a device-scope
 * release/acquire ticket.  Off by default: slower on MI355X (config 3 layer
 * 292.5 -> 293.9 us, config 5 794.2 -> 797.8 us), because every rank block
 * then reads all pairs' experts, written on other XCDs, through device-scope
 * loads, which costs more than the kernel boundary it replaces (route + rank
 * 9.7 us, the routed rank 14.2 us at config 3).  Calls of one rank block
 * (decode sizes) always route in the rank launch.  Every setting gives
 * bitwise the same results. */
int rmda_moe_set_route_in_rank(rmda_moe_ctx_t *ctx, int on);
/* Fold the combine into the down GEMM (replaces moe_combine's own dispatch,
 * src/qwen.c:887-906, inside rmda_moe_layer; off by default).  Each down-GEMM
 * wave that stores the last of a token's rows for 64 output columns sums
 * them there, in j order, exactly as the combine kernel does, so the output
 * is bitwise the same; the fused layer then launches no combine kernel when
 * the streaming tile runs.  Packed weights only (otherwise ignored).
 * Slower on MI355X (layer 0.296 -> 0.346 ms): the rows
 * must be stored through to the device coherence point and counted with
 * device-scope atomics, because a token's rows are stored on several XCDs. */
int rmda_moe_set_fused_combine(rmda_moe_ctx_t *ctx, int on);
/* Sticky error: RMDA_OK or the first failure's code, with a message. */
int rmda_moe_ctx_error(const rmda_moe_ctx_t *ctx);
const char *rmda_moe_ctx_message(const rmda_moe_ctx_t *ctx);
void rmda_moe_ctx_clear_error(rmda_moe_ctx_t *ctx);
/* Wait for all enqueued work: the replacement of mda_vkc_flush
 * (src/vkc.c:655-668).  Reports asynchronous HIP errors. */
int rmda_moe_sync(rmda_moe_ctx_t *ctx);
/* Library version string and the gfx target it was built for. */
const char *rmda_moe_version(void);
/* RMDA_MOE_ABI_VERSION of the header the library was built with. */
int rmda_moe_abi_version(void);

/* ---- per-stage drop-ins (one per reference kernel, buffers in binding order) ---- */

/* moe_route (shader/moe_route.comp; dispatched at src/qwen.c:799-811).
 * For each row r: top `topk` of proj[r*stride + 0..experts) by value,
 * descending, ties to the lower expert index, NaN and values <= -3e38 never
 * selected; idx[r*topk+j] = expert, wt[r*topk+j] = exp(l_j - l_0) / sum_j.
 * count[e] = number of (r, j) that selected e.  Unlike the reference, count is
 * overwritten (the reference adds into a buffer the host zero-filled first,
 * src/qwen.c:794).  A pair with no selectable expert gets idx RMDA_NONE and is
 * not counted (the reference indexes count[~0u] there).
 * Requires experts <= 512, 1 <= topk <= min(16, experts), stride >= experts. */
int rmda_moe_route(rmda_moe_ctx_t *ctx, const rmda_pc_moe_route_t *pc,
                   const float *proj, uint32_t *idx, float *wt, uint32_t *count);

/* moe_scan (shader/moe_scan.comp; src/qwen.c:812-821).
 * off[e] = sum_{e'<e} ceil(count[e']/tile)*tile; tiles[t] = e for each of
 * expert e's tiles and RMDA_NONE for every other t < n_tiles (the reference
 * relies on a host fill for those, src/qwen.c:796; n_tiles is that fill's
 * length, mrows/tile).  Requires experts <= 512, tile >= 1. */
int rmda_moe_scan(rmda_moe_ctx_t *ctx, const rmda_pc_moe_scan_t *pc,
                  const uint32_t *count, uint32_t *off, uint32_t *tiles, uint32_t n_tiles);

/* moe_scatter (shader/moe_scatter.comp; src/qwen.c:822-835).
 * slot[pr] = off[e] + (number of pr' < pr with idx[pr'] == e), e = idx[pr]:
 * the stable order the reference's atomic counter produces when run
 * sequentially, here produced deterministically.  Row pr/topk of x16
 * (d8 16-byte chunks) is copied bitwise to row slot[pr] of xp.  Pairs with
 * idx RMDA_NONE get slot RMDA_NONE and copy nothing.  `fill` is scratch of
 * `experts` words: treated as zero on entry, left holding the per-expert
 * counts (what the reference's atomics leave there).  Rows of xp that no pair
 * targets are not written: a caller that runs rmda_moe_mm on xp next must
 * zero-fill xp first, as the reference does (src/qwen.c:798), because
 * rmda_moe_mm computes every row of each tile the map names, the segments'
 * padding rows included.
 * `experts` is taken from the context's last rmda_moe_route call unless set
 * with rmda_moe_scatter_experts().  Requires rows*topk <= RMDA_CTX_MAX_PAIRS
 * and 16-byte aligned x16 and xp. */
int rmda_moe_scatter(rmda_moe_ctx_t *ctx, const rmda_pc_moe_scatter_t *pc,
                     const uint32_t *idx, const uint32_t *off, uint32_t *fill,
                     const uint16_t *x16, uint16_t *xp, uint32_t *slot);
int rmda_moe_scatter_experts(rmda_moe_ctx_t *ctx, uint32_t experts);

/* matmul_f16_moe (shader/matmul_f16_moe.comp; src/qwen.c:770-786).
 * For each 128-row tile t of A with e = tiles[t] != RMDA_NONE:
 * C[r, 0..n) = (A[r, :] . B[e][0..n)[:]) / (scale(sa) * scale(sb)) for the
 * 128 rows r of the tile; fp16 inputs, fp32 accumulate, fp32 output.
 * B is [experts][n][k] fp16 (HF [out, in] per expert).  Rows of tiles marked
 * RMDA_NONE are not written.  amax holds the fp16 scale slots (may be NULL if
 * sa == sb == RMDA_NO_SLOT).  Requires m % 128 == 0, n % 128 == 0,
 * k % 32 == 0 (the reference's grid and K-step) and 16-byte aligned a, b, c. */
int rmda_moe_mm(rmda_moe_ctx_t *ctx, const rmda_pc_moe_mm_t *pc,
                const uint16_t *a, const uint16_t *b, float *c,
                const uint32_t *amax, const uint32_t *tiles);

/* moe_combine (shader/moe_combine.comp; src/qwen.c:887-906).
 * acc[r,c] = sum_j wt[r,j] * y[slot[r,j], c]
 *          + sigmoid(proj[r*pstride + sg_off]) * sh[r*d + c];
 * h[r, s, c] += acc * 2 * sigmoid(inj[r*inj_stride + inj_off + s] / hc), s < hc.
 * Extension: sh == NULL drops the shared-expert term (proj unused then);
 * pairs with slot RMDA_NONE contribute nothing. */
int rmda_moe_combine(rmda_moe_ctx_t *ctx, const rmda_pc_moe_combine_t *pc,
                     const float *wt, const uint32_t *slot, const float *y,
                     const float *proj, const float *sh, const float *inj, float *h);

/* Plain-output combine (no hyper-connection streams): out[r,c] = acc as fp16.
 * Same acc as rmda_moe_combine. */
int rmda_moe_combine_plain(rmda_moe_ctx_t *ctx, const rmda_pc_moe_combine_t *pc,
                           const float *wt, const uint32_t *slot, const float *y,
                           const float *proj, const float *sh, uint16_t *out);

/* qwen_elem (shader/qwen_elem.comp; used at src/qwen.c:848-857, :879-884).
 * op 0: y[r*n+c] = silu(a[r*astride+ao+c]) * a[r*astride+bo+c];
 * op 1: y[r*n+c] = silu(a[r*astride+ao+c] * scale); silu(v) = v/(1+exp(-v)). */
int rmda_qwen_elem(rmda_moe_ctx_t *ctx, const rmda_pc_qwen_elem_t *pc,
                   const float *a, float *y);

/* absmax (shader/absmax.comp): amax[slot] = max(amax[slot], max_i |x[i]|) on
 * the float bit patterns (values are non-negative). */
int rmda_absmax(rmda_moe_ctx_t *ctx, const rmda_pc_absmax_t *pc,
                const float *x, uint32_t *amax);

/* cast_f16 (shader/cast_f16.comp): dst[i] = fp16(src[i] * scale(slot)),
 * scale = 2^(141 - biased_exponent(amax[slot])), 1 for RMDA_NO_SLOT or a
 * zero / non-finite amax.  Round to nearest even. */
int rmda_cast_f16(rmda_moe_ctx_t *ctx, const rmda_pc_cast_t *pc,
                  const float *src, uint16_t *dst, const uint32_t *amax);

/* qwen_bf16 (shader/qwen_bf16.comp; src/qwen.c:386-390): in place, each
 * 32-bit word holding two bf16 becomes two fp16 (round to nearest even). */
int rmda_qwen_bf16(rmda_moe_ctx_t *ctx, const rmda_pc_qwen_bf16_t *pc, uint32_t *w);

/* ---- router projection (replaces the dense fp16 GEMM into `p`, src/qwen.c:845) ---- */

/* proj[r*stride + c] = x16[r, :] . w[c, :] for c < cols, plus bias[c] for
 * c < nbias when bias != NULL.  x16 is rows x d fp16, w is cols x d fp32
 * (HF [out, in]: rows 0..E-1 the router, row E the shared-expert gate when
 * present, as in the reference's packed p layout, src/qwen.c:444-449).
 * fp32 arithmetic in one fixed order that the CPU oracle replays exactly:
 * d is cut into 8 contiguous chunks; each chunk is a sequential fmaf chain
 * from 0; the chunk sums are added left to right; then the bias.
 * Requires d % 128 == 0 and 1 <= cols <= stride, cols <= 65536. */
typedef struct rmda_moe_router_t {
    uint32_t rows;
    uint32_t d;
    uint32_t cols;
    uint32_t stride;
    uint32_t nbias;
} rmda_moe_router_t;

int rmda_moe_router(rmda_moe_ctx_t *ctx, const rmda_moe_router_t *pc,
                    const uint16_t *x16, const float *w, const float *bias, float *proj);

/* The router on a slot-scaled cast, as src/qwen.c:844-845 feeds it
 * (mda_qwen_mm(q, sx, ...) on the cast mda_qwen_cast made with slot sx):
 * x16 is x cast by rmda_cast_f16 with slot `slot` of amax, and each chunk
 * sum is multiplied by the inverse of that slot's power-of-two scale before
 * the bias is added.  For activations in fp16's normal range the logits
 * equal rmda_moe_router's on the unscaled cast bit for bit; outside it
 * (subnormal, or beyond 65504) they keep the precision of the scaled cast.
 * slot == RMDA_NO_SLOT is rmda_moe_router.  Same requirements. */
int rmda_moe_router_slot(rmda_moe_ctx_t *ctx, const rmda_moe_router_t *pc, const uint16_t *x16, uint32_t slot,
                         const uint32_t *amax, const float *w, const float *bias, float *proj);

/* ---- fused MoE layer (replaces mda_qwen_moe_rec, src/qwen.c:838-907) ---- */

typedef struct rmda_moe_shape_t {
    uint32_t rows;    /* tokens T in this call */
    uint32_t d;       /* hidden size */
    uint32_t experts; /* routed experts E */
    uint32_t topk;    /* k */
    uint32_t inter;   /* routed expert intermediate size I */
    uint32_t shared;  /* shared expert intermediate size I_s, 0 = none */
} rmda_moe_shape_t;

/* Alignment: x, the weights, packed, out, h and workspace must be 16-byte
 * aligned, bias and inj 4-byte aligned (RMDA_ERR_ARG otherwise), like the
 * reference's storage-buffer offsets. */
typedef struct rmda_moe_layer_args_t {
    const uint16_t *x;          /* rows x d fp16 activations, or NULL when x32 is given */
    const float *w_router;      /* (experts [+1 shared gate]) x d fp32 */
    const float *bias;          /* experts fp32 router bias, or NULL */
    const uint16_t *w_gate_up;  /* [experts][2*inter][d] fp16: gate rows then up rows */
    const uint16_t *w_down;     /* [experts][d][inter] fp16 */
    const uint16_t *w_sh_gate_up; /* [2*shared][d] fp16 or NULL when shared == 0 */
    const uint16_t *w_sh_down;    /* [d][shared] fp16 or NULL when shared == 0 */
    uint16_t *out;              /* rows x d fp16 */
    void *workspace;            /* >= rmda_moe_workspace_bytes(shape) bytes */
    size_t workspace_bytes;
    const uint16_t *packed;     /* weights from rmda_moe_pack_weights, or NULL: then
                                   the kernels read w_router / w_gate_up / w_down /
                                   w_sh_* (the HF tensors above are ignored when set) */
    /* Hyper-connection epilogue (src/qwen.c:887-906, shader/moe_combine.comp:36-38):
     * with h != NULL the layer output y (fp32, before any rounding) is injected
     * into hc residual streams in place,
     *   h[r][s][c] += y[r][c] * 2 * sigmoid(inj[r*inj_stride + inj_off + s] / hc), s < hc,
     * and `out` may be NULL (it is written only when given). */
    float *h;                   /* rows x hc x d fp32, or NULL */
    const float *inj;           /* rows x inj_stride fp32 injection logits */
    uint32_t inj_stride;
    uint32_t inj_off;
    uint32_t hc;                /* 1 .. 8 streams (the reference uses 4) */
    /* fp32 activations (the chunk's sc->x, src/qwen.c:844), in place of x
     * (exactly one of the two is given).  The layer then runs the reference's
     * fp16 scale-slot protocol (src/qwen.c:500-539): x's absmax goes into a
     * fresh slot and x is cast to fp16 times 2^(141 - exponent(absmax))
     * (absmax.comp, cast_f16.comp), which the router and gate_up divide out;
     * the SwiGLU output is kept in fp32 and cast with a slot of its own
     * (src/qwen.c:858-877), which down divides out.  Down's rows (fp32 in
     * the reference, src/qwen.c:878) stay fp32 up to the combine with
     * HF-layout weights; with packed weights they are stored as fp16 times
     * 2^-c, where 2^c exceeds the down weights' largest row sum of |w| (a
     * bound the packing computes), so that no row can overflow, and the
     * combine multiplies the power of two back.  So activations far outside
     * fp16's range (say 1e-6 or 1e6) route and multiply as in the reference.
     * For inputs that are fp16 values in fp16's normal range the routing is
     * bitwise that of x = those values.  Needs rmda_moe_workspace_bytes_x32
     * of workspace; the combine is never folded into down in this mode. */
    const float *x32;
} rmda_moe_layer_args_t;

/* Device views into the workspace after rmda_moe_layer (byte offsets), so a
 * caller can inspect routing: proj [rows][proj_stride] fp32, idx/wt/slot
 * [rows*topk], count/off [experts]. */
typedef struct rmda_moe_ws_layout_t {
    size_t proj;
    size_t idx;
    size_t wt;
    size_t count;
    size_t off;
    size_t slot;
    size_t total;
    uint32_t proj_stride;
    /* grouped-GEMM work list: items uint4 {group, first sorted row, rows, 0};
     * n_items counts the weight-streaming tile's items (up to 192 rows),
     * n_items_hot the compute tile's (up to 256 rows); one of the two is 0 */
    size_t items;
    size_t n_items;
    size_t n_items_hot;
} rmda_moe_ws_layout_t;

size_t rmda_moe_workspace_bytes(const rmda_moe_shape_t *shape);
/* Workspace of rmda_moe_layer with args->x32 set: the scaled fp16 copy of x
 * and the fp32 SwiGLU output / expert rows in place of the fp16 expert rows
 * (config 3: 188.1 MB against 104.7 MB). */
size_t rmda_moe_workspace_bytes_x32(const rmda_moe_shape_t *shape);
int rmda_moe_workspace_layout(const rmda_moe_shape_t *shape, rmda_moe_ws_layout_t *out);

/* The whole layer: router -> route -> scan -> permutation -> grouped SwiGLU
 * gate_up GEMM -> grouped down GEMM -> (shared expert) -> combine, enqueued on
 * the context stream with no host synchronisation.
 * out[r] = sum_j wt[r,j] * FFN_{idx[r,j]}(x[r]) (+ sigmoid(g_r) * FFN_shared(x[r])).
 * Expert segments are padded to multiples of 16 rows (off[] is
 * rmda_moe_scan with tile 16, so the activations between the two GEMMs are
 * stored in whole 16-row blocks); the permutation is the stable order of
 * rmda_moe_scatter over those offsets.  Requires d % 256 == 0,
 * inter % 128 == 0, shared == 0 or shared == inter, experts <= 512,
 * topk <= 16. */
int rmda_moe_layer(rmda_moe_ctx_t *ctx, const rmda_moe_shape_t *shape,
                   const rmda_moe_layer_args_t *args);

/* Allocation-free variant of rmda_moe_layer.  It has no counterpart in the
 * reference (whose recording always runs on caller-allocated scratch): it is
 * for callers that cannot allocate, such as code under HIP graph capture or a
 * serving loop that forbids hipMalloc.  Same arguments and results as
 * rmda_moe_layer, except that args->workspace must be NULL and
 * args->workspace_bytes 0: the workspace is the library's static device array
 * of RMDA_STATIC_WS_BYTES, one per device, reserved when the code object is
 * loaded and held until the process ends.  Shapes whose
 * rmda_moe_workspace_bytes (with x32: rmda_moe_workspace_bytes_x32) exceeds
 * it fail with RMDA_ERR_CAPACITY (config 3, T=2048 x d=2048 x 128 experts
 * top-8, needs 104.7 MB, and 188.1 MB with x32).  The call allocates
 * nothing and enqueues only kernels (the rank ticket it needs zeroed is
 * cleared by the router kernel).  Every call on a device shares that device's
 * array and leaves its contents behind, so calls that overlap on one device
 * (two streams, or two contexts, in flight at once) race. */
#define RMDA_STATIC_WS_BYTES ((size_t)128 << 20)
int rmda_moe_layer_static(rmda_moe_ctx_t *ctx, const rmda_moe_shape_t *shape, const rmda_moe_layer_args_t *args);

/* ---- expert-weight packing (replaces the per-layer weight conversion at
 * upload, src/qwen.c:376-394: qwen_bf16 converts the bf16 expert weights to
 * fp16 in place after each layer's upload) ---- */

/* Bytes of one layer's packed weights: routed gate_up and down, the shared
 * expert's gate_up and down when shape->shared > 0 (fp16, same element
 * count as the HF tensors), then the fp32 router matrix (experts [+1 shared
 * gate] rows, padded to a multiple of 64), then 256 bytes whose first word
 * is the down weights' largest row sum of |w| (fp32; rows whose sum is not
 * finite left out), for the x32 mode's fp16 expert rows.  0 when the shape
 * is rejected. */
size_t rmda_moe_packed_bytes(const rmda_moe_shape_t *shape);

/* Reorder one layer's HF-layout weights (w_router [E (+1)][d] fp32,
 * w_gate_up [E][2I][d], w_down [E][d][I], and w_sh_gate_up [2I_s][d],
 * w_sh_down [d][I_s] when shared > 0) into the order the kernels stream
 * them.  Each 256-row x K-step expert-weight slab becomes one contiguous
 * block in exactly the layout the grouped GEMM keeps it in LDS, so every
 * weight load is a contiguous KiB; the router matrix becomes
 * [d/16][cols rounded up to 64][4][4], element (k, c) at
 * ((k/16)*cpad + c)*16 + (k%4)*4 + (k%16)/4, so that one wave's load of a
 * 16-column MFMA tile for 16 k is a contiguous KiB.  With bf16 != 0 the expert weights are bf16 and are converted to
 * fp16 (round to nearest even) on the way, in place of qwen_bf16; the router
 * matrix is copied exactly.  Enqueued on the context stream; `packed` must
 * hold rmda_moe_packed_bytes(shape) bytes and must not overlap the inputs.
 * All pointers 16-byte aligned (RMDA_ERR_ARG otherwise).
 * A packed buffer is valid for contexts of the same library build. */
int rmda_moe_pack_weights(rmda_moe_ctx_t *ctx, const rmda_moe_shape_t *shape, const float *w_router,
                          const uint16_t *w_gate_up, const uint16_t *w_down, const uint16_t *w_sh_gate_up,
                          const uint16_t *w_sh_down, int bf16, uint16_t *packed);

/* ---- safetensors weights (replaces src/safet.c: mda_safet_read, _tensor,
 * _open_set, _find, :29-63,147-163,236-275) ---- */

typedef struct rmda_st rmda_st_t;

enum {
    RMDA_ST_BF16 = 0,
    RMDA_ST_F16 = 1,
    RMDA_ST_F32 = 2,
    RMDA_ST_I64 = 3,
    RMDA_ST_I32 = 4,
    RMDA_ST_U8 = 5,
    RMDA_ST_OTHER = 15 /* indexed, but no element size is known */
};
#define RMDA_ST_MAX_DIMS 4

typedef struct rmda_st_tensor_t {
    const void *data; /* host pointer into the mapped file */
    uint64_t bytes;
    uint32_t dtype;   /* RMDA_ST_* */
    uint32_t ndim;
    uint64_t shape[RMDA_ST_MAX_DIMS];
    uint32_t file;    /* shard index */
} rmda_st_tensor_t;

/* Map a .safetensors file, or a directory holding model.safetensors.index.json
 * (every shard its weight_map names) or model.safetensors, and index the
 * headers.  Offsets are checked against the data section and dtype x shape.
 * Returns RMDA_OK or RMDA_ERR_ARG; rmda_st_message() says why (per thread). */
int rmda_st_open(const char *path, rmda_st_t **out);
void rmda_st_close(rmda_st_t *st);
const char *rmda_st_message(void);
uint32_t rmda_st_count(const rmda_st_t *st);
const char *rmda_st_name(const rmda_st_t *st, uint32_t i);
/* RMDA_ERR_ARG when no shard holds `name` (the reference's "missing"). */
int rmda_st_find(const rmda_st_t *st, const char *name, rmda_st_tensor_t *out);

/* ---- per-layer weight upload (replaces the staging banks, upload and
 * qwen_bf16 conversion of src/qwen.c:228-247,366-394,441-452,1101-1134) ----
 *
 * Reads one layer's MoE tensors from `st`, named `prefix` + (the reference's
 * names, src/qwen.c:441-452):
 *   gate.weight                  [E][d]        bf16/f32 -> fp32 router rows
 *   shared_expert_gate.weight    [1][d]        (shared > 0) router row E
 *   experts.gate_up_proj         [E][2I][d]    bf16/f16 (or [E*2I][d])
 *   experts.down_proj            [E][d][I]     bf16/f16 (or [E*d][I])
 *   shared_expert.gate_proj.weight, .up_proj.weight [I_s][d], .down_proj.weight [d][I_s]
 * e.g. prefix "model.language_model.layers.7.mlp.".  The bytes go from the
 * mapped file into one of two pinned host staging banks, then with one
 * asynchronous copy to device staging and through the pack kernels into
 * `packed` (rmda_moe_packed_bytes(shape) bytes), all on the context's upload
 * stream, so uploading layer l+1 overlaps computing layer l.  The call
 * returns once the host copy is done and the device work is enqueued; a bank
 * is reused only after its previous upload has finished.  Staging grows to
 * the largest layer seen (this call may allocate; rmda_moe_layer never
 * does).  Requires the same shape rules as rmda_moe_layer. */
int rmda_moe_upload_layer(rmda_moe_ctx_t *ctx, const rmda_st_t *st, const char *prefix,
                          const rmda_moe_shape_t *shape, uint16_t *packed);
/* Make the context's compute stream wait for every upload enqueued so far
 * (no host blocking). */
int rmda_moe_upload_wait(rmda_moe_ctx_t *ctx);

/* ---- stage profiler (replaces the reference's timestamp profiler:
 * mda_vkc_prof_begin / mda_vkc_prof_mark / mda_vkc_prof_report,
 * src/vkc.c:580-653, which writes a timestamp after every dispatch) ---- */

/* Stages of rmda_moe_layer, in launch order. */
enum {
    RMDA_STAGE_ROUTER = 0,  /* router projection (fp32 logits)           */
    RMDA_STAGE_ROUTE = 1,   /* top-k gating                              */
    RMDA_STAGE_RANK = 2,    /* counts, offsets, stable ranks, work list  */
    RMDA_STAGE_PERMUTE = 3, /* slots + sorted-row -> token map           */
    RMDA_STAGE_GATE_UP = 4, /* grouped gate_up GEMM with SwiGLU epilogue */
    RMDA_STAGE_DOWN = 5,    /* grouped down GEMM                         */
    RMDA_STAGE_COMBINE = 6, /* weighted gather-sum (+ shared expert)     */
    RMDA_PROF_STAGES = 7
};

/* Start accumulating per-stage GPU time of every later rmda_moe_layer call:
 * a hipEvent is recorded on the context stream before the first stage and
 * after each stage (created once, here; never in the layer call).  Every
 * RMDA_PROF_RING layer calls the events are harvested, which waits for the
 * stream: profiled runs are for measurement only. */
#define RMDA_PROF_RING 64u
int rmda_moe_prof_begin(rmda_moe_ctx_t *ctx);
/* Stop, wait for the stream, and return the summed milliseconds per stage
 * (ms[RMDA_PROF_STAGES]) and the number of layer calls they cover. */
int rmda_moe_prof_end(rmda_moe_ctx_t *ctx, double *ms, uint32_t *layers);
/* Summed length (ms) of an empty interval per profiled call since
 * rmda_moe_prof_begin: two events recorded back to back on the stream, i.e.
 * what one stage boundary costs by itself; subtract it from a stage's
 * per-call average for the stage's own time.  A stage whose launch a call
 * skipped (the top-k fused into the router, the permutation written by the
 * rank kernel) adds no time and no event for that call. */
int rmda_moe_prof_empty_ms(rmda_moe_ctx_t *ctx, double *ms);
/* Name of stage i ("router", "route", ...), or NULL. */
const char *rmda_moe_prof_stage_name(uint32_t i);

/* ---- synthetic inputs (bench and tests) ---- */

/* dst[i] = fp16 / fp32 of std * z_i where z_i is the standardised
 * Irwin-Hall(4) variate of counter hash (stream, seed, i): exact integer and
 * IEEE float steps only, so any host reproduces it bit for bit. */
int rmda_moe_fill_normal_f16(rmda_moe_ctx_t *ctx, uint16_t *dst, size_t n,
                             uint64_t stream, uint64_t seed, float std);
int rmda_moe_fill_normal_f32(rmda_moe_ctx_t *ctx, float *dst, size_t n,
                             uint64_t stream, uint64_t seed, float std);

/* ---- the qwen.c MoE recording (src/qwen.c:770-907) over the stage entry
 * points ----
 * The reference records a layer's MoE with three functions on its
 * mda_qwen_t: mda_qwen_moe_mm (:770-786), mda_qwen_route_rec (:788-836) and
 * mda_qwen_moe_rec (:838-907), with its scratch buffers and fp16 scale
 * slots (:500-539) kept in mda_qwen_t.  These are the same three over
 * device pointers, with that state gathered in rmda_qwen_moe_t, so that a
 * qwen.c keeps its signatures and forwards to them.  They run the
 * reference's sequence stage by stage (128-row segments, scaled fp16 casts,
 * fp32 GEMM outputs); rmda_moe_layer is the fused fast path.
 * Differences, as for the stage entry points: the router is the fp32
 * rmda_moe_router on the slot-scaled cast of x, each chunk sum multiplied
 * by the slot's inverse scale (its p holds the experts' logits and, with a
 * shared expert, the shared gate in column `experts`; the shared gate/up
 * projections come from w_sh_gate_up through rmda_moe_mm instead of from
 * further p columns).  All functions are enqueue-only, return a status and
 * leave it sticky in ctx; nothing is allocated. */
#define RMDA_QWEN_TILE 128u       /* MDA_QWEN_TILE, src/qwen.h:14 */
#define RMDA_QWEN_MAX_SLOTS 16u   /* fp16 scale slots per chunk */

typedef struct rmda_qwen_moe_t {
    rmda_moe_ctx_t *ctx;
    /* the mda_qwen_cfg_t fields the MoE uses */
    uint32_t d;
    uint32_t experts;
    uint32_t topk;
    uint32_t inter;
    uint32_t shared;            /* 0 or the shared expert's intermediate size */
    /* hyper-connection streams of the combine (MDA_QWEN_HC, cfg.hc_rank,
     * MDA_QWEN_HC_PAD in the reference) */
    uint32_t hc;
    uint32_t hc_rank;
    uint32_t inj_stride;
    /* device weights */
    const float *w_router;        /* [experts (+1 shared gate)][d] fp32 */
    const uint16_t *w_gate_up;    /* [experts][2*inter][d] fp16 */
    const uint16_t *w_down;       /* [experts][d][inter] fp16 */
    const uint16_t *w_sh_gate_up; /* [2*shared][d] fp16, or NULL */
    const uint16_t *w_sh_down;    /* [d][shared] fp16, or NULL */
    /* device scratch of rmda_qwen_moe_scratch_bytes(q) bytes, laid out for
     * chunks of up to max_rows rows (mda_qwen_scratch, src/qwen.c:149-185) */
    uint32_t max_rows;
    void *scratch;
    size_t scratch_bytes;
    uint32_t n_slots;             /* scale slots taken in the current chunk */
} rmda_qwen_moe_t;

/* Device views into the scratch (byte offsets), for callers and tests:
 * p [rows][p_stride] fp32, idx/wt/slot [rows*topk], count/off [experts],
 * xp [mrows][d] fp16, amax [RMDA_QWEN_MAX_SLOTS], hp [mrows][inter] fp32
 * (the SwiGLU output) and hp16 [mrows][inter] fp16 (its scaled cast; after
 * rmda_qwen_moe_rec only their rows that hold routed pairs are defined),
 * tiles [mrows / 128] (the 128-row tile map). */
typedef struct rmda_qwen_moe_layout_t {
    size_t p;
    size_t idx;
    size_t wt;
    size_t count;
    size_t off;
    size_t slot;
    size_t xp;
    size_t amax;
    size_t total;
    uint32_t p_stride;
    /* added after the fields above, which keep their offsets */
    size_t hp;
    size_t hp16;
    size_t tiles;
} rmda_qwen_moe_layout_t;

/* Scratch bytes for q's configuration and max_rows (0 when rejected). */
size_t rmda_qwen_moe_scratch_bytes(const rmda_qwen_moe_t *q);
int rmda_qwen_moe_layout(const rmda_qwen_moe_t *q, rmda_qwen_moe_layout_t *out);

/* mda_qwen_moe_mm: C = A . W[e]^T / (scale(sa)), 128-row tiles mapped to
 * experts by the tile map route_rec left in the scratch. */
int rmda_qwen_moe_mm(rmda_qwen_moe_t *q, const uint16_t *a, uint32_t sa, const uint16_t *w, float *out,
                     uint32_t m, uint32_t n, uint32_t k);

/* mda_qwen_route_rec: top-k of the scratch's p, 128-row segment offsets and
 * tile map, and the scatter of the scaled activations into xp (whose rows
 * are zero-filled first, src/qwen.c:793-798).  mrows = rows*topk +
 * experts*127 rounded up to 128 (mda_qwen_moe_rows, src/qwen.c:68-70). */
int rmda_qwen_route_rec(rmda_qwen_moe_t *q, uint32_t rows, uint32_t mrows);

/* mda_qwen_moe_rec for one chunk of `rows` tokens of fp32 activations x
 * [rows][d]: scale slots reset, x cast with a slot, router, route_rec,
 * gate_up, SwiGLU, hp cast with a slot, down, the shared expert, combine.
 * With h != NULL the combine injects into the hyper-connection streams,
 * h[r][s][c] += y * 2 * sigmoid(inj[r*inj_stride + hc_rank + s] / hc)
 * (shader/moe_combine.comp:36-38); with out != NULL it writes y as fp16. */
int rmda_qwen_moe_rec(rmda_qwen_moe_t *q, const float *x, const float *inj, float *h, uint16_t *out,
                      uint32_t rows);

#ifdef __cplusplus
}
#endif

#endif
