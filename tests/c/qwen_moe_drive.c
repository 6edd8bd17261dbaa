/* A C caller of the library, shaped like the qwen.c forwarders a maintainer
 * adds (mda_qwen_moe_rec / mda_qwen_moe_pack / mda_qwen_moe_fused over a
 * minimal mda_qwen_t, as in the reference's src/qwen.c:770-907 call sites).
 * It builds a layer's inputs with the library's fill kernels (the same
 * streams as rmda_moe/configs.py), runs the fused layer on packed weights and
 * the stage-by-stage recording, both injecting into hyper-connection streams,
 * and writes h_fused then h_rec (rows x hc x d fp32) to the output file.
 *
 *   qwen_moe_drive OUT rows d experts topk inter shared hc hc_rank inj_stride seed
 *
 * Test infrastructure: tests/test_gpu_c_driver.py compares its output with
 * the same calls made through the Python binding. */
#include <stdbool.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "rmda_moe.h"

/* ---- the minimal host side of qwen.c that the forwarders touch ---- */
typedef struct {
    void *dev; /* device address a HIP build of the view carries */
    size_t sz;
} mda_vkc_buf_t;

typedef struct {
    bool fail; /* sticky failure flag (src/vkc.c:15-20) */
} mda_vkc_t;

typedef struct {
    uint32_t d, experts, topk, inter, shared, hc, hc_rank, hc_pad;
} mda_qwen_cfg_t;

typedef struct {
    mda_vkc_buf_t x; /* the chunk's fp32 activations */
    mda_vkc_buf_t t; /* hyper-connection injection logits */
} mda_qwen_scratch_t;

typedef struct {
    mda_vkc_t *c;
    mda_qwen_cfg_t cfg;
    mda_qwen_scratch_t sc;
    rmda_moe_ctx_t *moe;
    rmda_qwen_moe_t qm;
    void *ws;
    size_t ws_bytes;
    uint16_t *packed;
} mda_qwen_t;

/* ---- the forwarders ---- */
static void moe_ck(mda_qwen_t *q, int rc) {
    if (rc != RMDA_OK && q->c->fail == false) {
        fprintf(stderr, "rmda_moe: %s\n", rmda_moe_ctx_message(q->moe));
        q->c->fail = true;
    }
}

static void mda_qwen_moe_rec(mda_qwen_t *q, mda_vkc_buf_t *h, uint32_t rows) {
    moe_ck(q, rmda_qwen_moe_rec(&q->qm, (const float *)q->sc.x.dev, (const float *)q->sc.t.dev, (float *)h->dev,
                                NULL, rows));
}

static void mda_qwen_moe_pack(mda_qwen_t *q) {
    mda_qwen_cfg_t cfg = q->cfg;
    rmda_moe_shape_t s = {0, cfg.d, cfg.experts, cfg.topk, cfg.inter, cfg.shared};
    moe_ck(q, rmda_moe_pack_weights(q->moe, &s, q->qm.w_router, q->qm.w_gate_up, q->qm.w_down, q->qm.w_sh_gate_up,
                                    q->qm.w_sh_down, /*bf16=*/0, q->packed));
}

static void mda_qwen_moe_fused(mda_qwen_t *q, const uint16_t *x16, float *h, uint32_t rows) {
    mda_qwen_cfg_t cfg = q->cfg;
    rmda_moe_shape_t s = {rows, cfg.d, cfg.experts, cfg.topk, cfg.inter, cfg.shared};
    rmda_moe_layer_args_t a = {
        .x = x16, .w_router = q->qm.w_router, .bias = NULL,
        .out = NULL, .workspace = q->ws, .workspace_bytes = q->ws_bytes,
        .packed = q->packed,
        .h = h, .inj = (const float *)q->sc.t.dev, .inj_stride = cfg.hc_pad, .inj_off = cfg.hc_rank, .hc = cfg.hc,
    };
    moe_ck(q, rmda_moe_layer(q->moe, &s, &a));
}

/* ---- driver ---- */
#define CHECK_HIP(x)                                                                   \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            exit(2);                                                                   \
        }                                                                              \
    } while (0)

static void *dalloc(size_t bytes) {
    void *p = NULL;
    CHECK_HIP(hipMalloc(&p, bytes > 0 ? bytes : 16));
    return p;
}

static float h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t u;
    if (e == 0x1f) {
        u = s | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        u = s | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        u = s;
    } else {
        e = 113u;
        while ((m & 0x400u) == 0) {
            m <<= 1;
            e -= 1;
        }
        u = s | (e << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int main(int argc, char **argv) {
    if (argc != 12) {
        fprintf(stderr, "usage: %s OUT rows d experts topk inter shared hc hc_rank inj_stride seed\n", argv[0]);
        return 1;
    }
    const char *out_path = argv[1];
    const uint32_t rows = (uint32_t)strtoul(argv[2], NULL, 10);
    mda_qwen_cfg_t cfg = {0};
    cfg.d = (uint32_t)strtoul(argv[3], NULL, 10);
    cfg.experts = (uint32_t)strtoul(argv[4], NULL, 10);
    cfg.topk = (uint32_t)strtoul(argv[5], NULL, 10);
    cfg.inter = (uint32_t)strtoul(argv[6], NULL, 10);
    cfg.shared = (uint32_t)strtoul(argv[7], NULL, 10);
    cfg.hc = (uint32_t)strtoul(argv[8], NULL, 10);
    cfg.hc_rank = (uint32_t)strtoul(argv[9], NULL, 10);
    cfg.hc_pad = (uint32_t)strtoul(argv[10], NULL, 10);
    const uint64_t seed = strtoull(argv[11], NULL, 10);
    const size_t d = cfg.d, E = cfg.experts, I = cfg.inter, S = cfg.shared;
    const size_t cols = E + (S > 0 ? 1 : 0);

    mda_vkc_t vk = {false};
    mda_qwen_t q;
    memset(&q, 0, sizeof(q));
    q.c = &vk;
    q.cfg = cfg;
    if (rmda_moe_ctx_create(&q.moe, 0, NULL) != RMDA_OK) {
        fprintf(stderr, "rmda_moe_ctx_create failed\n");
        return 2;
    }
    /* weights and activations: the streams of rmda_moe/configs.py */
    uint16_t *x16 = dalloc(rows * d * 2);
    float *w_router = dalloc(cols * d * 4);
    uint16_t *w_gu = dalloc(E * 2 * I * d * 2);
    uint16_t *w_dn = dalloc(E * d * I * 2);
    uint16_t *w_sgu = S > 0 ? dalloc(2 * S * d * 2) : NULL;
    uint16_t *w_sdn = S > 0 ? dalloc(d * S * 2) : NULL;
    moe_ck(&q, rmda_moe_fill_normal_f16(q.moe, x16, rows * d, 1, seed, 1.0f));
    moe_ck(&q, rmda_moe_fill_normal_f32(q.moe, w_router, cols * d, 2, seed, 0.02f));
    moe_ck(&q, rmda_moe_fill_normal_f16(q.moe, w_gu, E * 2 * I * d, 3, seed, 0.02f));
    moe_ck(&q, rmda_moe_fill_normal_f16(q.moe, w_dn, E * d * I, 4, seed, 0.02f));
    if (S > 0) {
        moe_ck(&q, rmda_moe_fill_normal_f16(q.moe, w_sgu, 2 * S * d, 5, seed, 0.02f));
        moe_ck(&q, rmda_moe_fill_normal_f16(q.moe, w_sdn, d * S, 6, seed, 0.02f));
    }
    /* hyper-connection streams and injection logits: streams 11 and 12 */
    const size_t hn = rows * cfg.hc * d;
    float *h0 = dalloc(hn * 4);
    float *h_fused = dalloc(hn * 4);
    float *h_rec = dalloc(hn * 4);
    float *inj = dalloc(rows * cfg.hc_pad * 4);
    moe_ck(&q, rmda_moe_fill_normal_f32(q.moe, h0, hn, 11, seed, 1.0f));
    moe_ck(&q, rmda_moe_fill_normal_f32(q.moe, inj, rows * cfg.hc_pad, 12, seed, 3.0f));
    CHECK_HIP(hipDeviceSynchronize());
    CHECK_HIP(hipMemcpy(h_fused, h0, hn * 4, hipMemcpyDeviceToDevice));
    CHECK_HIP(hipMemcpy(h_rec, h0, hn * 4, hipMemcpyDeviceToDevice));
    /* the recording takes fp32 activations: the exact widening of x16 */
    uint16_t *xh = malloc(rows * d * 2);
    float *xf = malloc(rows * d * 4);
    CHECK_HIP(hipMemcpy(xh, x16, rows * d * 2, hipMemcpyDeviceToHost));
    for (size_t i = 0; i < rows * d; i += 1) {
        xf[i] = h2f(xh[i]);
    }
    float *x32 = dalloc(rows * d * 4);
    CHECK_HIP(hipMemcpy(x32, xf, rows * d * 4, hipMemcpyHostToDevice));
    q.sc.x.dev = x32;
    q.sc.x.sz = rows * d * 4;
    q.sc.t.dev = inj;
    q.sc.t.sz = rows * cfg.hc_pad * 4;

    /* load time: the recording's configuration and scratch, the packed
     * weights and the fused layer's workspace */
    q.qm.ctx = q.moe;
    q.qm.d = cfg.d;
    q.qm.experts = cfg.experts;
    q.qm.topk = cfg.topk;
    q.qm.inter = cfg.inter;
    q.qm.shared = cfg.shared;
    q.qm.hc = cfg.hc;
    q.qm.hc_rank = cfg.hc_rank;
    q.qm.inj_stride = cfg.hc_pad;
    q.qm.w_router = w_router;
    q.qm.w_gate_up = w_gu;
    q.qm.w_down = w_dn;
    q.qm.w_sh_gate_up = w_sgu;
    q.qm.w_sh_down = w_sdn;
    q.qm.max_rows = rows;
    q.qm.scratch_bytes = rmda_qwen_moe_scratch_bytes(&q.qm);
    q.qm.scratch = dalloc(q.qm.scratch_bytes);
    rmda_moe_shape_t s = {rows, cfg.d, cfg.experts, cfg.topk, cfg.inter, cfg.shared};
    q.ws_bytes = rmda_moe_workspace_bytes(&s);
    q.ws = dalloc(q.ws_bytes);
    q.packed = dalloc(rmda_moe_packed_bytes(&s));
    if (q.qm.scratch_bytes == 0 || q.ws_bytes == 0) {
        fprintf(stderr, "configuration rejected\n");
        return 2;
    }
    mda_qwen_moe_pack(&q);

    /* one chunk through each path (mda_vkc_begin .. mda_vkc_flush) */
    mda_qwen_moe_fused(&q, x16, h_fused, rows);
    mda_vkc_buf_t hb = {h_rec, hn * 4};
    mda_qwen_moe_rec(&q, &hb, rows);
    moe_ck(&q, rmda_moe_sync(q.moe));
    if (vk.fail) {
        return 3;
    }
    float *host = malloc(hn * 4);
    FILE *f = fopen(out_path, "wb");
    if (f == NULL) {
        perror(out_path);
        return 2;
    }
    CHECK_HIP(hipMemcpy(host, h_fused, hn * 4, hipMemcpyDeviceToHost));
    fwrite(host, 4, hn, f);
    CHECK_HIP(hipMemcpy(host, h_rec, hn * 4, hipMemcpyDeviceToHost));
    fwrite(host, 4, hn, f);
    fclose(f);
    printf("qwen_moe_drive: rows %u d %u experts %u topk %u inter %u shared %u: ok\n", rows, cfg.d, cfg.experts,
           cfg.topk, cfg.inter, cfg.shared);
    rmda_moe_ctx_destroy(q.moe);
    return 0;
}
