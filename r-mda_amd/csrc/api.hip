// C ABI of the MoE path: context, sticky errors, argument checks, the
// per-stage drop-ins and the fused layer driver.  Replaces, for this path
// only, the reference's Vulkan dispatch (mda_vkc_run, src/vkc.c:771-789) and
// the recording in mda_qwen_moe_rec / mda_qwen_route_rec / mda_qwen_moe_mm
// (src/qwen.c:770-907).  Every call only enqueues work on the context stream.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <thread>
#include <vector>

#include "common.h"

constexpr uint32_t kHintSlots = 64;

struct rmda_moe_ctx {
    int device;
    hipStream_t stream;
    int err;
    char msg[256];
    // fixed scratch for rmda_moe_scatter (allocated once at creation)
    uint32_t *fixed_ws;
    // this device's copy of the allocation-free layer's `scratch` array
    void *static_ws;
    uint32_t *lrank;
    uint32_t *hist;
    uint32_t *done;
    uint32_t scatter_experts;
    // grouped-GEMM configuration (RMDA_MOE_GEMM_VARIANT overrides; tuning only)
    rmda_gemm2_cfg_t g2;
    // compute tile for hot experts: rows that make an expert hot (0 = never
    // use the tile) and its pipeline depth (RMDA_MOE_HOT_MIN and
    // RMDA_MOE_HOT_STAGES override; tuning only)
    uint32_t hot_min;
    int hot_stages;
    int hot_sched;
    // tile policy (RMDA_TILE_*; RMDA_MOE_TILE_POLICY overrides, tuning only)
    // and the words the rank kernel reports its tile choice to (pinned host
    // memory, mapped into the device): one per (packed weights, rows) key in
    // a small direct-mapped table, so that a context serving many layers
    // reads each layer's own last choice
    int tile_policy;
    uint32_t *tile_hint_host;  // [kHintSlots]
    uint32_t *tile_hint_dev;
    const void *hint_key_w[kHintSlots];
    uint32_t hint_key_rows[kHintSlots];
    // combine folded into the down GEMM (rmda_moe_set_fused_combine;
    // RMDA_MOE_FUSED_COMBINE sets the initial value)
    int fused_combine;
    // top-k folded into the rank launch above one rank block
    // (rmda_moe_set_route_in_rank; RMDA_MOE_ROUTE_IN_RANK sets the initial
    // value); one rank block always routes in the rank launch
    int route_rank;
    // stage profiler: a ring of per-call event sets, harvested when full
    int prof_on;
    int prof_made;
    uint32_t prof_pending;
    uint32_t prof_layers;
    double prof_ms[RMDA_PROF_STAGES];
    double prof_empty_ms;  // summed length of one empty interval per call
    // per call: events opening the call and closing each stage, then one more
    // recorded right after the opening one (an empty interval); a stage whose
    // launch the call skipped records no event (bit st of prof_skip)
    hipEvent_t prof_ev[RMDA_PROF_RING][RMDA_PROF_STAGES + 2];
    uint32_t prof_skip[RMDA_PROF_RING];
    // weight upload: a stream of its own and two staging banks (pinned host +
    // device), created at the first upload
    int up_made;
    hipStream_t up_stream;
    uint32_t up_seq;
    size_t up_cap;  // bytes per bank
    uint8_t *up_host[2];
    uint8_t *up_dev[2];
    hipEvent_t up_done[2];  // bank b's last upload (copy + pack) finished
    hipEvent_t up_after;    // the compute stream's work queued before an upload's pack
    int up_used[2];
};

// Workspace of the allocation-free layer (rmda_moe_layer_static): one copy
// on every device the library runs on, held until the process ends.  Host
// code never uses this name as an address: rmda_moe_ctx_create looks up the
// device's copy with hipGetSymbolAddress (once per device) and every use goes
// through that pointer.
static __device__ __align__(256) uint8_t scratch[RMDA_STATIC_WS_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_static_mu;
void *g_static_ws[kMaxDevices];  // per device: the address of its `scratch`

constexpr size_t kHistBlocks = (RMDA_CTX_MAX_PAIRS + RMDA_RANK_BLOCK - 1) / RMDA_RANK_BLOCK;

int fail(rmda_moe_ctx_t *c, int code, const char *fmt, ...) {
    if (c != nullptr && c->err == RMDA_OK) {
        c->err = code;
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(c->msg, sizeof(c->msg), fmt, ap);
        va_end(ap);
    }
    return code;
}

// Entry guard: null context, sticky error, and the context's device current.
int enter(rmda_moe_ctx_t *c) {
    if (c == nullptr) {
        return RMDA_ERR_ARG;
    }
    if (c->err != RMDA_OK) {
        return RMDA_ERR_STICKY;
    }
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != c->device) {
        if (hipSetDevice(c->device) != hipSuccess) {
            return fail(c, RMDA_ERR_HIP, "hipSetDevice(%d) failed", c->device);
        }
    }
    return RMDA_OK;
}

int hip_check(rmda_moe_ctx_t *c, hipError_t e, const char *what) {
    if (e != hipSuccess) {
        return fail(c, RMDA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    }
    return RMDA_OK;
}

// true when p (NULL allowed) is a multiple of a bytes: the kernels' 16-byte
// vector loads and LDS DMA need 16-byte aligned rows
bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

size_t align256(size_t x) {
    return (x + 255) & ~(size_t)255;
}

// Tile-choice hints of RMDA_TILE_ADAPTIVE: forget every key and choice.
void hint_clear(rmda_moe_ctx_t *c) {
    for (uint32_t i = 0; i < kHintSlots; i += 1) {
        c->hint_key_w[i] = nullptr;
        c->hint_key_rows[i] = 0;
        __atomic_store_n(&c->tile_hint_host[i], 0u, __ATOMIC_RELAXED);
    }
}

// The hint slot of a call on weights w with `rows` tokens, and the tile the
// last call with the same key chose (1 streaming, 2 compute), or 0 when the
// slot held another key (then claimed for this one) or no choice has landed
// yet.  A kernel of the slot's previous key still in flight may store its
// choice after the claim; that costs one call the other tile, never a
// different result (both tiles give the same bits).
uint32_t hint_lookup(rmda_moe_ctx_t *c, const void *w, uint32_t rows, uint32_t *slot) {
    const uint64_t h = ((uint64_t)reinterpret_cast<uintptr_t>(w) >> 8) * 0x9E3779B97F4A7C15ull ^
                       (uint64_t)rows * 0xC2B2AE3D27D4EB4Full;
    const uint32_t i = (uint32_t)(h >> 58) % kHintSlots;
    *slot = i;
    if (c->hint_key_w[i] == w && c->hint_key_rows[i] == rows) {
        const uint32_t v = __atomic_load_n(&c->tile_hint_host[i], __ATOMIC_RELAXED);
        return v == 1u || v == 2u ? v : 0u;
    }
    c->hint_key_w[i] = w;
    c->hint_key_rows[i] = rows;
    __atomic_store_n(&c->tile_hint_host[i], 0u, __ATOMIC_RELAXED);
    return 0u;
}

const char *const kStageNames[RMDA_PROF_STAGES] = {"router", "route", "rank", "permute",
                                                   "gate_up", "down", "combine"};

// Wait for the last recorded event set and fold every pending call's stage
// intervals into the running sums (mda_vkc_prof_collect, src/vkc.c:617-628).
int prof_harvest(rmda_moe_ctx_t *c) {
    if (c->prof_pending == 0) {
        return RMDA_OK;
    }
    // the last event the last pending call recorded (a skipped final stage,
    // e.g. a combine folded into the down GEMM, records none)
    const uint32_t lp = c->prof_pending - 1;
    uint32_t ev_last = RMDA_PROF_STAGES + 1;
    for (uint32_t st = RMDA_PROF_STAGES; st-- > 0;) {
        if (((c->prof_skip[lp] >> st) & 1u) == 0) {
            ev_last = st + 1;
            break;
        }
    }
    int rc = hip_check(c, hipEventSynchronize(c->prof_ev[lp][ev_last]), "profiler hipEventSynchronize");
    for (uint32_t i = 0; i < c->prof_pending && rc == RMDA_OK; i += 1) {
        float ms = 0.0f;
        rc = hip_check(c, hipEventElapsedTime(&ms, c->prof_ev[i][0], c->prof_ev[i][RMDA_PROF_STAGES + 1]),
                       "profiler hipEventElapsedTime");
        c->prof_empty_ms += ms;
        hipEvent_t prev = c->prof_ev[i][RMDA_PROF_STAGES + 1];
        for (uint32_t st = 0; st < RMDA_PROF_STAGES && rc == RMDA_OK; st += 1) {
            if ((c->prof_skip[i] >> st) & 1u) {
                continue;  // no launch, no event: the next stage's interval starts at `prev`
            }
            rc = hip_check(c, hipEventElapsedTime(&ms, prev, c->prof_ev[i][st + 1]), "profiler hipEventElapsedTime");
            c->prof_ms[st] += ms;
            prev = c->prof_ev[i][st + 1];
        }
    }
    c->prof_layers += c->prof_pending;
    c->prof_pending = 0;
    return rc;
}

// Record the event that closes stage `st - 1` (st = 0 opens the call and
// records the empty interval right after).
int prof_mark(rmda_moe_ctx_t *c, uint32_t st) {
    if (!c->prof_on) {
        return RMDA_OK;
    }
    int rc = hip_check(c, hipEventRecord(c->prof_ev[c->prof_pending][st], c->stream), "profiler hipEventRecord");
    if (st == 0) {
        c->prof_skip[c->prof_pending] = 0;
        if (rc == RMDA_OK) {
            rc = hip_check(c, hipEventRecord(c->prof_ev[c->prof_pending][RMDA_PROF_STAGES + 1], c->stream),
                           "profiler hipEventRecord");
        }
    }
    return rc;
}

// Stage `st` launched nothing in this call: it records no event and adds no time.
void prof_skip(rmda_moe_ctx_t *c, uint32_t st) {
    if (c->prof_on) {
        c->prof_skip[c->prof_pending] |= 1u << st;
    }
}

struct LayerPlan {
    size_t proj, idx, wt, lrank, slot, rowtok, count, off, hist, done, n_items, n_items_hot, items, hp, fc_cnt, xs16,
        xpart, xslot, hslot, hparts, ye, total;
    uint32_t ps, npairs, nblocks, max_items, sh_rows, sh_row0, groups_rows;
};

int check_shape(const rmda_moe_shape_t *s, char *why, size_t n) {
    if (s->d == 0 || s->d % 256 != 0) {
        snprintf(why, n, "d=%u must be a positive multiple of 256", s->d);
        return 0;
    }
    if (s->experts == 0 || s->experts > RMDA_MAX_EXPERTS) {
        snprintf(why, n, "experts=%u must be in 1..%u", s->experts, RMDA_MAX_EXPERTS);
        return 0;
    }
    if (s->topk == 0 || s->topk > RMDA_MAX_TOPK || s->topk > s->experts) {
        snprintf(why, n, "topk=%u must be in 1..min(%u, experts)", s->topk, RMDA_MAX_TOPK);
        return 0;
    }
    if (s->inter == 0 || s->inter % 128 != 0) {
        snprintf(why, n, "inter=%u must be a positive multiple of 128", s->inter);
        return 0;
    }
    if (s->shared != 0 && s->shared != s->inter) {
        snprintf(why, n, "shared=%u must be 0 or equal to inter=%u", s->shared, s->inter);
        return 0;
    }
    if ((uint64_t)s->rows * s->topk + s->rows >= (1ull << 31)) {
        snprintf(why, n, "rows*topk too large");
        return 0;
    }
    return 1;
}

// x32: the slot-scaled mode (fp32 activations): the scaled fp16 copy of x,
// the absmax parts and two slot words, and a last region that holds first
// the fp32 SwiGLU output (hp32) and then the expert rows (fp16 scaled by the
// packed weights' bound, or fp32 ye32 for HF-layout weights), where the
// default mode's is the fp16 ye.  Every offset but that of the last region's
// end is the same in both modes.
LayerPlan plan_layer(const rmda_moe_shape_t *s, bool x32 = false) {
    LayerPlan p{};
    const uint32_t T = s->rows;
    const uint32_t K = s->topk;
    const uint32_t E = s->experts;
    p.ps = E + (s->shared > 0 ? 1u : 0u);
    p.npairs = T * K;
    p.nblocks = p.npairs == 0 ? 1 : (p.npairs + RMDA_RANK_BLOCK - 1) / RMDA_RANK_BLOCK;
    p.sh_rows = s->shared > 0 ? T : 0;
    p.max_items = p.npairs / RMDA_GEMM2_BM + E + (p.sh_rows + RMDA_GEMM2_BM - 1) / RMDA_GEMM2_BM;
    // expert segments are padded to RMDA_HP_ROWS rows (at most 15 per expert),
    // and the shared expert's rows follow at a multiple of RMDA_HP_ROWS
    const uint32_t hpr = RMDA_HP_ROWS;
    p.sh_row0 = (p.npairs + E * (hpr - 1) + hpr - 1) / hpr * hpr;
    p.groups_rows = p.sh_row0 + (p.sh_rows + hpr - 1) / hpr * hpr;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        size_t at = o;
        o = align256(o + bytes);
        return at;
    };
    p.proj = take((size_t)T * p.ps * 4);
    p.idx = take((size_t)p.npairs * 4);
    p.wt = take((size_t)p.npairs * 4);
    p.lrank = take((size_t)p.npairs * 4);
    p.slot = take((size_t)p.npairs * 4);
    p.rowtok = take((size_t)(p.sh_row0 + RMDA_ROWTOK_PAD) * 4);
    p.count = take((size_t)E * 4);
    p.off = take((size_t)E * 4);
    p.hist = take((size_t)p.nblocks * E * 4);
    p.done = take(4);
    p.n_items = take(4);
    p.n_items_hot = take(4);
    // one list serves both tiles: the hot tile's items (RMDA_GEMM_HOT_BM rows)
    // are never more than the streaming tile's
    p.items = take((size_t)p.max_items * 16);
    p.hp = take((size_t)p.groups_rows * s->inter * 2);
    // arrival counters of the folded combine, one per (token, 64 columns)
    p.fc_cnt = take((size_t)T * (s->d / RMDA_FC_COLS) * 4);
    p.xs16 = take(x32 ? (size_t)T * s->d * 2 : 0);
    p.xpart = take(x32 ? (size_t)RMDA_XCAST_PARTS * 4 : 0);
    p.xslot = take(x32 ? 4 : 0);
    p.hslot = take(x32 ? 4 : 0);
    p.hparts = take(x32 ? RMDA_AMAX_BYTES : 0);  // gate_up's partial SwiGLU absmax words
    p.ye = take(x32 ? (size_t)p.groups_rows * std::max(s->d, s->inter) * 4 : (size_t)p.groups_rows * s->d * 2);
    p.total = o;
    return p;
}

// element offsets (halves) of the four weight sets inside a packed buffer
// Offsets in 16-bit units.  Every region size is a multiple of 256 units
// (d % 256 == 0), so each region starts 512-byte aligned.
struct PackPlan {
    size_t gate_up, down, sh_gate_up, sh_down, router, bound, total;
};

PackPlan plan_pack(const rmda_moe_shape_t *s) {
    PackPlan p{};
    const size_t d = s->d;
    const uint32_t cols = s->experts + (s->shared > 0 ? 1u : 0u);
    p.gate_up = 0;
    p.down = p.gate_up + (size_t)s->experts * 2 * s->inter * d;
    p.sh_gate_up = p.down + (size_t)s->experts * d * s->inter;
    p.sh_down = p.sh_gate_up + (size_t)2 * s->shared * d;
    p.router = p.sh_down + d * s->shared;
    // the down weights' row-sum bound (one fp32 word; 256 bytes kept)
    p.bound = p.router + 2 * d * rmda_router_cpad(cols);  // fp32 router rows before it
    p.total = p.bound + 128;
    return p;
}

template <typename T>
T *at(void *base, size_t off) {
    return reinterpret_cast<T *>(reinterpret_cast<char *>(base) + off);
}

}  // namespace

extern "C" {

const char *rmda_moe_version(void) {
    return "rmda_moe 0.3 (gfx950, wave64, fp16 MFMA)";
}

int rmda_moe_abi_version(void) {
    return RMDA_MOE_ABI_VERSION;
}

int rmda_moe_ctx_create(rmda_moe_ctx_t **out, int device, void *stream) {
    if (out == nullptr) {
        return RMDA_ERR_ARG;
    }
    *out = nullptr;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
        return RMDA_ERR_DEVICE;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        return RMDA_ERR_DEVICE;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        return RMDA_ERR_DEVICE;
    }
    int prev = -1;
    (void)hipGetDevice(&prev);
    if (hipSetDevice(device) != hipSuccess) {
        return RMDA_ERR_DEVICE;
    }
    rmda_moe_ctx_t *c = new rmda_moe_ctx_t();
    c->device = device;
    c->stream = reinterpret_cast<hipStream_t>(stream);
    c->err = RMDA_OK;
    c->msg[0] = 0;
    const size_t words = (size_t)RMDA_CTX_MAX_PAIRS + kHistBlocks * RMDA_MAX_EXPERTS + 64;
    if (hipMalloc(&c->fixed_ws, words * 4) != hipSuccess) {
        delete c;
        return RMDA_ERR_HIP;
    }
    c->lrank = c->fixed_ws;
    c->hist = c->lrank + RMDA_CTX_MAX_PAIRS;
    c->done = c->hist + kHistBlocks * RMDA_MAX_EXPERTS;
    // the rank ticket must start at zero; the kernel leaves it at zero
    if (hipMemset(c->done, 0, 64 * 4) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        (void)hipFree(c->fixed_ws);
        delete c;
        return RMDA_ERR_HIP;
    }
    // this device's copy of the allocation-free layer's workspace, looked up
    // once per device with the device current
    if (device < kMaxDevices) {
        std::lock_guard<std::mutex> lock(g_static_mu);
        if (g_static_ws[device] == nullptr) {
            void *ptr = nullptr;
            if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
                (void)hipFree(c->fixed_ws);
                delete c;
                return RMDA_ERR_HIP;
            }
            g_static_ws[device] = ptr;
        }
        c->static_ws = g_static_ws[device];
    }
    c->scatter_experts = 0;
    c->g2 = rmda_gemm2_variant(0);
    if (const char *v = getenv("RMDA_MOE_GEMM_VARIANT")) {
        c->g2 = rmda_gemm2_variant(atoi(v));
    }
    c->g2.grid = prop.multiProcessorCount > 0 ? (uint32_t)prop.multiProcessorCount : 256u;
    c->hot_min = RMDA_GEMM_HOT_MIN;
    if (const char *v = getenv("RMDA_MOE_HOT_MIN")) {
        c->hot_min = (uint32_t)strtoul(v, nullptr, 10);
    }
    c->hot_stages = 4;
    if (const char *v = getenv("RMDA_MOE_HOT_STAGES")) {
        c->hot_stages = atoi(v) == 5 ? 5 : 4;
    }
    c->hot_sched = 0;
    if (const char *v = getenv("RMDA_MOE_HOT_SCHED")) {
        c->hot_sched = atoi(v);
    }
    c->route_rank = 0;
    if (const char *v = getenv("RMDA_MOE_ROUTE_IN_RANK")) {
        c->route_rank = atoi(v) != 0 ? 1 : 0;
    }
    c->fused_combine = 0;
    if (const char *v = getenv("RMDA_MOE_FUSED_COMBINE")) {
        c->fused_combine = atoi(v) != 0 ? 1 : 0;
    }
    c->tile_policy = RMDA_TILE_ADAPTIVE;
    if (const char *v = getenv("RMDA_MOE_TILE_POLICY")) {  // tuning only
        const int pol = atoi(v);
        c->tile_policy = pol >= RMDA_TILE_ADAPTIVE && pol <= RMDA_TILE_HOT ? pol : RMDA_TILE_ADAPTIVE;
    }
    if (hipHostMalloc(reinterpret_cast<void **>(&c->tile_hint_host), kHintSlots * 4, hipHostMallocMapped) !=
            hipSuccess ||
        hipHostGetDevicePointer(reinterpret_cast<void **>(&c->tile_hint_dev), c->tile_hint_host, 0) != hipSuccess) {
        (void)hipFree(c->fixed_ws);
        delete c;
        return RMDA_ERR_HIP;
    }
    hint_clear(c);
    if (prev >= 0 && prev != device) {
        (void)hipSetDevice(prev);
    }
    *out = c;
    return RMDA_OK;
}

void rmda_moe_ctx_destroy(rmda_moe_ctx_t *ctx) {
    if (ctx == nullptr) {
        return;
    }
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->up_made) {
        (void)hipStreamSynchronize(ctx->up_stream);
        for (int b = 0; b < 2; b += 1) {
            (void)hipHostFree(ctx->up_host[b]);
            (void)hipFree(ctx->up_dev[b]);
            (void)hipEventDestroy(ctx->up_done[b]);
        }
        (void)hipEventDestroy(ctx->up_after);
        (void)hipStreamDestroy(ctx->up_stream);
    }
    (void)hipFree(ctx->fixed_ws);
    (void)hipHostFree(ctx->tile_hint_host);
    if (ctx->prof_made) {
        for (uint32_t i = 0; i < RMDA_PROF_RING; i += 1) {
            for (uint32_t st = 0; st <= RMDA_PROF_STAGES; st += 1) {
                (void)hipEventDestroy(ctx->prof_ev[i][st]);
            }
        }
    }
    delete ctx;
}

int rmda_moe_prof_begin(rmda_moe_ctx_t *ctx) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (!ctx->prof_made) {
        for (uint32_t i = 0; i < RMDA_PROF_RING && rc == RMDA_OK; i += 1) {
            for (uint32_t st = 0; st <= RMDA_PROF_STAGES + 1 && rc == RMDA_OK; st += 1) {
                rc = hip_check(ctx, hipEventCreate(&ctx->prof_ev[i][st]), "profiler hipEventCreate");
            }
        }
        if (rc != RMDA_OK) {
            return rc;
        }
        ctx->prof_made = 1;
    }
    ctx->prof_on = 1;
    ctx->prof_pending = 0;
    ctx->prof_layers = 0;
    for (uint32_t st = 0; st < RMDA_PROF_STAGES; st += 1) {
        ctx->prof_ms[st] = 0.0;
    }
    ctx->prof_empty_ms = 0.0;
    return RMDA_OK;
}

int rmda_moe_prof_empty_ms(rmda_moe_ctx_t *ctx, double *ms) {
    if (ctx == nullptr || ms == nullptr) {
        return RMDA_ERR_ARG;
    }
    *ms = ctx->prof_empty_ms;
    return RMDA_OK;
}

int rmda_moe_prof_end(rmda_moe_ctx_t *ctx, double *ms, uint32_t *layers) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (!ctx->prof_on) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_prof_end: profiler not started");
    }
    rc = prof_harvest(ctx);
    ctx->prof_on = 0;
    if (rc != RMDA_OK) {
        return rc;
    }
    for (uint32_t st = 0; st < RMDA_PROF_STAGES; st += 1) {
        if (ms != nullptr) {
            ms[st] = ctx->prof_ms[st];
        }
    }
    if (layers != nullptr) {
        *layers = ctx->prof_layers;
    }
    return RMDA_OK;
}

const char *rmda_moe_prof_stage_name(uint32_t i) {
    return i < RMDA_PROF_STAGES ? kStageNames[i] : nullptr;
}

int rmda_moe_set_stream(rmda_moe_ctx_t *ctx, void *stream) {
    if (ctx == nullptr) {
        return RMDA_ERR_ARG;
    }
    ctx->stream = reinterpret_cast<hipStream_t>(stream);
    return RMDA_OK;
}

int rmda_moe_set_hot_rows(rmda_moe_ctx_t *ctx, uint32_t rows) {
    if (ctx == nullptr) {
        return RMDA_ERR_ARG;
    }
    ctx->hot_min = rows;
    hint_clear(ctx);  // the next call on every layer chooses afresh
    return RMDA_OK;
}

int rmda_moe_set_tile_policy(rmda_moe_ctx_t *ctx, int policy) {
    if (ctx == nullptr || policy < RMDA_TILE_ADAPTIVE || policy > RMDA_TILE_HOT) {
        return RMDA_ERR_ARG;
    }
    ctx->tile_policy = policy;
    hint_clear(ctx);
    return RMDA_OK;
}

int rmda_moe_set_route_in_rank(rmda_moe_ctx_t *ctx, int on) {
    if (ctx == nullptr) {
        return RMDA_ERR_ARG;
    }
    ctx->route_rank = on != 0 ? 1 : 0;
    return RMDA_OK;
}

int rmda_moe_set_fused_combine(rmda_moe_ctx_t *ctx, int on) {
    if (ctx == nullptr) {
        return RMDA_ERR_ARG;
    }
    ctx->fused_combine = on != 0 ? 1 : 0;
    return RMDA_OK;
}

int rmda_moe_ctx_error(const rmda_moe_ctx_t *ctx) {
    return ctx == nullptr ? RMDA_ERR_ARG : ctx->err;
}

const char *rmda_moe_ctx_message(const rmda_moe_ctx_t *ctx) {
    return ctx == nullptr ? "null context" : ctx->msg;
}

void rmda_moe_ctx_clear_error(rmda_moe_ctx_t *ctx) {
    if (ctx != nullptr) {
        ctx->err = RMDA_OK;
        ctx->msg[0] = 0;
    }
}

int rmda_moe_sync(rmda_moe_ctx_t *ctx) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

// ---- per-stage drop-ins ----

int rmda_moe_route(rmda_moe_ctx_t *ctx, const rmda_pc_moe_route_t *pc, const float *proj, uint32_t *idx,
                   float *wt, uint32_t *count) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (pc == nullptr || proj == nullptr || idx == nullptr || wt == nullptr || count == nullptr) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_route: null argument");
    }
    if (pc->experts == 0 || pc->experts > RMDA_MAX_EXPERTS) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_route: experts=%u not in 1..%u", pc->experts, RMDA_MAX_EXPERTS);
    }
    if (pc->topk == 0 || pc->topk > RMDA_MAX_TOPK || pc->topk > pc->experts) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_route: topk=%u not in 1..min(%u, experts)", pc->topk,
                    RMDA_MAX_TOPK);
    }
    if (pc->stride < pc->experts) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_route: stride=%u < experts=%u", pc->stride, pc->experts);
    }
    const uint64_t npairs = (uint64_t)pc->rows * pc->topk;
    if (npairs <= RMDA_CTX_MAX_PAIRS) {
        // top-k without atomics, then the counts from an LDS histogram (one
        // workgroup up to RMDA_COUNT1_MAX_PAIRS pairs, else rank_kernel's
        // per-block histograms): 16 K atomic adds onto E counters contend,
        // 31 us against 7.8 us at config 3
        rc = hip_check(ctx, rmda_launch_route(ctx->stream, proj, idx, wt, nullptr, pc->rows, pc->experts, pc->topk,
                                              pc->stride),
                       "route");
        if (rc == RMDA_OK && npairs <= RMDA_COUNT1_MAX_PAIRS) {
            // one workgroup's LDS histogram: no hand-off between blocks
            rc = hip_check(ctx, rmda_launch_count(ctx->stream, idx, (uint32_t)npairs, pc->experts, count),
                           "route counts");
        } else if (rc == RMDA_OK) {
            rmda_rank_args_t ra{};
            ra.idx = idx;
            ra.npairs = (uint32_t)npairs;
            ra.experts = pc->experts;
            ra.tile = 1;
            ra.lrank = ctx->lrank;
            ra.hist = ctx->hist;
            ra.count = count;
            ra.done = ctx->done;
            rc = hip_check(ctx, rmda_launch_rank(ctx->stream, &ra), "route counts");
        }
    } else {
        rc = hip_check(ctx, rmda_launch_zero(ctx->stream, count, pc->experts, 0), "zero count");
        if (rc == RMDA_OK) {
            rc = hip_check(ctx, rmda_launch_route(ctx->stream, proj, idx, wt, count, pc->rows, pc->experts, pc->topk,
                                                  pc->stride),
                           "route");
        }
    }
    if (rc == RMDA_OK) {
        ctx->scatter_experts = pc->experts;
    }
    return rc;
}

int rmda_moe_scan(rmda_moe_ctx_t *ctx, const rmda_pc_moe_scan_t *pc, const uint32_t *count, uint32_t *off,
                  uint32_t *tiles, uint32_t n_tiles) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (pc == nullptr || count == nullptr || off == nullptr || (tiles == nullptr && n_tiles > 0)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_scan: null argument");
    }
    if (pc->experts == 0 || pc->experts > RMDA_MAX_EXPERTS || pc->tile == 0) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_scan: experts=%u tile=%u", pc->experts, pc->tile);
    }
    return hip_check(ctx, rmda_launch_scan(ctx->stream, count, off, tiles, n_tiles, pc->experts, pc->tile),
                     "scan");
}

int rmda_moe_scatter_experts(rmda_moe_ctx_t *ctx, uint32_t experts) {
    if (ctx == nullptr) {
        return RMDA_ERR_ARG;
    }
    if (experts == 0 || experts > RMDA_MAX_EXPERTS) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_scatter_experts: experts=%u", experts);
    }
    ctx->scatter_experts = experts;
    return RMDA_OK;
}

int rmda_moe_scatter(rmda_moe_ctx_t *ctx, const rmda_pc_moe_scatter_t *pc, const uint32_t *idx,
                     const uint32_t *off, uint32_t *fill, const uint16_t *x16, uint16_t *xp, uint32_t *slot) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (pc == nullptr || idx == nullptr || off == nullptr || fill == nullptr || slot == nullptr ||
        (xp != nullptr && x16 == nullptr)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_scatter: null argument");
    }
    if (!aligned(x16, 16) || !aligned(xp, 16)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_scatter: x16 and xp must be 16-byte aligned");
    }
    if (ctx->scatter_experts == 0) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_scatter: expert count unknown (call rmda_moe_route or "
                                       "rmda_moe_scatter_experts first)");
    }
    const uint64_t npairs = (uint64_t)pc->rows * pc->topk;
    if (npairs > RMDA_CTX_MAX_PAIRS) {
        return fail(ctx, RMDA_ERR_CAPACITY, "rmda_moe_scatter: rows*topk=%llu exceeds %u",
                    (unsigned long long)npairs, RMDA_CTX_MAX_PAIRS);
    }
    if (pc->topk == 0 || pc->topk > RMDA_MAX_TOPK || (xp != nullptr && pc->d8 == 0)) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_scatter: topk=%u d8=%u", pc->topk, pc->d8);
    }
    if (xp != nullptr && npairs <= RMDA_SCATTER1_MAX_PAIRS) {
        return hip_check(ctx, rmda_launch_scatter1(ctx->stream, idx, off, fill, pc->rows, pc->topk,
                                                   ctx->scatter_experts, slot, x16, xp, pc->d8),
                         "scatter");
    }
    rmda_rank_args_t ra{};
    ra.idx = idx;
    ra.npairs = (uint32_t)npairs;
    ra.experts = ctx->scatter_experts;
    ra.tile = 1;
    ra.lrank = ctx->lrank;
    ra.hist = ctx->hist;
    ra.count = fill;  // the reference's atomics leave the per-expert counts in fill
    ra.off = nullptr;
    ra.off_in = off;
    ra.done = ctx->done;
    rc = hip_check(ctx, rmda_launch_rank(ctx->stream, &ra), "rank");
    if (rc != RMDA_OK) {
        return rc;
    }
    return hip_check(ctx, rmda_launch_permute(ctx->stream, idx, ctx->lrank, ctx->hist, (uint32_t)npairs, pc->topk,
                                              ctx->scatter_experts, slot, nullptr, x16, xp, pc->d8),
                     "permute");
}

// rmda_moe_mm, and for the recording's own calls the same with the
// segments' offsets and counts (live_off, live_count): rows past a segment's
// routed rows are then not computed, and C keeps its old values there.
// With swi (the recording's gate_up; a shape the persistent kernel takes)
// the kernel writes SwiGLU(C) to swi->out and its absmax to amax[swi->so]
// instead of C, and *swi->fused says whether it did.
struct mm_swiglu_t {
    float *out;
    uint32_t so;
    bool fused;
};
static int moe_mm(rmda_moe_ctx_t *ctx, const rmda_pc_moe_mm_t *pc, const uint16_t *a, const uint16_t *b, float *c,
                  const uint32_t *amax, const uint32_t *tiles, const uint32_t *live_off,
                  const uint32_t *live_count, mm_swiglu_t *swi = nullptr) {
    if (swi != nullptr) {
        swi->fused = false;
    }
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (pc == nullptr || a == nullptr || b == nullptr || c == nullptr || tiles == nullptr ||
        (amax == nullptr && (pc->sa != RMDA_NO_SLOT || pc->sb != RMDA_NO_SLOT))) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_mm: null argument");
    }
    if (!aligned(a, 16) || !aligned(b, 16) || !aligned(c, 16)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_mm: a, b and c must be 16-byte aligned");
    }
    if (pc->m % RMDA_MM_TILE != 0 || pc->n == 0 || pc->n % RMDA_MM_TILE != 0 || pc->k == 0 || pc->k % 32 != 0) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_mm: m=%u n=%u k=%u (need m,n %% 128 == 0, k %% 32 == 0)", pc->m,
                    pc->n, pc->k);
    }
    rmda_gemm_args_t g{};
    g.mode = RMDA_GEMM_F32;
    g.a = a;
    g.lda = pc->k;
    g.w = b;
    g.shared_group = RMDA_NONE;
    g.n_w = pc->n;
    g.k = pc->k;
    g.n_out = pc->n;
    g.out = c;
    g.ldo = pc->n;
    g.max_items = pc->m / RMDA_MM_TILE;
    g.tiles = tiles;
    g.amax = amax;
    g.sa = pc->sa;
    g.sb = pc->sb;
    if (rmda_ref_mm_supported(&g)) {
        g.live_off = live_off;
        g.live_count = live_count;
        if (swi != nullptr && swi->out != nullptr) {
            g.f32_swiglu = 1;
            g.so = swi->so;
            g.out = swi->out;
            g.ldo = pc->n / 2;
            swi->fused = true;
        }
        return hip_check(ctx, rmda_launch_ref_mm(ctx->stream, &g, ctx->g2.grid), "moe_mm");
    }
    return hip_check(ctx, rmda_launch_gemm(ctx->stream, &g), "moe_mm");  // computes every row
}

int rmda_moe_mm(rmda_moe_ctx_t *ctx, const rmda_pc_moe_mm_t *pc, const uint16_t *a, const uint16_t *b, float *c,
                const uint32_t *amax, const uint32_t *tiles) {
    return moe_mm(ctx, pc, a, b, c, amax, tiles, nullptr, nullptr);
}

static int combine_common(rmda_moe_ctx_t *ctx, const rmda_pc_moe_combine_t *pc, const float *wt,
                          const uint32_t *slot, const float *y, const float *proj, const float *sh,
                          const float *inj, float *h, uint16_t *out) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (pc == nullptr || wt == nullptr || slot == nullptr || y == nullptr || (sh != nullptr && proj == nullptr) ||
        (out == nullptr && pc->hc > 0 && (inj == nullptr || h == nullptr))) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_combine: null argument");
    }
    if (pc->topk == 0 || pc->topk > RMDA_MAX_TOPK) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_combine: topk=%u", pc->topk);
    }
    return hip_check(ctx, rmda_launch_combine(ctx->stream, pc, wt, slot, y, proj, sh, inj, h, out), "combine");
}

int rmda_moe_combine(rmda_moe_ctx_t *ctx, const rmda_pc_moe_combine_t *pc, const float *wt, const uint32_t *slot,
                     const float *y, const float *proj, const float *sh, const float *inj, float *h) {
    return combine_common(ctx, pc, wt, slot, y, proj, sh, inj, h, nullptr);
}

int rmda_moe_combine_plain(rmda_moe_ctx_t *ctx, const rmda_pc_moe_combine_t *pc, const float *wt,
                           const uint32_t *slot, const float *y, const float *proj, const float *sh,
                           uint16_t *out) {
    if (out == nullptr) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_combine_plain: null out");
    }
    return combine_common(ctx, pc, wt, slot, y, proj, sh, nullptr, nullptr, out);
}

int rmda_qwen_elem(rmda_moe_ctx_t *ctx, const rmda_pc_qwen_elem_t *pc, const float *a, float *y) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (pc == nullptr || a == nullptr || y == nullptr) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_qwen_elem: null argument");
    }
    if (pc->op > 1) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_qwen_elem: op=%u", pc->op);
    }
    return hip_check(ctx, rmda_launch_elem(ctx->stream, pc, a, y), "qwen_elem");
}

int rmda_absmax(rmda_moe_ctx_t *ctx, const rmda_pc_absmax_t *pc, const float *x, uint32_t *amax) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (pc == nullptr || x == nullptr || amax == nullptr || pc->slot == RMDA_NO_SLOT) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_absmax: null argument or no slot");
    }
    return hip_check(ctx, rmda_launch_absmax(ctx->stream, pc, x, amax), "absmax");
}

int rmda_cast_f16(rmda_moe_ctx_t *ctx, const rmda_pc_cast_t *pc, const float *src, uint16_t *dst,
                  const uint32_t *amax) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (pc == nullptr || src == nullptr || dst == nullptr || (amax == nullptr && pc->slot != RMDA_NO_SLOT)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_cast_f16: null argument");
    }
    return hip_check(ctx, rmda_launch_cast(ctx->stream, pc, src, dst, amax), "cast_f16");
}

int rmda_qwen_bf16(rmda_moe_ctx_t *ctx, const rmda_pc_qwen_bf16_t *pc, uint32_t *w) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (pc == nullptr || w == nullptr) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_qwen_bf16: null argument");
    }
    return hip_check(ctx, rmda_launch_bf16(ctx->stream, pc->n, w), "qwen_bf16");
}

int rmda_moe_router(rmda_moe_ctx_t *ctx, const rmda_moe_router_t *pc, const uint16_t *x16, const float *w,
                    const float *bias, float *proj) {
    return rmda_moe_router_slot(ctx, pc, x16, RMDA_NO_SLOT, nullptr, w, bias, proj);
}

int rmda_moe_router_slot(rmda_moe_ctx_t *ctx, const rmda_moe_router_t *pc, const uint16_t *x16, uint32_t slot,
                         const uint32_t *amax, const float *w, const float *bias, float *proj) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (pc == nullptr || x16 == nullptr || w == nullptr || proj == nullptr ||
        (slot != RMDA_NO_SLOT && amax == nullptr)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_router: null argument");
    }
    if (!aligned(amax, 4)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_router: amax not 4-byte aligned");
    }
    if (pc->d == 0 || pc->d % 128 != 0 || pc->cols == 0 || pc->cols > 65536 || pc->stride < pc->cols) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_router: d=%u cols=%u stride=%u (need d %% 128 == 0, "
                                         "1 <= cols <= stride)",
                    pc->d, pc->cols, pc->stride);
    }
    if (pc->rows == 0) {
        return RMDA_OK;
    }
    return hip_check(ctx,
                     rmda_launch_router(ctx->stream, x16, w, 0, bias, proj, pc->rows, pc->d, pc->cols, pc->stride,
                                        bias != nullptr ? pc->nbias : 0, nullptr, 0, nullptr,
                                        slot != RMDA_NO_SLOT ? amax + slot : nullptr),
                     "router");
}

// ---- fused layer ----

size_t rmda_moe_workspace_bytes(const rmda_moe_shape_t *shape) {
    if (shape == nullptr) {
        return 0;
    }
    char why[128];
    if (!check_shape(shape, why, sizeof(why))) {
        return 0;
    }
    return plan_layer(shape).total;
}

size_t rmda_moe_workspace_bytes_x32(const rmda_moe_shape_t *shape) {
    if (shape == nullptr) {
        return 0;
    }
    char why[128];
    if (!check_shape(shape, why, sizeof(why))) {
        return 0;
    }
    return plan_layer(shape, true).total;
}

int rmda_moe_workspace_layout(const rmda_moe_shape_t *shape, rmda_moe_ws_layout_t *out) {
    if (shape == nullptr || out == nullptr) {
        return RMDA_ERR_ARG;
    }
    char why[128];
    if (!check_shape(shape, why, sizeof(why))) {
        return RMDA_ERR_SHAPE;
    }
    const LayerPlan p = plan_layer(shape);
    out->proj = p.proj;
    out->idx = p.idx;
    out->wt = p.wt;
    out->count = p.count;
    out->off = p.off;
    out->slot = p.slot;
    out->total = p.total;
    out->proj_stride = p.ps;
    out->items = p.items;
    out->n_items = p.n_items;
    out->n_items_hot = p.n_items_hot;
    return RMDA_OK;
}

// One grouped GEMM of the fused layer over the load buckets: the compute
// tile's launch reads the hot count, the streaming tile's the other (the rank
// kernel left one of the two at zero); tile_mode 1 or 2 launches only the
// tile the rank kernel was told to cut its list for.
static int gemm_pair(rmda_moe_ctx_t *ctx, hipStream_t s, rmda_gemm_args_t g, rmda_gemm2_cfg_t cfg, bool packed,
                     const uint32_t *n_items_hot, uint32_t tile_mode, const char *what) {
    if (tile_mode != 1u) {
        rmda_gemm_args_t h = g;
        h.n_items = n_items_hot;
        h.fc = rmda_fc_t{};  // the compute tile leaves the combine to combine16_kernel
        const int rc = hip_check(ctx, rmda_launch_gemm_hot(s, &h, cfg.grid, ctx->hot_stages, ctx->hot_sched), what);
        if (rc != RMDA_OK || tile_mode == 2u) {
            return rc;
        }
    }
    return hip_check(ctx, rmda_launch_gemm2(s, &g, cfg, packed ? 1 : 0), what);
}

int rmda_moe_layer(rmda_moe_ctx_t *ctx, const rmda_moe_shape_t *shape, const rmda_moe_layer_args_t *args) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (shape == nullptr || args == nullptr || (args->x == nullptr && args->x32 == nullptr) ||
        (args->packed == nullptr && (args->w_router == nullptr || args->w_gate_up == nullptr ||
                                     args->w_down == nullptr)) ||
        (args->out == nullptr && args->h == nullptr) || args->workspace == nullptr) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_layer: null argument");
    }
    if (args->x != nullptr && args->x32 != nullptr) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_layer: give x (fp16) or x32 (fp32), not both");
    }
    if (args->h != nullptr &&
        (args->inj == nullptr || args->hc == 0 || args->hc > RMDA_MAX_HC || args->inj_stride < args->inj_off + args->hc)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_layer: hyper-connection streams need inj and 1 <= hc <= %u "
                    "with inj_off + hc <= inj_stride (hc=%u, inj_off=%u, inj_stride=%u)", RMDA_MAX_HC, args->hc,
                    args->inj_off, args->inj_stride);
    }
    if (!aligned(args->x, 16) || !aligned(args->w_router, 16) || !aligned(args->w_gate_up, 16) ||
        !aligned(args->w_down, 16) || !aligned(args->w_sh_gate_up, 16) || !aligned(args->w_sh_down, 16) ||
        !aligned(args->packed, 16) || !aligned(args->out, 16) || !aligned(args->workspace, 16) ||
        !aligned(args->h, 16) || !aligned(args->x32, 16) || !aligned(args->bias, 4) || !aligned(args->inj, 4)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_layer: x, weights, out, h and workspace must be 16-byte aligned");
    }
    char why[128];
    if (!check_shape(shape, why, sizeof(why))) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_layer: %s", why);
    }
    if (shape->shared > 0 && args->packed == nullptr &&
        (args->w_sh_gate_up == nullptr || args->w_sh_down == nullptr)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_layer: shared expert weights missing");
    }
    // fp32 activations: the reference's slot-scaled casts (see rmda_moe_layer_args_t::x32)
    const bool x32 = args->x32 != nullptr;
    const LayerPlan p = plan_layer(shape, x32);
    if (args->workspace_bytes < p.total) {
        return fail(ctx, RMDA_ERR_WORKSPACE, "rmda_moe_layer: workspace %zu bytes < %zu%s", args->workspace_bytes,
                    p.total, x32 ? " (rmda_moe_workspace_bytes_x32)" : "");
    }
    if (shape->rows == 0) {
        return RMDA_OK;
    }
    void *ws = args->workspace;
    const uint32_t T = shape->rows;
    const uint32_t E = shape->experts;
    const uint32_t K = shape->topk;
    const uint32_t I = shape->inter;
    const uint32_t d = shape->d;
    hipStream_t s = ctx->stream;
    float *proj = at<float>(ws, p.proj);
    uint32_t *idx = at<uint32_t>(ws, p.idx);
    float *wt = at<float>(ws, p.wt);
    uint32_t *lrank = at<uint32_t>(ws, p.lrank);
    uint32_t *slot = at<uint32_t>(ws, p.slot);
    uint32_t *rowtok = at<uint32_t>(ws, p.rowtok);
    uint32_t *done = at<uint32_t>(ws, p.done);
    uint16_t *hp = at<uint16_t>(ws, p.hp);
    uint16_t *ye = at<uint16_t>(ws, p.ye);
    // the activations the router and gate_up read, and (x32) the two slots
    const uint16_t *xin = x32 ? at<uint16_t>(ws, p.xs16) : args->x;
    uint32_t *xslot = x32 ? at<uint32_t>(ws, p.xslot) : nullptr;
    uint32_t *hslot = x32 ? at<uint32_t>(ws, p.hslot) : nullptr;
    const uint16_t *packed = args->packed;
    const PackPlan pk = plan_pack(shape);
    const uint16_t *w_gu = packed != nullptr ? packed + pk.gate_up : args->w_gate_up;
    const uint16_t *w_dn = packed != nullptr ? packed + pk.down : args->w_down;
    const uint16_t *w_sgu = packed != nullptr ? packed + pk.sh_gate_up : args->w_sh_gate_up;
    const uint16_t *w_sdn = packed != nullptr ? packed + pk.sh_down : args->w_sh_down;
    const float *w_rt = packed != nullptr ? reinterpret_cast<const float *>(packed + pk.router) : args->w_router;
    const uint32_t *ye_bound = packed != nullptr ? reinterpret_cast<const uint32_t *>(packed + pk.bound) : nullptr;

    if (ctx->prof_on && ctx->prof_pending == RMDA_PROF_RING) {
        rc = prof_harvest(ctx);
        if (rc != RMDA_OK) {
            return rc;
        }
    }
    rc = prof_mark(ctx, 0);
    // fp32 activations: x's absmax into a fresh slot and the scaled fp16 cast
    // the router and gate_up read (absmax.comp + cast_f16.comp,
    // src/qwen.c:517-539, :844); the second launch also clears gate_up's
    // partial absmax words
    if (rc == RMDA_OK && x32) {
        rc = hip_check(ctx, rmda_launch_x_absmax(s, args->x32, (size_t)T * d, at<uint32_t>(ws, p.xpart)),
                       "layer x absmax");
        if (rc == RMDA_OK) {
            rc = hip_check(ctx,
                           rmda_launch_x_cast(s, args->x32, (size_t)T * d, at<uint32_t>(ws, p.xpart),
                                              at<uint16_t>(ws, p.xs16), xslot, at<uint32_t>(ws, p.hparts)),
                           "layer x cast");
        }
    }
    // A0 router projection (+ zero the rank ticket for this call) with the A1
    // top-k fused in when one workgroup can hold a token's whole logit row
    const bool fuse_route = p.ps <= rmda_route_fuse_max_cols();
    rmda_route_fuse_t fz{E, K, idx, wt};
    if (rc == RMDA_OK) {
        rc = hip_check(ctx,
                       rmda_launch_router(s, xin, w_rt, packed != nullptr, args->bias, proj, T, d, p.ps, p.ps,
                                          args->bias != nullptr ? E : 0, done, 1, fuse_route ? &fz : nullptr,
                                          xslot),
                       "layer router");
    }
    if (rc == RMDA_OK) {
        rc = prof_mark(ctx, RMDA_STAGE_ROUTER + 1);
    }
    // A1 top-k (unless fused above).  The rank kernel routes the rows itself
    // when its blocks can rank without a hand-off of block totals (one rank
    // block, or up to RMDA_RANK_ALL_MAX pairs, where every rank block counts
    // every pair), so the chain before gate_up is two launches (router, rank)
    // instead of three.
    const bool self_perm = p.nblocks == 1 ||
                           (p.npairs <= RMDA_RANK_ALL_MAX && (reinterpret_cast<uintptr_t>(idx) & 15u) == 0);
    const bool route_in_rank = !fuse_route && self_perm && (ctx->route_rank != 0 || p.nblocks == 1);
    if (rc == RMDA_OK && !fuse_route && !route_in_rank) {
        rc = hip_check(ctx, rmda_launch_route(s, proj, idx, wt, nullptr, T, E, K, p.ps), "layer route");
        if (rc == RMDA_OK) {
            rc = prof_mark(ctx, RMDA_STAGE_ROUTE + 1);
        }
    } else if (rc == RMDA_OK) {
        prof_skip(ctx, RMDA_STAGE_ROUTE);
    }
    // Tile of the two GEMMs (0: both launch, the rank kernel decides; 1: the
    // streaming tile only; 2: the compute tile only).  No expert can be hot
    // with fewer rows than hot_min (a token adds at most one row per expert).
    const bool hot_possible = packed != nullptr && ctx->hot_min > 0 && T >= ctx->hot_min;
    uint32_t tile_mode = 1;
    uint32_t hint_slot = 0;
    if (hot_possible) {
        switch (ctx->tile_policy) {
        case RMDA_TILE_STREAM: tile_mode = 1; break;
        case RMDA_TILE_HOT: tile_mode = 2; break;
        case RMDA_TILE_AUTO: tile_mode = 0; break;
        default: tile_mode = hint_lookup(ctx, packed, T, &hint_slot);
        }
    }
    // The combine folds into the down GEMM when the streaming tile runs it on
    // packed weights; when the compute tile may run instead, combine16_kernel
    // is enqueued too and does the combine only if that tile ran.
    const bool fold_combine =
        ctx->fused_combine != 0 && packed != nullptr && ctx->g2.spec != 0 && tile_mode != 2u && !x32;
    // A2 counts, offsets, block bases and the GEMM work list
    if (rc == RMDA_OK) {
        rmda_rank_args_t ra{};
        ra.idx = idx;
        ra.npairs = p.npairs;
        ra.experts = E;
        ra.tile = RMDA_HP_ROWS;  // segments start at multiples of 16 rows (the hp block layout)
        ra.lrank = lrank;
        ra.hist = at<uint32_t>(ws, p.hist);
        ra.count = at<uint32_t>(ws, p.count);
        ra.off = at<uint32_t>(ws, p.off);
        ra.done = done;
        ra.items = at<uint32_t>(ws, p.items);
        ra.n_items = at<uint32_t>(ws, p.n_items);
        ra.bm = RMDA_GEMM2_BM;
        // load buckets: packed weights can take the compute tile when hot
        // experts hold most rows (hot_min 0: never; the hot count is then 0)
        ra.n_items_hot = at<uint32_t>(ws, p.n_items_hot);
        ra.bm_hot = RMDA_GEMM_HOT_BM;
        ra.hot_min = hot_possible ? ctx->hot_min : 0u;
        ra.force = tile_mode;
        ra.hint_out =
            ctx->tile_policy == RMDA_TILE_ADAPTIVE && hot_possible ? ctx->tile_hint_dev + hint_slot : nullptr;
        ra.shared_rows = p.sh_rows;
        ra.shared_row0 = p.sh_row0;
        // all pairs in one rank block, or few enough pairs that every block
        // counts them all: the rank blocks write the permutation too
        ra.topk = K;
        if (route_in_rank) {
            ra.route_proj = proj;
            ra.route_rows = T;
            ra.route_stride = p.ps;
            ra.route_idx = idx;
            ra.route_wt = wt;
        }
        if (fold_combine) {
            ra.fc_cnt = at<uint32_t>(ws, p.fc_cnt);
            ra.fc_nblk = d / RMDA_FC_COLS;
            ra.fc_rows = T;
            ra.fc_shared = shape->shared > 0 ? 1u : 0u;
            ra.fc_zero_out = args->out;
            ra.fc_d = d;
        }
        if (self_perm) {
            ra.slot = slot;
            ra.rowtok = rowtok;
            ra.topk = K;
            ra.count_all = p.nblocks > 1 ? 1u : 0u;
        }
        rc = hip_check(ctx, rmda_launch_rank(s, &ra), "layer rank");
    }
    if (rc == RMDA_OK) {
        rc = prof_mark(ctx, RMDA_STAGE_RANK + 1);
    }
    // A3 permutation (slots + row -> token map; x is gathered, not copied)
    if (rc == RMDA_OK && !self_perm) {
        rc = hip_check(ctx,
                       rmda_launch_permute(s, idx, lrank, at<uint32_t>(ws, p.hist), p.npairs, K, E, slot, rowtok,
                                           nullptr, nullptr, 0),
                       "layer permute");
        if (rc == RMDA_OK) {
            rc = prof_mark(ctx, RMDA_STAGE_PERMUTE + 1);
        }
    } else if (rc == RMDA_OK) {
        prof_skip(ctx, RMDA_STAGE_PERMUTE);
    }
    rmda_gemm_args_t g{};
    g.items = at<uint32_t>(ws, p.items);
    g.n_items = at<uint32_t>(ws, p.n_items);
    g.max_items = p.max_items;
    g.shared_group = shape->shared > 0 ? E : RMDA_NONE;
    g.shared_row0 = p.sh_row0;
    g.sa = RMDA_NO_SLOT;
    g.sb = RMDA_NO_SLOT;
    // A4-A6 gate_up with SwiGLU epilogue -> hp16
    if (rc == RMDA_OK) {
        g.mode = RMDA_GEMM_SWIGLU;
        g.a = xin;
        g.xscale = xslot;
        g.hp32 = x32 ? at<float>(ws, p.ye) : nullptr;  // fp32 SwiGLU output, cast below
        g.hp_amax = x32 ? at<uint32_t>(ws, p.hparts) : nullptr;
        g.rowtok = rowtok;
        g.a_rows = T;
        g.lda = d;
        g.w = w_gu;
        g.w_shared = w_sgu;
        g.n_w = 2 * I;
        g.k = d;
        g.n_out = I;
        g.inter = I;
        g.out = hp;
        g.ldo = I;
        // The default configuration streams gate_up's gathered rows through a
        // ring of two-K-step slots when experts average 32 rows or more
        // (configs 3 and 5: -2.1% / -2.4% gate_up); at decode sizes, where
        // almost every activation row is padding, the single ring is faster
        // (config 2: +5% with the activation ring).
        rmda_gemm2_cfg_t gu = ctx->g2;
        if (gu.spec == 6 && (uint64_t)T * K >= 32ull * E) {
            gu.spec = 7;
        }
        // the compute tile first (it has work only when the rank kernel cut
        // the list for it), then the streaming tile (work only otherwise)
        rc = gemm_pair(ctx, s, g, gu, packed != nullptr, at<uint32_t>(ws, p.n_items_hot), tile_mode, "layer gate_up");
    }
    // x32: hp's slot-scaled fp16 cast (src/qwen.c:858-877), routed and shared rows
    if (rc == RMDA_OK && x32) {
        rc = hip_check(ctx,
                       rmda_launch_hp_cast(s, at<float>(ws, p.ye), hp, at<uint32_t>(ws, p.hparts), hslot,
                                           at<uint32_t>(ws, p.off), at<uint32_t>(ws, p.count), E, I, p.sh_row0,
                                           p.sh_rows),
                       "layer hp cast");
    }
    if (rc == RMDA_OK) {
        rc = prof_mark(ctx, RMDA_STAGE_GATE_UP + 1);
    }
    // A7 down -> ye16 (the shared expert's rows follow the routed rows)
    if (rc == RMDA_OK) {
        g.mode = RMDA_GEMM_F16;
        g.a = hp;
        g.rowtok = nullptr;
        g.xscale = nullptr;
        g.hp32 = nullptr;
        g.hp_amax = nullptr;
        // x32: fp16 expert rows scaled by the packed weights' row-sum bound;
        // fp32 rows (the reference's ye) for HF-layout weights, which carry
        // no bound
        g.yscale = hslot;
        g.ye32 = x32 && packed == nullptr ? at<float>(ws, p.ye) : nullptr;
        g.ye_bound = x32 && packed != nullptr ? ye_bound : nullptr;
        // experts averaging 64 rows or more: either tile writes its fp16
        // rows with non-temporal stores.  Same-box A/B: config 3 layer -1.2
        // to -1.5% (down 93.6 -> 85.2 us, the combine, which then reads them
        // from HBM, 10.0 -> 12.9), config 4 (compute tile) -1.8%, config 5
        // (80 rows) -0.6 to -0.7%; at 40 rows (the teacher's shape) +0.35%
        // and at 8 (decode) +1.7%, hence the bound
        g.ye_nt = p.npairs >= 64ull * E ? 1u : 0u;
        g.lda = I;
        g.w = w_dn;
        g.w_shared = w_sdn;
        g.n_w = d;
        g.k = I;
        g.n_out = d;
        g.inter = 0;
        g.out = ye;
        g.ldo = d;
        if (fold_combine) {
            g.fc.cnt = at<uint32_t>(ws, p.fc_cnt);
            g.fc.nblk = d / RMDA_FC_COLS;
            g.fc.rowtok = rowtok;
            g.fc.slot = slot;
            g.fc.wt = wt;
            g.fc.proj = proj;
            g.fc.pstride = p.ps;
            g.fc.sg_off = E;
            g.fc.topk = K;
            g.fc.has_shared = shape->shared > 0 ? 1u : 0u;
            g.fc.out = args->out;
            g.fc.hc = rmda_hc_t{args->h, args->inj, args->inj_stride, args->inj_off, args->hc};
        }
        rc = gemm_pair(ctx, s, g, ctx->g2, packed != nullptr, at<uint32_t>(ws, p.n_items_hot), tile_mode,
                       "layer down");
    }
    if (rc == RMDA_OK) {
        rc = prof_mark(ctx, RMDA_STAGE_DOWN + 1);
    }
    // A8/A9 combine (+ sigmoid-gated shared expert, + hyper-connection streams)
    const rmda_hc_t hcp{args->h, args->inj, args->inj_stride, args->inj_off, args->hc};
    if (rc == RMDA_OK && x32 && packed == nullptr) {
        // fp32 expert rows: the reference's combine arithmetic
        // (shader/moe_combine.comp:26-40), fp16 out and/or the streams
        const float *ye32 = at<float>(ws, p.ye);
        const rmda_pc_moe_combine_t pm{T, d, K, p.ps, E, args->inj_stride, args->inj_off, args->h != nullptr ? args->hc : 0u};
        rc = hip_check(ctx,
                       rmda_launch_combine(s, &pm, wt, slot, ye32, proj,
                                           shape->shared > 0 ? ye32 + (size_t)p.sh_row0 * d : nullptr, args->inj,
                                           args->h, args->out),
                       "layer combine");
        if (rc == RMDA_OK) {
            rc = prof_mark(ctx, RMDA_STAGE_COMBINE + 1);
        }
    } else if (rc == RMDA_OK && !(fold_combine && tile_mode == 1u)) {
        rc = hip_check(ctx,
                       rmda_launch_combine16(s, wt, slot, ye, proj, p.ps, E, p.sh_row0, shape->shared > 0, args->out,
                                             T, d, K, &hcp, fold_combine ? at<uint32_t>(ws, p.n_items_hot) : nullptr,
                                             x32 ? hslot : nullptr, x32 ? ye_bound : nullptr),
                       "layer combine");
        if (rc == RMDA_OK) {
            rc = prof_mark(ctx, RMDA_STAGE_COMBINE + 1);
        }
    } else if (rc == RMDA_OK) {
        prof_skip(ctx, RMDA_STAGE_COMBINE);
    }
    if (rc == RMDA_OK && ctx->prof_on) {
        ctx->prof_pending += 1;
    }
    return rc;
}

int rmda_moe_layer_static(rmda_moe_ctx_t *ctx, const rmda_moe_shape_t *shape, const rmda_moe_layer_args_t *args) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (shape == nullptr || args == nullptr) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_layer_static: null argument");
    }
    if (args->workspace != nullptr || args->workspace_bytes != 0) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_layer_static: takes no workspace (workspace must be NULL, "
                    "workspace_bytes 0); the library's static scratch is used");
    }
    if (ctx->static_ws == nullptr) {
        return fail(ctx, RMDA_ERR_DEVICE, "rmda_moe_layer_static: no static scratch on device %d", ctx->device);
    }
    char why[128];
    if (!check_shape(shape, why, sizeof(why))) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_layer_static: %s", why);
    }
    const size_t need = plan_layer(shape, args->x32 != nullptr).total;
    if (need > RMDA_STATIC_WS_BYTES) {
        return fail(ctx, RMDA_ERR_CAPACITY, "rmda_moe_layer_static: this shape needs %zu bytes of workspace, "
                    "beyond the static scratch's %zu (RMDA_STATIC_WS_BYTES); use rmda_moe_layer with a workspace",
                    need, (size_t)RMDA_STATIC_WS_BYTES);
    }
    rmda_moe_layer_args_t a = *args;
    a.workspace = ctx->static_ws;
    a.workspace_bytes = RMDA_STATIC_WS_BYTES;
    return rmda_moe_layer(ctx, shape, &a);
}

size_t rmda_moe_packed_bytes(const rmda_moe_shape_t *shape) {
    if (shape == nullptr) {
        return 0;
    }
    char why[128];
    if (!check_shape(shape, why, sizeof(why))) {
        return 0;
    }
    return plan_pack(shape).total * 2;
}

}  // extern "C"

namespace {

// Enqueue every pack kernel of one layer on stream s; bf16 flags per tensor.
int pack_layer(rmda_moe_ctx_t *ctx, hipStream_t s, const rmda_moe_shape_t *shape, const float *w_router,
               const uint16_t *gu, int gu_bf16, const uint16_t *dn, int dn_bf16, const uint16_t *sgu, int sgu_bf16,
               const uint16_t *sdn, int sdn_bf16, uint16_t *packed) {
    const PackPlan pk = plan_pack(shape);
    const uint32_t E = shape->experts, d = shape->d, I = shape->inter, S = shape->shared;
    const int bk = (int)ctx->g2.bk;
    int rc = hip_check(ctx, rmda_launch_pack(s, gu, packed + pk.gate_up, E, 2 * I, d, I, 1, bk, gu_bf16),
                       "pack gate_up");
    if (rc == RMDA_OK) {
        rc = hip_check(ctx, rmda_launch_pack(s, dn, packed + pk.down, E, d, I, I, 0, bk, dn_bf16), "pack down");
    }
    if (rc == RMDA_OK && S > 0) {
        rc = hip_check(ctx, rmda_launch_pack(s, sgu, packed + pk.sh_gate_up, 1, 2 * S, d, S, 1, bk, sgu_bf16),
                       "pack shared gate_up");
    }
    if (rc == RMDA_OK && S > 0) {
        rc = hip_check(ctx, rmda_launch_pack(s, sdn, packed + pk.sh_down, 1, d, S, S, 0, bk, sdn_bf16),
                       "pack shared down");
    }
    if (rc == RMDA_OK) {
        rc = hip_check(ctx,
                       rmda_launch_router_pack(s, w_router, reinterpret_cast<float *>(packed + pk.router),
                                               E + (S > 0 ? 1u : 0u), d),
                       "pack router");
    }
    // the largest row sum of |w| over the packed down weights (routed and
    // shared), which sizes the slot-scaled mode's fp16 expert rows; the rest
    // of its 256 bytes is zero, so equal weights pack to equal buffers
    uint32_t *bound = reinterpret_cast<uint32_t *>(packed + pk.bound);
    if (rc == RMDA_OK) {
        rc = hip_check(ctx, rmda_launch_zero(s, bound, 64, 0), "pack bound fill");
    }
    if (rc == RMDA_OK) {
        rc = hip_check(ctx, rmda_launch_row_abs_max(s, packed + pk.down, E, d, I, bk, bound), "pack down bound");
    }
    if (rc == RMDA_OK && S > 0) {
        rc = hip_check(ctx, rmda_launch_row_abs_max(s, packed + pk.sh_down, 1, d, S, bk, bound),
                       "pack shared down bound");
    }
    return rc;
}

}  // namespace

extern "C" {

int rmda_moe_pack_weights(rmda_moe_ctx_t *ctx, const rmda_moe_shape_t *shape, const float *w_router,
                          const uint16_t *w_gate_up, const uint16_t *w_down, const uint16_t *w_sh_gate_up,
                          const uint16_t *w_sh_down, int bf16, uint16_t *packed) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (shape == nullptr || w_router == nullptr || w_gate_up == nullptr || w_down == nullptr || packed == nullptr ||
        (shape->shared > 0 && (w_sh_gate_up == nullptr || w_sh_down == nullptr))) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_pack_weights: null argument");
    }
    if (!aligned(w_router, 16) || !aligned(w_gate_up, 16) || !aligned(w_down, 16) || !aligned(w_sh_gate_up, 16) ||
        !aligned(w_sh_down, 16) || !aligned(packed, 16)) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_pack_weights: weights and packed must be 16-byte aligned");
    }
    char why[128];
    if (!check_shape(shape, why, sizeof(why))) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_pack_weights: %s", why);
    }
    return pack_layer(ctx, ctx->stream, shape, w_router, w_gate_up, bf16, w_down, bf16, w_sh_gate_up, bf16,
                      w_sh_down, bf16, packed);
}

}  // extern "C"

namespace {

// One tensor of an upload: where it comes from and where it goes in a bank.
struct UpPiece {
    const uint8_t *src;
    size_t bytes;
    size_t dst;  // byte offset in the bank
};

uint64_t st_elems(const rmda_st_tensor_t &t) {
    uint64_t n = 1;
    for (uint32_t i = 0; i < t.ndim; i += 1) {
        n *= t.shape[i];
    }
    return n;
}

int up_find(rmda_moe_ctx_t *ctx, const rmda_st_t *st, const char *prefix, const char *suffix, uint64_t elems,
            uint64_t last_dim, bool f32_ok, rmda_st_tensor_t *t) {
    char name[512];
    snprintf(name, sizeof(name), "%s%s", prefix, suffix);
    if (rmda_st_find(st, name, t) != RMDA_OK) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_upload_layer: %s", rmda_st_message());
    }
    const bool dt_ok = t->dtype == RMDA_ST_BF16 || (f32_ok ? t->dtype == RMDA_ST_F32 : t->dtype == RMDA_ST_F16);
    if (!dt_ok) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_upload_layer: %s has dtype code %u (want bf16 or %s)", name,
                    t->dtype, f32_ok ? "f32" : "f16");
    }
    if (t->ndim == 0 || st_elems(*t) != elems || t->shape[t->ndim - 1] != last_dim) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_upload_layer: %s has %llu elements, last dim %llu; want %llu, %llu",
                    name, (unsigned long long)st_elems(*t), (unsigned long long)t->shape[t->ndim - 1],
                    (unsigned long long)elems, (unsigned long long)last_dim);
    }
    return RMDA_OK;
}

// Copy pieces into the pinned bank with up to 8 threads (page faults of the
// mapped file dominate; they proceed in parallel).
void up_copy(uint8_t *bank, const std::vector<UpPiece> &pieces) {
    size_t total = 0;
    for (const UpPiece &p : pieces) {
        total += p.bytes;
    }
    unsigned nt = std::thread::hardware_concurrency();
    nt = std::max(1u, std::min(8u, nt));
    if (total < ((size_t)64 << 20)) {
        nt = 1;
    }
    const size_t chunk = (total + nt - 1) / nt;
    auto work = [&](unsigned k) {
        // thread k copies global byte range [k*chunk, (k+1)*chunk) of the concatenation
        const size_t lo = (size_t)k * chunk;
        const size_t hi = std::min(total, lo + chunk);
        size_t base = 0;
        for (const UpPiece &p : pieces) {
            const size_t a = std::max(lo, base);
            const size_t b = std::min(hi, base + p.bytes);
            if (a < b) {
                memcpy(bank + p.dst + (a - base), p.src + (a - base), b - a);
            }
            base += p.bytes;
        }
    };
    if (nt == 1) {
        work(0);
        return;
    }
    std::vector<std::thread> th;
    for (unsigned k = 1; k < nt; k += 1) {
        th.emplace_back(work, k);
    }
    work(0);
    for (std::thread &t : th) {
        t.join();
    }
}

int up_reserve(rmda_moe_ctx_t *ctx, size_t bytes) {
    if (!ctx->up_made) {
        int rc = hip_check(ctx, hipStreamCreateWithFlags(&ctx->up_stream, hipStreamNonBlocking), "upload stream");
        for (int b = 0; rc == RMDA_OK && b < 2; b += 1) {
            rc = hip_check(ctx, hipEventCreateWithFlags(&ctx->up_done[b], hipEventDisableTiming), "upload event");
        }
        if (rc == RMDA_OK) {
            rc = hip_check(ctx, hipEventCreateWithFlags(&ctx->up_after, hipEventDisableTiming), "upload event");
        }
        if (rc != RMDA_OK) {
            return rc;
        }
        ctx->up_made = 1;
    }
    if (bytes <= ctx->up_cap) {
        return RMDA_OK;
    }
    int rc = hip_check(ctx, hipStreamSynchronize(ctx->up_stream), "upload sync");
    for (int b = 0; b < 2; b += 1) {
        (void)hipHostFree(ctx->up_host[b]);
        (void)hipFree(ctx->up_dev[b]);
        ctx->up_host[b] = nullptr;
        ctx->up_dev[b] = nullptr;
        ctx->up_used[b] = 0;
    }
    ctx->up_cap = 0;
    for (int b = 0; rc == RMDA_OK && b < 2; b += 1) {
        rc = hip_check(ctx, hipHostMalloc(reinterpret_cast<void **>(&ctx->up_host[b]), bytes, hipHostMallocDefault),
                       "pinned upload staging");
        if (rc == RMDA_OK) {
            rc = hip_check(ctx, hipMalloc(reinterpret_cast<void **>(&ctx->up_dev[b]), bytes), "device upload staging");
        }
    }
    if (rc == RMDA_OK) {
        ctx->up_cap = bytes;
    }
    return rc;
}

}  // namespace

extern "C" {

int rmda_moe_upload_layer(rmda_moe_ctx_t *ctx, const rmda_st_t *st, const char *prefix,
                          const rmda_moe_shape_t *shape, uint16_t *packed) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (st == nullptr || prefix == nullptr || shape == nullptr || packed == nullptr) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_upload_layer: null argument");
    }
    char why[128];
    if (!check_shape(shape, why, sizeof(why))) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_upload_layer: %s", why);
    }
    const uint64_t E = shape->experts, d = shape->d, I = shape->inter, S = shape->shared;
    rmda_st_tensor_t tr{}, tg{}, tgu{}, tdn{}, tsg{}, tsu{}, tsd{};
    rc = up_find(ctx, st, prefix, "gate.weight", E * d, d, true, &tr);
    if (rc == RMDA_OK && S > 0) {
        rc = up_find(ctx, st, prefix, "shared_expert_gate.weight", d, d, true, &tg);
    }
    if (rc == RMDA_OK) {
        rc = up_find(ctx, st, prefix, "experts.gate_up_proj", E * 2 * I * d, d, false, &tgu);
    }
    if (rc == RMDA_OK) {
        rc = up_find(ctx, st, prefix, "experts.down_proj", E * d * I, I, false, &tdn);
    }
    if (rc == RMDA_OK && S > 0) {
        rc = up_find(ctx, st, prefix, "shared_expert.gate_proj.weight", S * d, d, false, &tsg);
    }
    if (rc == RMDA_OK && S > 0) {
        rc = up_find(ctx, st, prefix, "shared_expert.up_proj.weight", S * d, d, false, &tsu);
    }
    if (rc == RMDA_OK && S > 0) {
        rc = up_find(ctx, st, prefix, "shared_expert.down_proj.weight", d * S, S, false, &tsd);
    }
    if (rc != RMDA_OK) {
        return rc;
    }
    if (S > 0 && tsg.dtype != tsu.dtype) {
        return fail(ctx, RMDA_ERR_SHAPE, "rmda_moe_upload_layer: shared gate_proj and up_proj dtypes differ");
    }
    // bank layout: router fp32 rows (E [+1]) x d, then the raw expert tensors
    const uint64_t rows_r = E + (S > 0 ? 1 : 0);
    const size_t off_r = 0;
    const size_t off_gu = align256(off_r + rows_r * d * 4);
    const size_t off_dn = align256(off_gu + tgu.bytes);
    const size_t off_sgu = align256(off_dn + tdn.bytes);
    const size_t off_sdn = align256(off_sgu + (S > 0 ? tsg.bytes + tsu.bytes : 0));
    const size_t total = align256(off_sdn + (S > 0 ? tsd.bytes : 0));
    rc = up_reserve(ctx, total);
    if (rc != RMDA_OK) {
        return rc;
    }
    const uint32_t bank = ctx->up_seq % 2;
    if (ctx->up_used[bank]) {
        rc = hip_check(ctx, hipEventSynchronize(ctx->up_done[bank]), "wait for upload bank");
        if (rc != RMDA_OK) {
            return rc;
        }
    }
    uint8_t *host = ctx->up_host[bank];
    uint8_t *dev = ctx->up_dev[bank];
    // router rows: bf16 widens exactly to fp32
    float *rw = reinterpret_cast<float *>(host + off_r);
    auto put_rows = [&](const rmda_st_tensor_t &t, float *dst, uint64_t n) {
        if (t.dtype == RMDA_ST_F32) {
            memcpy(dst, t.data, n * 4);
        } else {
            const uint16_t *b = static_cast<const uint16_t *>(t.data);
            for (uint64_t i = 0; i < n; i += 1) {
                const uint32_t u = (uint32_t)b[i] << 16;
                memcpy(&dst[i], &u, 4);
            }
        }
    };
    put_rows(tr, rw, E * d);
    if (S > 0) {
        put_rows(tg, rw + E * d, d);
    }
    std::vector<UpPiece> pieces;
    pieces.push_back({static_cast<const uint8_t *>(tgu.data), tgu.bytes, off_gu});
    pieces.push_back({static_cast<const uint8_t *>(tdn.data), tdn.bytes, off_dn});
    if (S > 0) {
        // shared gate_up rows: the gate_proj rows, then the up_proj rows
        pieces.push_back({static_cast<const uint8_t *>(tsg.data), tsg.bytes, off_sgu});
        pieces.push_back({static_cast<const uint8_t *>(tsu.data), tsu.bytes, off_sgu + tsg.bytes});
        pieces.push_back({static_cast<const uint8_t *>(tsd.data), tsd.bytes, off_sdn});
    }
    up_copy(host, pieces);
    hipStream_t us = ctx->up_stream;
    rc = hip_check(ctx, hipMemcpyAsync(dev, host, total, hipMemcpyHostToDevice, us), "upload copy");
    // `packed` may still be read by layers already queued on the compute
    // stream (a rotation that reuses packed buffers): the pack kernels that
    // overwrite it wait for that work; the copy above does not need to
    if (rc == RMDA_OK) {
        rc = hip_check(ctx, hipEventRecord(ctx->up_after, ctx->stream), "upload event");
    }
    if (rc == RMDA_OK) {
        rc = hip_check(ctx, hipStreamWaitEvent(us, ctx->up_after, 0), "upload wait for queued layers");
    }
    if (rc == RMDA_OK) {
        rc = pack_layer(ctx, us, shape, reinterpret_cast<const float *>(dev + off_r),
                        reinterpret_cast<const uint16_t *>(dev + off_gu), tgu.dtype == RMDA_ST_BF16,
                        reinterpret_cast<const uint16_t *>(dev + off_dn), tdn.dtype == RMDA_ST_BF16,
                        reinterpret_cast<const uint16_t *>(dev + off_sgu), tsg.dtype == RMDA_ST_BF16,
                        reinterpret_cast<const uint16_t *>(dev + off_sdn), tsd.dtype == RMDA_ST_BF16, packed);
    }
    if (rc == RMDA_OK) {
        rc = hip_check(ctx, hipEventRecord(ctx->up_done[bank], us), "upload event");
    }
    if (rc == RMDA_OK) {
        ctx->up_used[bank] = 1;
        ctx->up_seq += 1;
    }
    return rc;
}

int rmda_moe_upload_wait(rmda_moe_ctx_t *ctx) {
    int rc = enter(ctx);
    if (rc != RMDA_OK || !ctx->up_made || ctx->up_seq == 0) {
        return rc;
    }
    // uploads run in order on the upload stream: the last one covers all
    const uint32_t last = (ctx->up_seq - 1) % 2;
    return hip_check(ctx, hipStreamWaitEvent(ctx->stream, ctx->up_done[last], 0), "wait for uploads");
}

int rmda_moe_fill_normal_f16(rmda_moe_ctx_t *ctx, uint16_t *dst, size_t n, uint64_t stream, uint64_t seed,
                             float std) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (dst == nullptr && n > 0) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_fill_normal_f16: null dst");
    }
    return hip_check(ctx, rmda_launch_fill_normal(ctx->stream, dst, n, 1, stream, seed, std), "fill f16");
}

int rmda_moe_fill_normal_f32(rmda_moe_ctx_t *ctx, float *dst, size_t n, uint64_t stream, uint64_t seed,
                             float std) {
    int rc = enter(ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (dst == nullptr && n > 0) {
        return fail(ctx, RMDA_ERR_ARG, "rmda_moe_fill_normal_f32: null dst");
    }
    return hip_check(ctx, rmda_launch_fill_normal(ctx->stream, dst, n, 0, stream, seed, std), "fill f32");
}

}  // extern "C"

// ---- the qwen.c MoE recording over the stage entry points ----

namespace {

struct ShimPlan {
    size_t a16, p, idx, wt, count, off, fill, tiles, slot, xp, g, hp, hp16, ye;
    size_t gs, hs, hs16, sh, tiles1, amax, wr, total;
    uint32_t ps, rows_pad, mrows;
};

uint32_t qwen_moe_rows(uint32_t rows, uint32_t topk, uint32_t experts) {
    // mda_qwen_moe_rows, src/qwen.c:68-70
    const uint64_t m = (uint64_t)rows * topk + (uint64_t)experts * (RMDA_QWEN_TILE - 1);
    return (uint32_t)((m + RMDA_QWEN_TILE - 1) / RMDA_QWEN_TILE * RMDA_QWEN_TILE);
}

bool shim_ok(const rmda_qwen_moe_t *q) {
    return q != nullptr && q->d > 0 && q->d % 256 == 0 && q->experts > 0 && q->experts <= RMDA_MAX_EXPERTS &&
           q->topk > 0 && q->topk <= RMDA_MAX_TOPK && q->topk <= q->experts && q->inter > 0 &&
           q->inter % 128 == 0 && q->shared % 128 == 0 && q->max_rows > 0 &&
           (uint64_t)q->max_rows * q->topk <= RMDA_CTX_MAX_PAIRS && q->hc <= RMDA_MAX_HC;
}

// Scratch layout, as mda_qwen_scratch sizes its MoE buffers (src/qwen.c:166-179)
ShimPlan plan_shim(const rmda_qwen_moe_t *q) {
    ShimPlan p{};
    const uint32_t T = q->max_rows, d = q->d, E = q->experts, K = q->topk, I = q->inter, S = q->shared;
    p.ps = E + (S > 0 ? 1u : 0u);
    p.rows_pad = (T + RMDA_QWEN_TILE - 1) / RMDA_QWEN_TILE * RMDA_QWEN_TILE;
    p.mrows = qwen_moe_rows(T, K, E);
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = align256(o + bytes);
        return at;
    };
    p.a16 = take((size_t)p.rows_pad * d * 2);
    p.p = take((size_t)T * p.ps * 4);
    p.idx = take((size_t)T * K * 4);
    p.wt = take((size_t)T * K * 4);
    p.count = take((size_t)E * 4);
    p.off = take((size_t)E * 4);
    p.fill = take((size_t)E * 4);
    p.tiles = take((size_t)p.mrows / RMDA_QWEN_TILE * 4);
    p.slot = take((size_t)T * K * 4);
    p.xp = take((size_t)p.mrows * d * 2);
    p.g = take((size_t)p.mrows * 2 * I * 4);
    p.hp = take((size_t)p.mrows * I * 4);
    p.hp16 = take((size_t)p.mrows * I * 2);
    p.ye = take((size_t)p.mrows * d * 4);
    if (S > 0) {
        p.gs = take((size_t)p.rows_pad * 2 * S * 4);
        p.hs = take((size_t)p.rows_pad * S * 4);
        p.hs16 = take((size_t)p.rows_pad * S * 2);
        p.sh = take((size_t)p.rows_pad * d * 4);
        p.tiles1 = take((size_t)p.rows_pad / RMDA_QWEN_TILE * 4);
    }
    p.amax = take((size_t)RMDA_QWEN_MAX_SLOTS * 4);
    // the router matrix in the packed order of the fused layer's router
    // (repacked by every recording: 2 bytes of traffic per weight byte)
    p.wr = take((size_t)d * rmda_router_cpad(p.ps) * 4);
    p.total = o;
    return p;
}

template <typename T>
T *scr(const rmda_qwen_moe_t *q, size_t off) {
    return reinterpret_cast<T *>(static_cast<uint8_t *>(q->scratch) + off);
}

// entry guard of the shim: context, configuration and scratch
int shim_enter(rmda_qwen_moe_t *q, const char *who, ShimPlan *plan) {
    if (q == nullptr) {
        return RMDA_ERR_ARG;
    }
    int rc = enter(q->ctx);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (!shim_ok(q)) {
        return fail(q->ctx, RMDA_ERR_SHAPE, "%s: unsupported configuration", who);
    }
    if (q->w_router == nullptr || q->w_gate_up == nullptr || q->w_down == nullptr ||
        (q->shared > 0 && (q->w_sh_gate_up == nullptr || q->w_sh_down == nullptr))) {
        return fail(q->ctx, RMDA_ERR_ARG, "%s: missing weights", who);
    }
    *plan = plan_shim(q);
    if (q->scratch == nullptr || q->scratch_bytes < plan->total) {
        return fail(q->ctx, RMDA_ERR_WORKSPACE, "%s: scratch %zu bytes < %zu", who, q->scratch_bytes, plan->total);
    }
    return RMDA_OK;
}

// mda_qwen_slot (src/qwen.c:505-515)
uint32_t shim_slot(rmda_qwen_moe_t *q) {
    if (q->n_slots >= RMDA_QWEN_MAX_SLOTS) {
        fail(q->ctx, RMDA_ERR_SHAPE, "rmda_qwen_moe: out of fp16 scale slots");
        return RMDA_NO_SLOT;
    }
    return q->n_slots++;
}

// mda_qwen_cast (src/qwen.c:517-539): absmax into a new slot, then the cast
int shim_cast(rmda_qwen_moe_t *q, const ShimPlan &p, const float *src, uint16_t *dst, uint32_t n, uint32_t *slot) {
    *slot = shim_slot(q);
    if (*slot == RMDA_NO_SLOT) {
        return q->ctx->err;
    }
    uint32_t *amax = scr<uint32_t>(q, p.amax);
    const rmda_pc_absmax_t pa{n, *slot};
    int rc = rmda_absmax(q->ctx, &pa, src, amax);
    if (rc == RMDA_OK) {
        const rmda_pc_cast_t pc{n, *slot};
        rc = rmda_cast_f16(q->ctx, &pc, src, dst, amax);
    }
    return rc;
}

}  // namespace

size_t rmda_qwen_moe_scratch_bytes(const rmda_qwen_moe_t *q) {
    return shim_ok(q) ? plan_shim(q).total : 0;
}

int rmda_qwen_moe_layout(const rmda_qwen_moe_t *q, rmda_qwen_moe_layout_t *out) {
    if (out == nullptr || !shim_ok(q)) {
        return RMDA_ERR_ARG;
    }
    const ShimPlan p = plan_shim(q);
    out->p = p.p;
    out->idx = p.idx;
    out->wt = p.wt;
    out->count = p.count;
    out->off = p.off;
    out->slot = p.slot;
    out->xp = p.xp;
    out->amax = p.amax;
    out->hp = p.hp;
    out->hp16 = p.hp16;
    out->tiles = p.tiles;
    out->total = p.total;
    out->p_stride = p.ps;
    return RMDA_OK;
}

namespace {

// mda_qwen_moe_mm's work; live = true (the recording) leaves the padding
// rows of each segment out of the GEMM, since nothing reads their results
int qwen_moe_mm(rmda_qwen_moe_t *q, const uint16_t *a, uint32_t sa, const uint16_t *w, float *out, uint32_t m,
                uint32_t n, uint32_t k, bool live, mm_swiglu_t *swi = nullptr) {
    ShimPlan p;
    int rc = shim_enter(q, "rmda_qwen_moe_mm", &p);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (m > p.mrows) {
        return fail(q->ctx, RMDA_ERR_SHAPE, "rmda_qwen_moe_mm: m=%u beyond the scratch's %u rows", m, p.mrows);
    }
    const rmda_pc_moe_mm_t pc{m, n, k, sa, RMDA_NO_SLOT};
    return moe_mm(q->ctx, &pc, a, w, out, scr<uint32_t>(q, p.amax), scr<uint32_t>(q, p.tiles),
                  live ? scr<uint32_t>(q, p.off) : nullptr, live ? scr<uint32_t>(q, p.count) : nullptr, swi);
}

}  // namespace

int rmda_qwen_moe_mm(rmda_qwen_moe_t *q, const uint16_t *a, uint32_t sa, const uint16_t *w, float *out, uint32_t m,
                     uint32_t n, uint32_t k) {
    return qwen_moe_mm(q, a, sa, w, out, m, n, k, false);
}

namespace {

// mda_qwen_route_rec's work; zero_xp = false leaves xp's padding rows as
// they are, for the recording below, which reads no padding row's result
int route_rec(rmda_qwen_moe_t *q, uint32_t rows, uint32_t mrows, bool zero_xp) {
    ShimPlan p;
    int rc = shim_enter(q, "rmda_qwen_route_rec", &p);
    if (rc != RMDA_OK) {
        return rc;
    }
    if (rows > q->max_rows || mrows != qwen_moe_rows(rows, q->topk, q->experts)) {
        return fail(q->ctx, RMDA_ERR_SHAPE, "rmda_qwen_route_rec: rows=%u mrows=%u (max_rows %u)", rows, mrows,
                    q->max_rows);
    }
    if (rows == 0) {
        return RMDA_OK;
    }
    // the reference zero-fills xp (src/qwen.c:798); count, fill and the tile
    // map need no fill here (route overwrites count, scatter takes fill as
    // zero, scan writes every tile)
    if (zero_xp) {
        rc = hip_check(q->ctx, rmda_launch_zero(q->ctx->stream, scr<uint32_t>(q, p.xp), (size_t)mrows * q->d / 2, 0),
                       "route_rec xp fill");
        if (rc != RMDA_OK) {
            return rc;
        }
    }
    const rmda_pc_moe_route_t pr{rows, q->experts, q->topk, p.ps};
    rc = rmda_moe_route(q->ctx, &pr, scr<float>(q, p.p), scr<uint32_t>(q, p.idx), scr<float>(q, p.wt),
                        scr<uint32_t>(q, p.count));
    if (rc == RMDA_OK) {
        const rmda_pc_moe_scan_t ps{q->experts, RMDA_QWEN_TILE};
        rc = rmda_moe_scan(q->ctx, &ps, scr<uint32_t>(q, p.count), scr<uint32_t>(q, p.off),
                           scr<uint32_t>(q, p.tiles), mrows / RMDA_QWEN_TILE);
    }
    if (rc == RMDA_OK) {
        rc = rmda_moe_scatter_experts(q->ctx, q->experts);
    }
    if (rc == RMDA_OK) {
        const rmda_pc_moe_scatter_t pt{rows, q->topk, q->d / 8};
        rc = rmda_moe_scatter(q->ctx, &pt, scr<uint32_t>(q, p.idx), scr<uint32_t>(q, p.off),
                              scr<uint32_t>(q, p.fill), scr<uint16_t>(q, p.a16), scr<uint16_t>(q, p.xp),
                              scr<uint32_t>(q, p.slot));
    }
    return rc;
}

}  // namespace

int rmda_qwen_route_rec(rmda_qwen_moe_t *q, uint32_t rows, uint32_t mrows) {
    return route_rec(q, rows, mrows, true);
}

int rmda_qwen_moe_rec(rmda_qwen_moe_t *q, const float *x, const float *inj, float *h, uint16_t *out,
                      uint32_t rows) {
    ShimPlan p;
    int rc = shim_enter(q, "rmda_qwen_moe_rec", &p);
    if (rc != RMDA_OK) {
        return rc;
    }
    rmda_moe_ctx_t *c = q->ctx;
    if (rows > q->max_rows) {
        return fail(c, RMDA_ERR_SHAPE, "rmda_qwen_moe_rec: rows=%u > max_rows=%u", rows, q->max_rows);
    }
    if (x == nullptr || (h == nullptr && out == nullptr) || (h != nullptr && (inj == nullptr || q->hc == 0))) {
        return fail(c, RMDA_ERR_ARG, "rmda_qwen_moe_rec: x, and out or (h, inj, hc > 0), are required");
    }
    if (rows == 0) {
        return RMDA_OK;
    }
    const uint32_t d = q->d, E = q->experts, K = q->topk, I = q->inter, S = q->shared;
    const uint32_t mrows = qwen_moe_rows(rows, K, E);
    const uint32_t rows_pad = (rows + RMDA_QWEN_TILE - 1) / RMDA_QWEN_TILE * RMDA_QWEN_TILE;
    uint32_t *amax = scr<uint32_t>(q, p.amax);
    // mda_qwen_slots_begin (src/qwen.c:500-503)
    q->n_slots = 0;
    rc = hip_check(c, rmda_launch_zero(c->stream, amax, RMDA_QWEN_MAX_SLOTS, 0), "moe_rec slot fill");
    // A0: x cast with a slot (src/qwen.c:844); the fp32 router reads the same
    // cast and multiplies each chunk sum by the slot's inverse scale, which
    // for fp16-range activations gives the logits of x itself bit for bit
    // and keeps activations outside that range (subnormal or above 65504 as
    // fp16) at full precision
    uint32_t sx = RMDA_NO_SLOT;
    if (rc == RMDA_OK) {
        rc = shim_cast(q, p, x, scr<uint16_t>(q, p.a16), rows * d, &sx);
    }
    // the router projection on the router matrix repacked into the order the
    // router kernel streams (3.6 us for 128 x 2048 at config 3; the HF-layout
    // kernel takes about three times as long as the packed one), the same
    // logits bit for bit
    if (rc == RMDA_OK) {
        rc = hip_check(c, rmda_launch_router_pack(c->stream, q->w_router, scr<float>(q, p.wr), p.ps, d),
                       "moe_rec router pack");
    }
    if (rc == RMDA_OK) {
        rc = hip_check(c,
                       rmda_launch_router(c->stream, scr<uint16_t>(q, p.a16), scr<float>(q, p.wr), 1, nullptr,
                                          scr<float>(q, p.p), rows, d, p.ps, p.ps, 0, nullptr, 0, nullptr, amax + sx),
                       "moe_rec router");
    }
    // A1-A3 (xp's padding rows are not zero-filled: the GEMMs, SwiGLU,
    // absmax and cast below compute the routed rows only)
    if (rc == RMDA_OK) {
        rc = route_rec(q, rows, mrows, false);
    }
    // A4-A7: gate_up, SwiGLU, hp cast with a slot, down (src/qwen.c:847-878).
    // The reference's GEMMs also run every padding row of each 128-row
    // segment (xp's zero rows, a third of the used rows at T=2048, E=128,
    // top-8); their g and ye rows are never read, so these GEMMs skip them.
    // gate_up writes SwiGLU(g) and its absmax (hp's scale slot) from its
    // epilogue, the same values as qwen_elem then absmax on g, so g itself
    // never goes to memory (where the persistent kernel does not take the
    // shape, g is written and the pass below computes them)
    uint32_t sh = RMDA_NO_SLOT;
    if (rc == RMDA_OK) {
        sh = shim_slot(q);  // the slot qwen.c takes after gate_up: the same index
        rc = sh == RMDA_NO_SLOT ? c->err : RMDA_OK;
    }
    mm_swiglu_t swi{scr<float>(q, p.hp), sh, false};
    if (rc == RMDA_OK) {
        rc = qwen_moe_mm(q, scr<uint16_t>(q, p.xp), sx, q->w_gate_up, scr<float>(q, p.g), mrows, 2 * I, d, true,
                         &swi);
    }
    // over the rows that hold routed pairs only: in the reference the padding
    // rows of each 128-row segment are zero in g (xp's zero rows), so their
    // SwiGLU is 0 and leaves the absmax unchanged, and nothing after reads
    // their hp or ye
    const rmda_rowmask_t live{scr<uint32_t>(q, p.tiles), scr<uint32_t>(q, p.off), scr<uint32_t>(q, p.count),
                              RMDA_QWEN_TILE};
    if (rc == RMDA_OK && !swi.fused) {
        const rmda_pc_qwen_elem_t pe{mrows, I, 2 * I, 0, I, 0, 1.0f};
        rc = hip_check(c, rmda_launch_elem_absmax_rows(c->stream, &pe, scr<float>(q, p.g), scr<float>(q, p.hp), amax,
                                                       sh, &live),
                       "moe_rec swiglu");
    }
    if (rc == RMDA_OK) {
        rc = hip_check(c, rmda_launch_cast_rows(c->stream, mrows, I, scr<float>(q, p.hp), scr<uint16_t>(q, p.hp16),
                                                amax, sh, &live),
                       "moe_rec hp cast");
    }
    if (rc == RMDA_OK) {
        rc = qwen_moe_mm(q, scr<uint16_t>(q, p.hp16), sh, q->w_down, scr<float>(q, p.ye), mrows, d, I, true);
    }
    // A8: the shared expert as one-expert grouped GEMMs over the padded rows
    // (src/qwen.c:879-886); rows past `rows` hold stale data and are unused
    if (rc == RMDA_OK && S > 0) {
        uint32_t *t1 = scr<uint32_t>(q, p.tiles1);
        rc = hip_check(c, rmda_launch_zero(c->stream, t1, rows_pad / RMDA_QWEN_TILE, 0), "moe_rec shared tiles");
        if (rc == RMDA_OK) {
            const rmda_pc_moe_mm_t pm{rows_pad, 2 * S, d, sx, RMDA_NO_SLOT};
            rc = rmda_moe_mm(c, &pm, scr<uint16_t>(q, p.a16), q->w_sh_gate_up, scr<float>(q, p.gs), amax, t1);
        }
        // SwiGLU with the absmax of hs folded in, then the scaled cast (as
        // for the routed experts above)
        uint32_t ss = RMDA_NO_SLOT;
        if (rc == RMDA_OK) {
            ss = shim_slot(q);
            rc = ss == RMDA_NO_SLOT ? c->err : RMDA_OK;
        }
        if (rc == RMDA_OK) {
            const rmda_pc_qwen_elem_t pe{rows, S, 2 * S, 0, S, 0, 1.0f};
            rc = hip_check(c, rmda_launch_elem_absmax(c->stream, &pe, scr<float>(q, p.gs), scr<float>(q, p.hs), amax,
                                                      ss),
                           "moe_rec shared swiglu");
        }
        if (rc == RMDA_OK) {
            const rmda_pc_cast_t pc{rows * S, ss};
            rc = rmda_cast_f16(c, &pc, scr<float>(q, p.hs), scr<uint16_t>(q, p.hs16), amax);
        }
        if (rc == RMDA_OK) {
            const rmda_pc_moe_mm_t pm{rows_pad, d, S, ss, RMDA_NO_SLOT};
            rc = rmda_moe_mm(c, &pm, scr<uint16_t>(q, p.hs16), q->w_sh_down, scr<float>(q, p.sh), amax, t1);
        }
    }
    // A9: combine (src/qwen.c:887-906)
    if (rc == RMDA_OK) {
        const rmda_pc_moe_combine_t pm{rows, d, K, p.ps, E, q->inj_stride, q->hc_rank, q->hc};
        const float *shp = S > 0 ? scr<float>(q, p.sh) : nullptr;
        if (h != nullptr) {
            rc = rmda_moe_combine(c, &pm, scr<float>(q, p.wt), scr<uint32_t>(q, p.slot), scr<float>(q, p.ye),
                                  scr<float>(q, p.p), shp, inj, h);
        }
        if (rc == RMDA_OK && out != nullptr) {
            rc = rmda_moe_combine_plain(c, &pm, scr<float>(q, p.wt), scr<uint32_t>(q, p.slot),
                                        scr<float>(q, p.ye), scr<float>(q, p.p), shp, out);
        }
    }
    return rc;
}
