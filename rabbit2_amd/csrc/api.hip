// C-ABI of the MoE-layer path (include/rbt2_hip.h): handle, model upload, workspace, dispatch of
// the gfx950 kernels, and the int 1/0 + stderr error convention of the reference engine
// (rabbit2/src/rabbit2.c:199-228 for the header checks, :455 for the forward() contract).
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "rbt2_internal.h"

using namespace rbt;

namespace {

constexpr uint64_t kAlign = 4096;  // rabbit2.c:56
constexpr uint64_t kTAlign = 64;   // rabbit2.c:57
constexpr uint64_t kHeader = 68;   // rabbit2.c:58
constexpr int kMaxTopK = 64;       // rabbit2.c:59

char g_init_err[512];

struct LayerOff {
    uint64_t attn_norm, wq, wk, wv, wo, q_norm, k_norm, ffn_norm, router, experts;
};

enum ProfKernel { kProfRouter, kProfTopk, kProfGateup, kProfDown, kProfDispatch, kProfCombine, kProfCount };
const char *const kProfNames[kProfCount] = {"router", "topk", "gateup", "down_combine", "dispatch", "combine"};

struct Profile {
    bool on = false;
    hipEvent_t ev[kProfCount][2] = {};
    bool used[kProfCount] = {};
    double total_ms[kProfCount] = {};
    uint64_t launches[kProfCount] = {};
};

struct Workspace {
    int tokens = 0, E = 0, K = 0, H = 0;
    float *probs = nullptr;       // [T][E]
    int32_t *routing = nullptr;   // [T][K]
    float *weights = nullptr;     // [T][K]
    float *hbuf = nullptr;        // [T*K][H]
    uint8_t *pre = nullptr;       // grouped-path lists and down outputs (prefill_workspace_bytes)
    size_t pre_bytes = 0;
};

}  // namespace

struct rbt_hip {
    int device = 0;
    hipStream_t stream = nullptr;
    int order = RBT_ORDER_AVX2;
    char err[512] = {0};
    // uploaded model
    uint8_t *model = nullptr;
    uint64_t model_size = 0;
    rbt_config cfg{};
    uint64_t expert_stride = 0, tok_emb = 0, final_norm = 0, lm_head = 0, layout_end = 0;
    std::vector<LayerOff> layers;
    Workspace ws;
    Profile prof;
    int fused_decode = 1;  // option "fused_decode": batch-1 top-k inside the gate/up kernel
    int prefill_min_tokens = kPrefillMinTokensDefault;  // option "prefill_min_tokens"
    const int32_t *expert_counts = nullptr;  // histogram of the last grouped-path call
    // staging for the host-pointer entry points
    void *stage = nullptr;
    uint64_t stage_bytes = 0;
};

namespace {

int fail(rbt_hip *h, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (h)
        snprintf(h->err, sizeof h->err, "%s", buf);
    else
        snprintf(g_init_err, sizeof g_init_err, "%s", buf);
    fprintf(stderr, "rbt2_hip: %s\n", buf);
    return 0;
}

#define HIP_OK(h, call)                                                                         \
    do {                                                                                        \
        hipError_t e_ = (call);                                                                 \
        if (e_ != hipSuccess) return fail((h), "%s failed: %s", #call, hipGetErrorString(e_)); \
    } while (0)

int set_device(rbt_hip *h) {
    HIP_OK(h, hipSetDevice(h->device));
    return 1;
}

uint64_t align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

uint64_t take(uint64_t *off, uint64_t n) {
    *off = align_up(*off, kTAlign);
    const uint64_t at = *off;
    *off += n;
    return at;
}

// rabbit2.c:158-193
void compute_layout(rbt_hip *h) {
    const rbt_config &c = h->cfg;
    const uint64_t E = c.dtype == RBT_DT_BF16 ? 2 : 4, F = 4, D = (uint64_t)c.dim;
    const uint64_t qd = (uint64_t)c.n_heads * c.head_dim, kvd = (uint64_t)c.n_kv_heads * c.head_dim;
    uint64_t off = kAlign;
    h->tok_emb = take(&off, (uint64_t)c.vocab * D * E);
    h->expert_stride = align_up(3 * (uint64_t)c.expert_hidden * D * E, kAlign);
    h->layers.assign((size_t)c.n_layers, LayerOff{});
    for (int l = 0; l < c.n_layers; l++) {
        LayerOff &ly = h->layers[(size_t)l];
        ly.attn_norm = take(&off, D * F);
        ly.wq = take(&off, qd * D * E);
        ly.wk = take(&off, kvd * D * E);
        ly.wv = take(&off, kvd * D * E);
        ly.wo = take(&off, D * qd * E);
        if (c.qk_norm) {
            ly.q_norm = take(&off, qd * F);
            ly.k_norm = take(&off, kvd * F);
        }
        ly.ffn_norm = take(&off, D * F);
        ly.router = take(&off, (uint64_t)c.n_experts * D * E);
        off = align_up(off, kAlign);
        ly.experts = off;
        off += (uint64_t)c.n_experts * h->expert_stride;
    }
    h->final_norm = take(&off, D * F);
    h->lm_head = take(&off, (uint64_t)c.vocab * D * E);
    h->layout_end = h->lm_head + (uint64_t)c.vocab * D * E;
}

int check_layer(rbt_hip *h, const rbt_moe_layer *L) {
    if (!L) return fail(h, "moe: layer descriptor is NULL");
    if (L->dim <= 0 || L->n_experts <= 0 || L->expert_hidden <= 0 || L->top_k <= 0 || L->top_k > L->n_experts ||
        L->top_k > kMaxTopK)
        return fail(h, "moe: invalid shape (dim %d, n_experts %d, top_k %d, expert_hidden %d)", L->dim, L->n_experts,
                    L->top_k, L->expert_hidden);
    if (L->dtype != RBT_DT_F32 && L->dtype != RBT_DT_BF16) return fail(h, "moe: invalid dtype %d", L->dtype);
    if (!L->router || !L->experts) return fail(h, "moe: router/experts pointer is NULL");
    const uint64_t esz = L->dtype == RBT_DT_BF16 ? 2 : 4;
    if (L->expert_stride < 3ull * L->expert_hidden * L->dim * esz)
        return fail(h, "moe: expert_stride %llu smaller than one expert (%llu bytes)",
                    (unsigned long long)L->expert_stride, (unsigned long long)(3ull * L->expert_hidden * L->dim * esz));
    return 1;
}

void ws_release(Workspace &w) {
    (void)hipFree(w.probs);
    (void)hipFree(w.routing);
    (void)hipFree(w.weights);
    (void)hipFree(w.hbuf);
    (void)hipFree(w.pre);
    w = Workspace{};
}

// Grows the workspace to hold T tokens of this shape (never shrinks). Allocation happens only here.
int ws_reserve(rbt_hip *h, int T, int E, int K, int H) {
    Workspace &w = h->ws;
    if (T <= w.tokens && E <= w.E && K <= w.K && H <= w.H) return 1;
    const int nT = T > w.tokens ? T : w.tokens, nE = E > w.E ? E : w.E, nK = K > w.K ? K : w.K,
              nH = H > w.H ? H : w.H;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    ws_release(w);
    h->expert_counts = nullptr;
    HIP_OK(h, hipMalloc(&w.probs, sizeof(float) * (size_t)nT * nE));
    HIP_OK(h, hipMalloc(&w.routing, sizeof(int32_t) * (size_t)nT * nK));
    HIP_OK(h, hipMalloc(&w.weights, sizeof(float) * (size_t)nT * nK));
    HIP_OK(h, hipMalloc(&w.hbuf, sizeof(float) * (size_t)nT * nK * nH));
    w.tokens = nT;
    w.E = nE;
    w.K = nK;
    w.H = nH;
    return 1;
}

// Grows the grouped-path workspace (never shrinks).
int pre_reserve(rbt_hip *h, size_t bytes) {
    Workspace &w = h->ws;
    if (bytes <= w.pre_bytes) return 1;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    (void)hipFree(w.pre);
    w.pre = nullptr;
    w.pre_bytes = 0;
    h->expert_counts = nullptr;
    HIP_OK(h, hipMalloc(&w.pre, bytes));
    w.pre_bytes = bytes;
    return 1;
}

int stage_reserve(rbt_hip *h, uint64_t bytes) {
    if (bytes <= h->stage_bytes) return 1;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    (void)hipFree(h->stage);
    h->stage = nullptr;
    h->stage_bytes = 0;
    HIP_OK(h, hipMalloc(&h->stage, bytes));
    h->stage_bytes = bytes;
    return 1;
}

// The launch context of kernel k: the handle stream, plus (when profiling) the event pair that
// hipExtLaunchKernel stamps with that kernel's own start and end.
Launch lc(rbt_hip *h, int k) {
    Launch L;
    L.s = h->stream;
    if (h->prof.on && k >= 0) {
        L.start = h->prof.ev[k][0];
        L.stop = h->prof.ev[k][1];
        h->prof.used[k] = true;
    }
    return L;
}

// Waits for the call's events and adds each bracketed kernel's duration.
int prof_collect(rbt_hip *h) {
    if (!h->prof.on) return 1;
    for (int k = 0; k < kProfCount; k++) {
        if (!h->prof.used[k]) continue;
        HIP_OK(h, hipEventSynchronize(h->prof.ev[k][1]));
        float ms = 0.0f;
        HIP_OK(h, hipEventElapsedTime(&ms, h->prof.ev[k][0], h->prof.ev[k][1]));
        h->prof.total_ms[k] += ms;
        h->prof.launches[k] += 1;
        h->prof.used[k] = false;
    }
    return 1;
}

}  // namespace

extern "C" {

int rbt_hip_init(rbt_hip **out, int device) {
    if (!out) return fail(nullptr, "init: out is NULL");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(nullptr, "init: no HIP device (%s)", hipGetErrorString(e));
    if (device < 0 || device >= n) return fail(nullptr, "init: device %d out of range (have %d)", device, n);
    rbt_hip *h = new rbt_hip();
    h->device = device;
    e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        fail(nullptr, "init: %s", hipGetErrorString(e));
        delete h;
        return 0;
    }
    *out = h;
    return 1;
}

void rbt_hip_free(rbt_hip *h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    ws_release(h->ws);
    for (int k = 0; k < kProfCount; k++)
        for (int j = 0; j < 2; j++)
            if (h->prof.ev[k][j]) (void)hipEventDestroy(h->prof.ev[k][j]);
    (void)hipFree(h->stage);
    (void)hipFree(h->model);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
}

const char *rbt_hip_last_error(const rbt_hip *h) { return h ? h->err : g_init_err; }

int rbt_hip_set_router_order(rbt_hip *h, int order) {
    if (!h) return fail(nullptr, "set_router_order: handle is NULL");
    if (order != RBT_ORDER_SCALAR && order != RBT_ORDER_AVX2) return fail(h, "router order must be 0 or 1");
    h->order = order;
    return 1;
}

int rbt_hip_upload(rbt_hip *h, const void *file, uint64_t file_size, rbt_config *cfg) {
    if (!h) return fail(nullptr, "upload: handle is NULL");
    const unsigned char *d = static_cast<const unsigned char *>(file);
    if (!d || file_size < kHeader || memcmp(d, "RBT2", 4) != 0) return fail(h, "bad magic: not a .rbt2 file");
    uint32_t version;
    memcpy(&version, d + 4, 4);
    if (version != 2) return fail(h, "unsupported .rbt2 version %u (need 2)", version);
    rbt_config c;
    memcpy(&c, d + 8, sizeof c);
    if (c.vocab <= 0 || c.dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 ||
        c.n_experts <= 0 || c.expert_hidden <= 0 || c.max_seq <= 0 || c.top_k <= 0 || c.top_k > c.n_experts ||
        c.top_k > kMaxTopK || c.head_dim % 2 != 0 || c.n_heads % c.n_kv_heads != 0 ||
        (c.dtype != RBT_DT_F32 && c.dtype != RBT_DT_BF16))
        return fail(h, "invalid config in header");
    h->cfg = c;
    compute_layout(h);
    if (h->layout_end > file_size)
        return fail(h, "file too small for its own config (%llu < %llu)", (unsigned long long)file_size,
                    (unsigned long long)h->layout_end);
    if (!set_device(h)) return 0;
    if (h->model) {
        HIP_OK(h, hipStreamSynchronize(h->stream));
        (void)hipFree(h->model);
        h->model = nullptr;
    }
    HIP_OK(h, hipMalloc(&h->model, h->layout_end));
    HIP_OK(h, hipMemcpy(h->model, file, h->layout_end, hipMemcpyHostToDevice));
    h->model_size = h->layout_end;
    if (cfg) *cfg = c;
    return 1;
}

int rbt_hip_layer(rbt_hip *h, int layer, rbt_moe_layer *out) {
    if (!h || !out) return fail(h, "layer: NULL argument");
    if (!h->model) return fail(h, "layer: no model uploaded");
    if (layer < 0 || layer >= h->cfg.n_layers) return fail(h, "layer %d out of range", layer);
    const LayerOff &ly = h->layers[(size_t)layer];
    out->dim = h->cfg.dim;
    out->n_experts = h->cfg.n_experts;
    out->top_k = h->cfg.top_k;
    out->expert_hidden = h->cfg.expert_hidden;
    out->dtype = h->cfg.dtype;
    out->norm_topk = h->cfg.norm_topk;
    out->router = h->model + ly.router;
    out->experts = h->model + ly.experts;
    out->expert_stride = h->expert_stride;
    out->router_bias = nullptr;
    return 1;
}

int rbt_hip_reserve(rbt_hip *h, const rbt_moe_layer *L, int max_tokens) {
    if (!h) return fail(nullptr, "reserve: handle is NULL");
    if (!check_layer(h, L) || !set_device(h)) return 0;
    if (max_tokens < 0) return fail(h, "reserve: negative token count");
    const int T = max_tokens > 0 ? max_tokens : 1;
    if (!ws_reserve(h, T, L->n_experts, L->top_k, L->expert_hidden)) return 0;
    if (T >= h->prefill_min_tokens)
        return pre_reserve(h, prefill_workspace_bytes(T, L->n_experts, L->top_k, L->dim));
    return 1;
}

int rbt_hip_moe_dev(rbt_hip *h, const rbt_moe_layer *L, const float *xb_dev, int T, float *x_dev, float *moe_dev,
                    int32_t *routing_dev, float *weights_dev) {
    if (!h) return fail(nullptr, "moe: handle is NULL");
    if (T < 0) return fail(h, "moe: negative token count");
    if (!check_layer(h, L)) return 0;
    if (T == 0) return 1;
    if (!xb_dev) return fail(h, "moe: xb is NULL");
    if (!set_device(h)) return 0;
    if (!ws_reserve(h, T, L->n_experts, L->top_k, L->expert_hidden)) return 0;
    Workspace &w = h->ws;
    int32_t *routing = routing_dev ? routing_dev : w.routing;
    float *weights = weights_dev ? weights_dev : w.weights;
    const bool decode_kernels = experts_decode_supported(L->dtype, T, L->top_k, L->dim, L->expert_hidden, L->experts,
                                                         L->expert_stride, xb_dev, w.hbuf);
    if (decode_kernels && h->fused_decode && T == 1 && L->n_experts <= kTopkInGateupMaxE) {
        // batch 1: router logits, then gate/up (with the top-k in every block), then down + combine
        HIP_OK(h, launch_router_logits(lc(h, kProfRouter), h->order, L->dtype, xb_dev, L->router, L->router_bias, T,
                                       L->n_experts, L->dim, w.probs));
        HIP_OK(h, launch_experts_decode(lc(h, kProfGateup), lc(h, kProfDown), L->dtype, L->experts, L->expert_stride,
                                        routing, weights, xb_dev, w.hbuf, T, L->top_k, L->dim, L->expert_hidden, x_dev,
                                        moe_dev, w.probs, L->n_experts, L->norm_topk));
        return prof_collect(h);
    }
    if (prefill_supported(L->dtype, T, h->prefill_min_tokens, L->n_experts, L->top_k, L->dim, L->expert_hidden,
                          L->experts, L->expert_stride, xb_dev)) {
        if (!pre_reserve(h, prefill_workspace_bytes(T, L->n_experts, L->top_k, L->dim))) return 0;
        // router, top-k and the activation split in one launch when it applies, else the two router
        // kernels (the grouped path then splits the activations itself)
        const bool fused = router_prefill_supported(h->order, L->dtype, T, L->n_experts, L->dim, L->top_k,
                                                    L->router, xb_dev);
        if (fused) {
            uint16_t *x_hi = nullptr, *x_lo = nullptr;
            prefill_x_planes(w.pre, T, L->n_experts, L->top_k, L->dim, &x_hi, &x_lo);
            HIP_OK(h, launch_router_prefill(lc(h, kProfRouter), L->dtype, xb_dev, L->router, L->router_bias, T,
                                            L->n_experts, L->dim, L->top_k, L->norm_topk, routing, weights, x_hi,
                                            x_lo));
        } else {
            HIP_OK(h, launch_router(lc(h, kProfRouter), lc(h, kProfTopk), h->order, L->dtype, xb_dev, L->router,
                                    L->router_bias, T, L->n_experts, L->dim, L->top_k, L->norm_topk, w.probs,
                                    routing, weights));
        }
        int32_t *counts = nullptr;
        HIP_OK(h, launch_prefill(lc(h, kProfDispatch), lc(h, kProfGateup), lc(h, kProfDown), lc(h, kProfCombine),
                                 L->experts, L->expert_stride, xb_dev, T, L->n_experts, L->top_k, L->dim,
                                 L->expert_hidden, routing, weights, w.hbuf, w.pre, x_dev, moe_dev, &counts, fused));
        h->expert_counts = counts;
        return prof_collect(h);
    }
    HIP_OK(h, launch_router(lc(h, kProfRouter), lc(h, kProfTopk), h->order, L->dtype, xb_dev, L->router,
                            L->router_bias, T, L->n_experts, L->dim, L->top_k, L->norm_topk, w.probs, routing,
                            weights));
    if (decode_kernels) {
        HIP_OK(h, launch_experts_decode(lc(h, kProfGateup), lc(h, kProfDown), L->dtype, L->experts, L->expert_stride,
                                        routing, weights, xb_dev, w.hbuf, T, L->top_k, L->dim, L->expert_hidden, x_dev,
                                        moe_dev, nullptr, L->n_experts, L->norm_topk));
    } else {
        HIP_OK(h, launch_gateup_gemv(lc(h, kProfGateup), L->dtype, L->experts, L->expert_stride, routing, xb_dev, T,
                                     L->top_k, L->dim, L->expert_hidden, w.hbuf));
        HIP_OK(h, launch_down_combine(lc(h, kProfDown), L->dtype, L->experts, L->expert_stride, routing, weights,
                                      w.hbuf, T, L->top_k, L->dim, L->expert_hidden, x_dev, moe_dev));
    }
    return prof_collect(h);
}

const int32_t *rbt_hip_expert_counts_dev(rbt_hip *h) { return h ? h->expert_counts : nullptr; }

int rbt_hip_moe(rbt_hip *h, int layer, const float *xb, int T, float *x_inout, int32_t *routing_out) {
    if (!h) return fail(nullptr, "moe: handle is NULL");
    rbt_moe_layer L;
    if (!rbt_hip_layer(h, layer, &L)) return 0;
    if (T < 0) return fail(h, "moe: negative token count");
    if (T == 0) return 1;
    if (!xb) return fail(h, "moe: xb is NULL");
    const uint64_t nx = (uint64_t)T * L.dim, nr = (uint64_t)T * L.top_k;
    const uint64_t xb_off = 0, x_off = align_up(nx * 4, 256), r_off = x_off + align_up(nx * 4, 256);
    if (!set_device(h) || !stage_reserve(h, r_off + nr * 4)) return 0;
    uint8_t *st = static_cast<uint8_t *>(h->stage);
    float *xb_d = reinterpret_cast<float *>(st + xb_off);
    float *x_d = x_inout ? reinterpret_cast<float *>(st + x_off) : nullptr;
    int32_t *r_d = reinterpret_cast<int32_t *>(st + r_off);
    HIP_OK(h, hipMemcpyAsync(xb_d, xb, nx * 4, hipMemcpyHostToDevice, h->stream));
    if (x_d) HIP_OK(h, hipMemcpyAsync(x_d, x_inout, nx * 4, hipMemcpyHostToDevice, h->stream));
    if (!rbt_hip_moe_dev(h, &L, xb_d, T, x_d, nullptr, r_d, nullptr)) return 0;
    if (x_d) HIP_OK(h, hipMemcpyAsync(x_inout, x_d, nx * 4, hipMemcpyDeviceToHost, h->stream));
    if (routing_out) HIP_OK(h, hipMemcpyAsync(routing_out, r_d, nr * 4, hipMemcpyDeviceToHost, h->stream));
    HIP_OK(h, hipStreamSynchronize(h->stream));
    return 1;
}

int rbt_hip_matvec_dev(rbt_hip *h, float *out_dev, const void *W_dev, int dtype, const float *x_dev, int rows,
                       int cols) {
    if (!h) return fail(nullptr, "matvec: handle is NULL");
    if (rows < 0 || cols <= 0) return fail(h, "matvec: invalid shape %d x %d", rows, cols);
    if (dtype != RBT_DT_F32 && dtype != RBT_DT_BF16) return fail(h, "matvec: invalid dtype %d", dtype);
    if (rows == 0) return 1;
    if (!out_dev || !W_dev || !x_dev) return fail(h, "matvec: NULL pointer");
    if (!set_device(h)) return 0;
    HIP_OK(h, launch_matvec(lc(h, -1), dtype, W_dev, x_dev, out_dev, rows, cols));
    return 1;
}

int rbt_hip_matvec(rbt_hip *h, float *out, uint64_t w_offset, const float *x, int rows, int cols) {
    if (!h) return fail(nullptr, "matvec: handle is NULL");
    if (!h->model) return fail(h, "matvec: no model uploaded");
    if (rows < 0 || cols <= 0) return fail(h, "matvec: invalid shape %d x %d", rows, cols);
    const uint64_t esz = h->cfg.dtype == RBT_DT_BF16 ? 2 : 4;
    if (w_offset > h->model_size || (uint64_t)rows * cols * esz > h->model_size - w_offset)
        return fail(h, "matvec: weights [%llu, +%llu) outside the uploaded model", (unsigned long long)w_offset,
                    (unsigned long long)((uint64_t)rows * cols * esz));
    if (rows == 0) return 1;
    if (!out || !x) return fail(h, "matvec: NULL pointer");
    const uint64_t o_off = align_up((uint64_t)cols * 4, 256);
    if (!set_device(h) || !stage_reserve(h, o_off + (uint64_t)rows * 4)) return 0;
    uint8_t *st = static_cast<uint8_t *>(h->stage);
    float *x_d = reinterpret_cast<float *>(st), *o_d = reinterpret_cast<float *>(st + o_off);
    HIP_OK(h, hipMemcpyAsync(x_d, x, (uint64_t)cols * 4, hipMemcpyHostToDevice, h->stream));
    HIP_OK(h, launch_matvec(lc(h, -1), h->cfg.dtype, h->model + w_offset, x_d, o_d, rows, cols));
    HIP_OK(h, hipMemcpyAsync(out, o_d, (uint64_t)rows * 4, hipMemcpyDeviceToHost, h->stream));
    HIP_OK(h, hipStreamSynchronize(h->stream));
    return 1;
}

int rbt_hip_malloc(rbt_hip *h, void **dev, uint64_t bytes) {
    if (!h || !dev) return fail(h, "malloc: NULL argument");
    *dev = nullptr;
    if (!set_device(h)) return 0;
    HIP_OK(h, hipMalloc(dev, bytes ? bytes : 1));
    return 1;
}

int rbt_hip_free_dev(rbt_hip *h, void *dev) {
    if (!h) return fail(nullptr, "free_dev: handle is NULL");
    if (!dev) return 1;
    if (!set_device(h)) return 0;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    HIP_OK(h, hipFree(dev));
    return 1;
}

int rbt_hip_h2d(rbt_hip *h, void *dst_dev, const void *src, uint64_t bytes) {
    if (!h) return fail(nullptr, "h2d: handle is NULL");
    if (!bytes) return 1;
    if (!dst_dev || !src) return fail(h, "h2d: NULL pointer");
    if (!set_device(h)) return 0;
    HIP_OK(h, hipMemcpyAsync(dst_dev, src, bytes, hipMemcpyHostToDevice, h->stream));
    HIP_OK(h, hipStreamSynchronize(h->stream));
    return 1;
}

int rbt_hip_d2h(rbt_hip *h, void *dst, const void *src_dev, uint64_t bytes) {
    if (!h) return fail(nullptr, "d2h: handle is NULL");
    if (!bytes) return 1;
    if (!dst || !src_dev) return fail(h, "d2h: NULL pointer");
    if (!set_device(h)) return 0;
    HIP_OK(h, hipMemcpyAsync(dst, src_dev, bytes, hipMemcpyDeviceToHost, h->stream));
    HIP_OK(h, hipStreamSynchronize(h->stream));
    return 1;
}

int rbt_hip_memset_dev(rbt_hip *h, void *dst_dev, int value, uint64_t bytes) {
    if (!h) return fail(nullptr, "memset: handle is NULL");
    if (!bytes) return 1;
    if (!dst_dev) return fail(h, "memset: NULL pointer");
    if (!set_device(h)) return 0;
    HIP_OK(h, hipMemsetAsync(dst_dev, value, bytes, h->stream));
    return 1;
}

int rbt_hip_synchronize(rbt_hip *h) {
    if (!h) return fail(nullptr, "synchronize: handle is NULL");
    if (!set_device(h)) return 0;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    return 1;
}

int rbt_hip_set_option(rbt_hip *h, const char *name, int64_t value) {
    if (!h || !name) return fail(h, "set_option: NULL argument");
    if (strcmp(name, "fused_decode") == 0) {
        h->fused_decode = value != 0;
    } else if (strcmp(name, "prefill_min_tokens") == 0) {
        if (value < 1 || value > 65536) return fail(h, "set_option: prefill_min_tokens must be in [1, 65536]");
        h->prefill_min_tokens = (int)value;
    } else {
        return fail(h, "set_option: unknown option '%s'", name);
    }
    return 1;
}

void *rbt_hip_stream(rbt_hip *h) { return h ? static_cast<void *>(h->stream) : nullptr; }

int rbt_hip_profile_enable(rbt_hip *h, int on) {
    if (!h) return fail(nullptr, "profile: handle is NULL");
    if (!set_device(h)) return 0;
    if (on && !h->prof.ev[0][0]) {
        for (int k = 0; k < kProfCount; k++)
            for (int j = 0; j < 2; j++) HIP_OK(h, hipEventCreate(&h->prof.ev[k][j]));
    }
    if (on) {
        for (int k = 0; k < kProfCount; k++) {
            h->prof.total_ms[k] = 0.0;
            h->prof.launches[k] = 0;
            h->prof.used[k] = false;
        }
    }
    h->prof.on = on != 0;
    return 1;
}

int rbt_hip_profile_get(rbt_hip *h, const char *kernel, double *total_ms, uint64_t *launches) {
    if (!h || !kernel) return fail(h, "profile_get: NULL argument");
    for (int k = 0; k < kProfCount; k++) {
        if (strcmp(kernel, kProfNames[k]) == 0) {
            if (total_ms) *total_ms = h->prof.total_ms[k];
            if (launches) *launches = h->prof.launches[k];
            return 1;
        }
    }
    return fail(h, "profile_get: unknown kernel name '%s'", kernel);
}

int rbt_hip_fill_normal(rbt_hip *h, void *dst_dev, int dtype, uint64_t n, uint64_t seed, uint64_t stream,
                        uint64_t first, float scale, float offset) {
    if (!h) return fail(nullptr, "fill_normal: handle is NULL");
    if (dtype != RBT_DT_F32 && dtype != RBT_DT_BF16) return fail(h, "fill_normal: invalid dtype %d", dtype);
    if (!n) return 1;
    if (!dst_dev) return fail(h, "fill_normal: NULL pointer");
    if (!set_device(h)) return 0;
    HIP_OK(h, launch_fill_normal(lc(h, -1), dst_dev, dtype, n, seed, stream, first, scale, offset));
    return 1;
}

}  // extern "C"
