// C-ABI of the MoE-layer path (include/rbt2_hip.h): handle, model upload, workspace, dispatch of
// the gfx950 kernels, and the int 1/0 + stderr error convention of the reference engine
// (rabbit2/src/rabbit2.c:199-228 for the header checks, :455 for the forward() contract).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <new>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "rbt2_internal.h"

using namespace rbt;

static __device__ __align__(256) uint8_t scratch[64u << 20];  // see kScratchBytes

namespace {

constexpr uint64_t kAlign = 4096;  // rabbit2.c:56
constexpr uint64_t kTAlign = 64;   // rabbit2.c:57
constexpr uint64_t kHeader = 68;   // rabbit2.c:58
constexpr int kMaxTopK = 64;       // rabbit2.c:59
// Largest device image rbt_hip_model_create lays out (no file bounds it); hipMalloc decides below it.
constexpr uint64_t kMaxImageBytes = 1ull << 50;

char g_init_err[512];

// Scratch of rbt_hip_moe_dev_noalloc: one array per GPU, for callers that cannot allocate. 64 MiB holds
// the workspace of a 512-token call at the OLMoE layer shape (52.2 MiB). Host code never uses the
// array's name as an address: rbt_hip_init looks up each device's own copy (hipGetSymbolAddress) once,
// with that device current, and every launch takes that address.
constexpr size_t kScratchBytes = 64u << 20;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

struct LayerOff {
    uint64_t attn_norm, wq, wk, wv, wo, q_norm, k_norm, ffn_norm, router, experts;
};

enum ProfKernel {
    kProfRouter, kProfTopk, kProfGateup, kProfDown, kProfDispatch, kProfCombine,
    // the rest of the forward pass (rbt_hip_forward with profiling on)
    kProfEmbed, kProfAttnNorm, kProfQkv, kProfAttn, kProfAttnMerge, kProfWo, kProfFfnNorm, kProfLmHead, kProfArgmax,
    kProfCount
};
const char *const kProfNames[kProfCount] = {"router", "topk", "gateup", "down_combine", "dispatch", "combine",
                                            "embed", "attn_norm", "qkv", "attention", "attn_merge", "wo", "ffn_norm",
                                            "lm_head", "argmax"};

// mode 1: one event pair per kernel kind, read after every call (each call waits for its work).
// mode 2 (deferred): every launch takes the next pair of a per-kind pool and nothing waits, so the
// timed calls run back to back as in a decode loop; the pairs taken are read (and the pool reused) when
// a synchronous call has waited for its work anyway, by rbt_hip_profile_get, or when a kind has
// kProfPoolMax pairs out. (HIP graphs do not time events, so neither mode is meant for stream capture.)
constexpr size_t kProfPoolMax = 4096;  // pairs per kind in mode 2 before a wait
struct Profile {
    int mode = 0;
    hipEvent_t ev[kProfCount][2] = {};
    bool used[kProfCount] = {};
    double total_ms[kProfCount] = {};
    uint64_t launches[kProfCount] = {};
    std::vector<hipEvent_t> pool[kProfCount];  // mode 2: pairs (2i, 2i + 1)
    size_t next[kProfCount] = {};              // mode 2: pairs taken and not yet read
};

// Decode state of the full forward pass (rbt_hip_state_init): one allocation carved into the KV cache
// and the per-step buffers.
struct DecodeState {
    int n_seq = 0;                // sequences stepped together (1 for the engine's single State)
    int ctx = 0, S = 0;           // context length, attention splits
    uint8_t *block = nullptr;     // the allocation
    float *kc = nullptr, *vc = nullptr;  // [n_seq][n_layers][ctx][kv_dim]
    float *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *ao = nullptr;
    float *part = nullptr;        // attention split partials [n_heads][S][hd + 2]
    uint16_t *xh = nullptr, *xl = nullptr;  // bf16 hi/lo matrix-core planes of n_seq rows of max(dim, q_dim)
    float2 *rope_cs = nullptr;    // [ctx][hd/2] (cos, sin) of the RoPE angles
    float2 *cand = nullptr;       // lm_head blocks' argmax candidates
    float *sprob = nullptr;       // sampler scratch [n_seq][vocab]
    int32_t *sidx = nullptr;      // sampler scratch [n_seq][vocab]
    float *logits = nullptr;      // [vocab]
    int32_t *routing = nullptr;   // [n_layers][n_seq][top_k]
    int32_t *seq = nullptr;       // [n_seq][ctx] token of each position
    StepState *st = nullptr;      // [n_seq]
};

// A tiled copy of one layer's experts (launch_prefill_layout), taken from the blobs at `experts`.
struct TiledLayer {
    const void *experts = nullptr;
    uint64_t stride = 0;
    int E = 0, D = 0, H = 0;
    void *buf = nullptr;
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
    DecodeState ds;
    Profile prof;
    int fused_decode = 1;  // option "fused_decode": batch-1 top-k inside the gate/up kernel
    int batch_mfma = 1;    // option "batch_mfma": batched dense matvecs on the matrix cores
    Sampling sampling;     // rbt_hip_set_sampling: how rbt_hip_generate* pick tokens
    uint64_t seed = 0;
    int prefill_min_tokens = kPrefillMinTokensDefault;  // option "prefill_min_tokens"
    int prefill_tile_rows = 0;  // option "prefill_tile_rows": rows per grouped-GEMM tile, 0 = by batch
    bool prefill_wide = true;   // option "prefill_wide": 128-row tiles 512 weight rows wide
    int gen_timed_from = 1;     // option "generate_timed_from": first generated step of ms_out[1]
    const int32_t *expert_counts = nullptr;  // histogram of the last grouped-path call
    // staging for the host-pointer entry points: device buffer and its pinned host twin
    void *stage = nullptr;
    uint64_t stage_bytes = 0;
    void *pin = nullptr;
    uint64_t pin_bytes = 0;
    // option "routing_history": every forward step also records its routing per sequence and position
    // (rbt_hip_routing_history), allocated with the decode state
    int routing_history = 0;
    int32_t *rhist = nullptr;  // [n_seq][ctx][n_layers][top_k]
    // pinned host ring the streaming generate reads tokens from
    int32_t *tok_host = nullptr;
    int tok_host_n = 0;
    // this device's scratch array (rbt_hip_moe_dev_noalloc), from hipGetSymbolAddress at init
    void *scratch = nullptr;
    // tiled copies of layers' experts for the 128-row grouped GEMMs (rbt_hip_prefill_layout), keyed by
    // the layer's expert blobs; built only when the caller asks, used while option "prefill_layout" is on
    std::vector<TiledLayer> tiled;
    int prefill_layout = 1;
    // expert residency counters in the engine's cache-stats terms (rabbit2.c:745-751): every expert is
    // read from the file once at upload (a miss) and every later use of a selected expert is a hit
    uint64_t cache_hits = 0, cache_misses = 0;
};

namespace {

// Host-side fault injection for the failure-path tests: RBT_HIP_FAULT="<kind>:<n>" makes the n-th
// (1-based; ":<n>" may be left out for the first) HIP call of that kind in this process report an
// error without making the call. Kinds: malloc (hipMalloc, hipHostMalloc), launch (kernel launches),
// copy (hipMemcpy*), sync (stream and event waits). Unset, nothing is injected. The device never sees
// an injected fault: the call that would have failed is simply not made.
struct FaultPlan {
    int kind = -1;  // 0 malloc, 1 launch, 2 copy, 3 sync; -1 none
    long nth = 1;
    long seen = 0;
    FaultPlan() {
        const char *v = getenv("RBT_HIP_FAULT");
        if (!v || !*v) return;
        static const char *const kinds[4] = {"malloc", "launch", "copy", "sync"};
        for (int k = 0; k < 4; k++) {
            const size_t n = strlen(kinds[k]);
            if (strncmp(v, kinds[k], n) == 0 && (v[n] == 0 || v[n] == ':')) {
                kind = k;
                if (v[n] == ':') nth = strtol(v + n + 1, nullptr, 10);
            }
        }
    }
};

int fault_kind(const char *call) {
    while (*call == '(' || *call == ' ') call++;  // launch macros pass their call parenthesised
    if (strstr(call, "hipMalloc") || strstr(call, "hipHostMalloc")) return 0;
    if (strncmp(call, "launch_", 7) == 0) return 1;
    if (strstr(call, "hipMemcpy")) return 2;
    if (strstr(call, "Synchronize")) return 3;
    return -1;
}

hipError_t fault_point(const char *call) {
    static FaultPlan plan;  // read once per process
    if (plan.kind < 0 || fault_kind(call) != plan.kind) return hipSuccess;
    if (++plan.seen != plan.nth) return hipSuccess;
    static const hipError_t err[4] = {hipErrorOutOfMemory, hipErrorLaunchFailure, hipErrorInvalidValue,
                                      hipErrorLaunchFailure};
    fprintf(stderr, "rbt2_hip: RBT_HIP_FAULT: injecting a failure into %.60s\n", call);
    return err[plan.kind];
}

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
        hipError_t e_ = fault_point(#call);                                                     \
        if (e_ == hipSuccess) e_ = (call);                                                      \
        if (e_ != hipSuccess) return fail((h), "%s failed: %s", #call, hipGetErrorString(e_)); \
    } while (0)

// A HIP call whose error the caller handles itself, with the same fault injection point; the text of
// the last such call that failed is kept for the caller's message (failed_call()).
thread_local const char *g_failed_call = "";
hipError_t note_call(hipError_t e, const char *call) {
    if (e != hipSuccess) g_failed_call = call;
    return e;
}
const char *failed_call() { return g_failed_call; }
#define HIP_TRY(call)                                                      \
    ([&]() -> hipError_t {                                                 \
        const hipError_t f_ = fault_point(#call);                          \
        return note_call(f_ != hipSuccess ? f_ : (call), #call);           \
    }())

int set_device(rbt_hip *h) {
    HIP_OK(h, hipSetDevice(h->device));
    return 1;
}

uint64_t align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

// The layout arithmetic runs in 128 bits: header fields are int32, so products such as vocab * dim *
// 4 can pass 2^64, and an offset that would wrap must still compare as "past the end of the file".
typedef unsigned __int128 u128;
u128 align_up128(u128 x, u128 a) { return (x + a - 1) / a * a; }
u128 take128(u128 *off, u128 n) {
    *off = align_up128(*off, kTAlign);
    const u128 at = *off;
    *off += n;
    return at;
}
uint64_t sat64(u128 v) { return v > (u128)UINT64_MAX ? UINT64_MAX : (uint64_t)v; }

// The offsets of one layer that starts at `off` (rabbit2.c:175-190); returns the offset past its
// experts (4 KiB aligned).
u128 layer_offsets(const rbt_config &c, u128 off, u128 stride, LayerOff *ly) {
    const u128 E = c.dtype == RBT_DT_BF16 ? 2 : 4, F = 4, D = (u128)c.dim;
    const u128 qd = (u128)c.n_heads * c.head_dim, kvd = (u128)c.n_kv_heads * c.head_dim;
    LayerOff o{};
    o.attn_norm = (uint64_t)take128(&off, D * F);
    o.wq = (uint64_t)take128(&off, qd * D * E);
    o.wk = (uint64_t)take128(&off, kvd * D * E);
    o.wv = (uint64_t)take128(&off, kvd * D * E);
    o.wo = (uint64_t)take128(&off, D * qd * E);
    if (c.qk_norm) {
        o.q_norm = (uint64_t)take128(&off, qd * F);
        o.k_norm = (uint64_t)take128(&off, kvd * F);
    }
    o.ffn_norm = (uint64_t)take128(&off, D * F);
    o.router = (uint64_t)take128(&off, (u128)c.n_experts * D * E);
    off = align_up128(off, kAlign);
    o.experts = (uint64_t)off;
    off += (u128)c.n_experts * stride;
    if (ly) *ly = o;
    return off;
}

// The file layout of a config (rabbit2.c:158-193), computed apart from any handle so that a rejected
// header leaves the handle's model untouched.
struct ModelLayout {
    rbt_config cfg{};
    uint64_t expert_stride = 0, tok_emb = 0, final_norm = 0, lm_head = 0, layout_end = 0;
    std::vector<LayerOff> layers;
};

// Fills *m for config c when its image ends at or before `limit` bytes; returns 0 (with *end_out =
// the image end, saturated to 2^64 - 1) otherwise, before allocating anything per layer, and -1 when
// the host cannot hold the per-layer table. Layers after
// the first start 4 KiB aligned (the previous experts end so), so all of them have the first aligned
// layer's size and the end has a closed form; every layer holds at least one 4 KiB expert stride, so
// a layout that fits has at most limit / 4096 layers.
int layout_of(const rbt_config &c, uint64_t limit, ModelLayout *m, uint64_t *end_out) {
    const u128 E = c.dtype == RBT_DT_BF16 ? 2 : 4, F = 4, D = (u128)c.dim;
    const u128 stride = align_up128(3 * (u128)c.expert_hidden * D * E, kAlign);
    u128 off = kAlign;
    const u128 tok_emb = take128(&off, (u128)c.vocab * D * E);
    const u128 after0 = layer_offsets(c, off, stride, nullptr);
    const u128 per_layer = layer_offsets(c, after0, stride, nullptr) - after0;
    u128 end_layers = after0 + (u128)(c.n_layers - 1) * per_layer;
    const u128 final_norm = take128(&end_layers, D * F);
    const u128 lm_head = take128(&end_layers, (u128)c.vocab * D * E);
    const u128 end = lm_head + (u128)c.vocab * D * E;
    if (end_out) *end_out = sat64(end);
    if (end > (u128)limit) return 0;
    m->cfg = c;
    m->expert_stride = (uint64_t)stride;
    m->tok_emb = (uint64_t)tok_emb;
    m->final_norm = (uint64_t)final_norm;
    m->lm_head = (uint64_t)lm_head;
    m->layout_end = (uint64_t)end;
    try {
        m->layers.assign((size_t)c.n_layers, LayerOff{});
    } catch (const std::bad_alloc &) {
        m->layers.clear();
        return -1;
    }
    u128 at = off;
    for (int l = 0; l < c.n_layers; l++) at = layer_offsets(c, at, stride, &m->layers[(size_t)l]);
    return 1;
}

// Makes a validated layout the handle's own (the device image must already hold it).
void adopt_layout(rbt_hip *h, ModelLayout &&m) {
    h->cfg = m.cfg;
    h->expert_stride = m.expert_stride;
    h->tok_emb = m.tok_emb;
    h->final_norm = m.final_norm;
    h->lm_head = m.lm_head;
    h->layout_end = m.layout_end;
    h->layers = std::move(m.layers);
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

// The pinned host twin of the stage (copies from and to it run asynchronously at full rate).
int pin_reserve(rbt_hip *h, uint64_t bytes) {
    if (bytes <= h->pin_bytes) return 1;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    if (h->pin) (void)hipHostFree(h->pin);
    h->pin = nullptr;
    h->pin_bytes = 0;
    HIP_OK(h, hipHostMalloc(&h->pin, bytes, hipHostMallocDefault));
    h->pin_bytes = bytes;
    return 1;
}

int prof_harvest(rbt_hip *h);

// The launch context of kernel k: the handle stream, plus (when profiling) the event pair that
// hipExtLaunchKernel stamps with that kernel's own start and end.
Launch lc(rbt_hip *h, int k) {
    Launch L;
    L.s = h->stream;
    Profile &P = h->prof;
    if (P.mode == 1 && k >= 0) {
        L.start = P.ev[k][0];
        L.stop = P.ev[k][1];
        P.used[k] = true;
    } else if (P.mode == 2 && k >= 0) {
        if (P.next[k] == kProfPoolMax && !prof_harvest(h)) return L;  // this launch goes untimed
        std::vector<hipEvent_t> &pool = P.pool[k];
        while (pool.size() < 2 * (P.next[k] + 1)) {
            hipEvent_t ev = nullptr;
            if (hipEventCreate(&ev) != hipSuccess) return L;  // out of events: this launch goes untimed
            pool.push_back(ev);
        }
        L.start = pool[2 * P.next[k]];
        L.stop = pool[2 * P.next[k] + 1];
        P.next[k]++;
    }
    return L;
}

Launch lc_timed(rbt_hip *h, int k) { return lc(h, k); }

// Mode 2: waits for the stream and adds the durations of every pair taken since the last read, which
// frees the pools for reuse.
int prof_harvest(rbt_hip *h) {
    Profile &P = h->prof;
    if (P.mode != 2) return 1;
    bool any = false;
    for (int k = 0; k < kProfCount; k++) any = any || P.next[k] > 0;
    if (!any) return 1;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    for (int k = 0; k < kProfCount; k++) {
        for (size_t i = 0; i < P.next[k]; i++) {
            float ms = 0.0f;
            HIP_OK(h, hipEventElapsedTime(&ms, P.pool[k][2 * i], P.pool[k][2 * i + 1]));
            P.total_ms[k] += ms;
        }
        P.launches[k] += P.next[k];
        P.next[k] = 0;
    }
    return 1;
}

// Mode 1: waits for the call's events and adds each bracketed kernel's duration.
int prof_collect(rbt_hip *h) {
    if (h->prof.mode != 1) return 1;
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

// the header checks of load_model (rabbit2.c:199-228)
bool config_ok(const rbt_config &c) {
    return !(c.vocab <= 0 || c.dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 ||
             c.n_experts <= 0 || c.expert_hidden <= 0 || c.max_seq <= 0 || c.top_k <= 0 || c.top_k > c.n_experts ||
             c.top_k > kMaxTopK || c.head_dim % 2 != 0 || c.n_heads % c.n_kv_heads != 0 ||
             (c.dtype != RBT_DT_F32 && c.dtype != RBT_DT_BF16));
}

// The header checks of load_model (rabbit2.c:199-228) on the first bytes of a file of file_size
// bytes: magic, version 2, a valid config, and a file at least as long as its own layout. On success
// *m holds the file's layout; nothing else is touched (errors go to err_h, which may be NULL).
int parse_header(ModelLayout *m, const unsigned char *d, uint64_t file_size, rbt_hip *err_h) {
    if (!d || file_size < kHeader || memcmp(d, "RBT2", 4) != 0) return fail(err_h, "bad magic: not a .rbt2 file");
    uint32_t version;
    memcpy(&version, d + 4, 4);
    if (version != 2) return fail(err_h, "unsupported .rbt2 version %u (need 2)", version);
    rbt_config c;
    memcpy(&c, d + 8, sizeof c);
    if (!config_ok(c)) return fail(err_h, "invalid config in header");
    uint64_t end = 0;
    const int r = layout_of(c, file_size, m, &end);
    if (r < 0) return fail(err_h, "no host memory for the layout of %d layers", c.n_layers);
    if (!r)
        return fail(err_h, "file too small for its own config (%llu < %llu)", (unsigned long long)file_size,
                    (unsigned long long)end);
    return 1;
}

// The tiled copy registered for layer L's experts, or nullptr (none, option off, other shape).
const void *tiled_for(const rbt_hip *h, const rbt_moe_layer *L) {
    if (!h->prefill_layout || L->dtype != RBT_DT_BF16) return nullptr;
    for (const TiledLayer &t : h->tiled)
        if (t.experts == L->experts && t.stride == L->expert_stride && t.E == L->n_experts && t.D == L->dim &&
            t.H == L->expert_hidden)
            return t.buf;
    return nullptr;
}

// Frees the tiled copies whose blobs lie in [lo, hi) (all of them for lo = hi = nullptr). The stream
// is idle: callers synchronise first.
void tiled_drop(rbt_hip *h, const uint8_t *lo, const uint8_t *hi) {
    std::vector<TiledLayer> keep;
    for (TiledLayer &t : h->tiled) {
        const uint8_t *p = static_cast<const uint8_t *>(t.experts);
        if (lo == nullptr || (p >= lo && p < hi))
            (void)hipFree(t.buf);
        else
            keep.push_back(t);
    }
    h->tiled.swap(keep);
}

// Retakes, asynchronously on the handle stream after the write that called it, every tiled copy whose
// blobs overlap the device bytes [dst, dst + bytes) that a library call has just written (rbt_hip_h2d,
// rbt_hip_memset_dev, rbt_hip_fill_normal): only the experts the write touched, in place, so later
// calls and graphs captured earlier read the new weights.
int tiled_follow_write(rbt_hip *h, const void *dst, uint64_t bytes) {
    const uint8_t *lo = static_cast<const uint8_t *>(dst);
    for (const TiledLayer &t : h->tiled) {
        const uint8_t *b = static_cast<const uint8_t *>(t.experts);
        const uint64_t span = (uint64_t)t.E * t.stride;
        if (lo >= b + span || lo + bytes <= b) continue;
        const uint64_t first = lo > b ? (uint64_t)(lo - b) : 0;
        const uint64_t last = std::min<uint64_t>(span, (uint64_t)(lo + bytes - b)) - 1;
        const int e0 = (int)(first / t.stride), e1 = (int)(last / t.stride) + 1;
        Launch Lx;
        Lx.s = h->stream;
        HIP_OK(h, launch_prefill_layout(Lx, b + (uint64_t)e0 * t.stride, t.stride, e1 - e0, t.D, t.H,
                                        static_cast<uint8_t *>(t.buf) + (uint64_t)e0 * prefill_layout_bytes(1, t.D, t.H)));
    }
    return 1;
}

// Builds (or rebuilds in place) the tiled copy of layer L's experts, asynchronously on the handle stream.
int tiled_build(rbt_hip *h, const rbt_moe_layer *L) {
    if (L->dtype != RBT_DT_BF16 || !prefill_layout_supported(L->dtype, L->dim, L->expert_hidden))
        return fail(h, "prefill_layout: no tiled layout for dtype %d, dim %d, expert_hidden %d (bf16, dim a "
                       "multiple of 256 and expert_hidden of 256)", L->dtype, L->dim, L->expert_hidden);
    if (!L->experts || L->n_experts < 1 || L->expert_stride % 16 != 0 ||
        (reinterpret_cast<uintptr_t>(L->experts) & 15u))
        return fail(h, "prefill_layout: bad layer (experts NULL or not 16-byte aligned)");
    TiledLayer *t = nullptr;
    for (TiledLayer &x : h->tiled)
        if (x.experts == L->experts) t = &x;
    if (t && (t->stride != L->expert_stride || t->E != L->n_experts || t->D != L->dim || t->H != L->expert_hidden)) {
        HIP_OK(h, hipStreamSynchronize(h->stream));
        (void)hipFree(t->buf);
        t->buf = nullptr;
    }
    if (!t) {
        h->tiled.push_back(TiledLayer{});
        t = &h->tiled.back();
        t->experts = L->experts;
    }
    t->stride = L->expert_stride;
    t->E = L->n_experts;
    t->D = L->dim;
    t->H = L->expert_hidden;
    if (!t->buf) {
        const hipError_t e = HIP_TRY(hipMalloc(&t->buf, prefill_layout_bytes(t->E, t->D, t->H)));
        if (e != hipSuccess) {
            h->tiled.erase(h->tiled.begin() + (t - h->tiled.data()));  // keep no entry without a copy
            return fail(h, "prefill_layout: hipMalloc of %llu bytes failed: %s",
                        (unsigned long long)prefill_layout_bytes(L->n_experts, L->dim, L->expert_hidden),
                        hipGetErrorString(e));
        }
    }
    Launch Lx;
    Lx.s = h->stream;
    HIP_OK(h, launch_prefill_layout(Lx, L->experts, L->expert_stride, L->n_experts, L->dim, L->expert_hidden, t->buf));
    return 1;
}

// Drops the handle's model image and decode state (the workspace stays: it depends on shapes only).
// Afterwards the handle holds no model until a new layout is adopted with its image.
int model_drop(rbt_hip *h) {
    if (!set_device(h)) return 0;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    (void)hipFree(h->ds.block);
    h->ds = DecodeState{};
    (void)hipFree(h->rhist);
    h->rhist = nullptr;
    if (h->model) {
        tiled_drop(h, h->model, h->model + h->model_size);
        (void)hipFree(h->model);
    }
    h->model = nullptr;
    h->model_size = 0;
    h->cfg = rbt_config{};
    h->layers.clear();
    h->expert_stride = h->tok_emb = h->final_norm = h->lm_head = h->layout_end = 0;
    return 1;
}

// Replaces the handle's model with a fresh device image of layout m (contents left to the caller).
// On failure the handle holds no model.
int model_alloc(rbt_hip *h, const ModelLayout &m) {
    if (!model_drop(h)) return 0;
    void *p = nullptr;
    HIP_OK(h, hipMalloc(&p, m.layout_end));
    h->model = static_cast<uint8_t *>(p);
    h->model_size = m.layout_end;
    // a copy keyed inside fresh memory belongs to blobs freed earlier (the stream is idle: model_drop)
    tiled_drop(h, h->model, h->model + h->model_size);
    return 1;
}

// ---- full forward pass: one step = forward(seq[pos], pos) (rabbit2.c:453-548) on the decode state.
// final: the final norm, lm_head and argmax (which appends the token past the prompt and advances pos);
// otherwise only pos advances. Everything is enqueued on the handle stream, nothing waits, so a step
// can be captured into a graph.
// The MoE block of the batched forward for 2..kRouterDecodeMaxT tokens on the grouped expert path: the
// RMSNorm and the router logits in one launch (router_decode_kernel<M, true>, E / 2 or E / 4 x T blocks: xb and
// the logits), top-k + the activation split, then dispatch, the grouped GEMMs and the combine into x
// (rabbit2.c:512-542 for each token).
int moe_grouped_norm(rbt_hip *h, const rbt_moe_layer *L, const float *nw, float eps, int T, float *x, float *xb,
                     int32_t *routing, const float *next_nw, uint16_t *next_hi, uint16_t *next_lo) {
    if (!ws_reserve(h, T, L->n_experts, L->top_k, L->expert_hidden)) return 0;
    if (!pre_reserve(h, prefill_workspace_bytes(T, L->n_experts, L->top_k, L->dim))) return 0;
    Workspace &w = h->ws;
    uint16_t *x_hi = nullptr, *x_lo = nullptr;
    prefill_x_planes(w.pre, T, L->n_experts, L->top_k, L->dim, &x_hi, &x_lo);
    HIP_OK(h, launch_router_norm(lc(h, kProfRouter), x, nw, eps, L->router, L->router_bias, T, L->n_experts, L->dim,
                                 w.probs, xb));
    HIP_OK(h, launch_topk_split(lc(h, kProfTopk), w.probs, T, L->n_experts, L->top_k, L->norm_topk, xb, L->dim, routing,
                                w.weights, x_hi, x_lo));
    int32_t *counts = nullptr;
    // the combine's event pair is taken only by the launch that runs it (launch_prefill's combine, or
    // the fused combine + RMSNorm below), so a deferred-profile pair is never left unrecorded
    Launch no_combine;
    no_combine.s = h->stream;
    HIP_OK(h, launch_prefill(lc(h, kProfDispatch), lc(h, kProfGateup), lc(h, kProfDown),
                             next_nw ? no_combine : lc(h, kProfCombine), L->experts, L->expert_stride, xb, T,
                             L->n_experts, L->top_k, L->dim, L->expert_hidden, routing, w.weights, w.hbuf, w.pre, x,
                             nullptr, &counts, true, next_nw == nullptr, h->prefill_tile_rows, tiled_for(h, L),
                             h->prefill_wide));
    h->expert_counts = counts;
    if (next_nw) {  // the combine, fused with the RMSNorm the next step starts with (xb and its planes)
        const float *y = nullptr;
        const int32_t *pos_of = nullptr;
        prefill_combine_inputs(w.pre, T, L->n_experts, L->top_k, L->dim, &y, &pos_of);
        HIP_OK(h, launch_combine_rmsnorm(lc(h, kProfCombine), y, pos_of, w.weights, L->top_k, T, L->dim, x, next_nw,
                                         eps, xb, next_hi, next_lo));
    }
    return prof_collect(h);
}

// Whether the batched step's q/k/v of layer l (and its lm_head) run on the matrix cores behind an
// RMSNorm launch that writes the planes (the branches of enqueue_step below).
bool qkv_mfma(const rbt_hip *h, int l, int B) {
    const rbt_config &c = h->cfg;
    const LayerOff &ly = h->layers[(size_t)l];
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    const void *W[3] = {h->model + ly.wq, h->model + ly.wk, h->model + ly.wv};
    const int rows[3] = {qd, kvd, kvd};
    return B > 1 && dense_supported(c.dtype, c.dim, W, rows) && h->batch_mfma &&
           dense_mfma_supported(c.dtype, B, c.dim, W, rows);
}
bool lm_head_mfma(const rbt_hip *h, int B) {
    const rbt_config &c = h->cfg;
    const void *W[3] = {h->model + h->lm_head, nullptr, nullptr};
    const int rows[3] = {c.vocab, 0, 0};
    return B > 1 && dense_supported(c.dtype, c.dim, W, rows) && h->batch_mfma &&
           dense_mfma_supported(c.dtype, B, c.dim, W, rows);
}

int enqueue_step(rbt_hip *h, bool final) {
    const rbt_config &c = h->cfg;
    DecodeState &ds = h->ds;
    const int B = ds.n_seq;
    const int D = c.dim, hd = c.head_dim, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
    // with profiling on (eager calls only), every launch is timed by its own event pair and collected
    // right away, since each kernel kind runs once per layer
#define STEP_LAUNCH(k, call)                  \
    do {                                      \
        const Launch L = lc(h, (k));          \
        HIP_OK(h, (call));                    \
        if (!prof_collect(h)) return 0;       \
    } while (0)
    STEP_LAUNCH(kProfEmbed, launch_embed(L, c.dtype, h->model + h->tok_emb, D, c.vocab, ds.st, ds.seq, ds.ctx, ds.x, B));
    bool xb_ready = false;  // the previous MoE block's combine already wrote xb and its planes
    for (int l = 0; l < c.n_layers; l++) {
        const bool have_xb = xb_ready;  // for this layer's q/k/v only
        xb_ready = false;
        const LayerOff &ly = h->layers[(size_t)l];
        const void *W[3] = {h->model + ly.wq, h->model + ly.wk, h->model + ly.wv};
        float *const out[3] = {ds.q, ds.k, ds.v};
        const int rows[3] = {qd, kvd, kvd};
        const float *attn_norm = reinterpret_cast<const float *>(h->model + ly.attn_norm);
        const bool dense = dense_supported(c.dtype, D, W, rows);
        if (B == 1 && dense) {
            STEP_LAUNCH(kProfQkv, launch_dense_norm(L, c.dtype, ds.x, attn_norm, c.rms_eps, D, W, out, rows));
        } else if (qkv_mfma(h, l, B)) {
            // batched on the matrix cores: the norm also writes the bf16 hi/lo planes of xb
            if (!have_xb)
                STEP_LAUNCH(kProfAttnNorm, launch_rmsnorm(L, ds.x, attn_norm, D, c.rms_eps, ds.xb, B, ds.xh, ds.xl));
            STEP_LAUNCH(kProfQkv, launch_dense_mfma(L, ds.xh, ds.xl, B, D, W, out, rows, nullptr));
        } else if (dense) {  // batched: the norm once per token, then every weight read once for all tokens
            STEP_LAUNCH(kProfAttnNorm, launch_rmsnorm(L, ds.x, attn_norm, D, c.rms_eps, ds.xb, B));
            STEP_LAUNCH(kProfQkv, launch_dense_batch(L, c.dtype, ds.xb, B, D, W, out, rows, nullptr));
        } else {
            for (int b = 0; b < B; b++) {
                float *const ob[3] = {ds.q + (size_t)b * qd, ds.k + (size_t)b * kvd, ds.v + (size_t)b * kvd};
                STEP_LAUNCH(kProfQkv, launch_norm_matvec(L, c.dtype, ds.x + (size_t)b * D, attn_norm, c.rms_eps, D,
                                                         W, ob, rows));
            }
        }
        const void *Wo[3] = {h->model + ly.wo, nullptr, nullptr};
        float *const no_out[3] = {nullptr, nullptr, nullptr};
        const int wo_rows[3] = {D, 0, 0};
        const bool wo_mfma = B > 1 && h->batch_mfma && dense_mfma_supported(c.dtype, B, qd, Wo, wo_rows);
        const bool direct = ds.S == 1;  // one split: the attention kernel writes ao (and the planes) itself
        const size_t cache = (size_t)l * ds.ctx * kvd, seq_stride = (size_t)c.n_layers * ds.ctx * kvd;
        STEP_LAUNCH(kProfAttn,
                    launch_attention(L, ds.q, ds.k, ds.v,
                                     c.qk_norm ? reinterpret_cast<const float *>(h->model + ly.q_norm) : ds.q,
                                     c.qk_norm ? reinterpret_cast<const float *>(h->model + ly.k_norm) : ds.k,
                                     c.qk_norm, c.rms_eps, c.n_heads, c.n_kv_heads, hd, ds.S, ds.st, ds.kc + cache,
                                     ds.vc + cache, seq_stride, ds.rope_cs, ds.part, B, direct ? ds.ao : nullptr,
                                     direct && wo_mfma ? ds.xh : nullptr, direct && wo_mfma ? ds.xl : nullptr));
        if (!direct)
            STEP_LAUNCH(kProfAttnMerge, launch_attn_merge(L, ds.part, c.n_heads, hd, ds.S, ds.ao, B,
                                                          wo_mfma ? ds.xh : nullptr, wo_mfma ? ds.xl : nullptr));
        if (wo_mfma) {
            STEP_LAUNCH(kProfWo, launch_dense_mfma(L, ds.xh, ds.xl, B, qd, Wo, no_out, wo_rows, ds.x));
        } else if (dense_supported(c.dtype, qd, Wo, wo_rows)) {
            if (B == 1)
                STEP_LAUNCH(kProfWo, launch_dense_resid(L, c.dtype, ds.ao, qd, h->model + ly.wo, D, ds.x));
            else
                STEP_LAUNCH(kProfWo, launch_dense_batch(L, c.dtype, ds.ao, B, qd, Wo, no_out, wo_rows, ds.x));
        } else {
            for (int b = 0; b < B; b++)
                STEP_LAUNCH(kProfWo, launch_wo(L, c.dtype, ds.ao + (size_t)b * qd, qd, h->model + ly.wo, D,
                                               ds.x + (size_t)b * D));
        }
        rbt_moe_layer ml;
        if (!rbt_hip_layer(h, l, &ml)) return 0;
        const float *ffn_norm = reinterpret_cast<const float *>(h->model + ly.ffn_norm);
        Workspace &w = h->ws;
        int32_t *routing = ds.routing + (size_t)l * B * c.top_k;
        if (B == 1 && h->fused_decode && c.n_experts <= kTopkInGateupMaxE &&
            experts_decode_supported(c.dtype, 1, c.top_k, D, c.expert_hidden, ml.experts, ml.expert_stride, ds.xb,
                                     w.hbuf) &&
            router_norm_supported(h->order, c.dtype, 1, D, ml.router, ds.x, ffn_norm)) {
            // the MoE block in three launches with the RMSNorm inside the router kernel (it also writes xb)
            STEP_LAUNCH(kProfRouter, launch_router_norm(L, ds.x, ffn_norm, c.rms_eps, ml.router, nullptr, 1,
                                                        c.n_experts, D, w.probs, ds.xb));
            HIP_OK(h, launch_experts_decode(lc(h, kProfGateup), lc(h, kProfDown), c.dtype, ml.experts,
                                            ml.expert_stride, routing, w.weights, ds.xb, w.hbuf, 1, c.top_k, D,
                                            c.expert_hidden, ds.x, nullptr, w.probs, c.n_experts, c.norm_topk));
            if (!prof_collect(h)) return 0;
        } else if (B > 1 && B <= kRouterDecodeMaxT && c.n_experts <= 64 &&
                   router_norm_supported(h->order, c.dtype, B, D, ml.router, ds.x, ffn_norm) &&
                   prefill_supported(c.dtype, B, h->prefill_min_tokens, c.n_experts, c.top_k, D, c.expert_hidden,
                                     ml.experts, ml.expert_stride, ds.xb)) {
            // the next step's first RMSNorm (next layer's q/k/v, or the lm_head) fused into the combine
            const float *next_nw = nullptr;
            const bool fusable = c.top_k <= 8 && D <= 4096;  // launch_combine_rmsnorm's limits
            if (fusable && l + 1 < c.n_layers && qkv_mfma(h, l + 1, B))
                next_nw = reinterpret_cast<const float *>(h->model + h->layers[(size_t)l + 1].attn_norm);
            else if (fusable && l + 1 == c.n_layers && final && lm_head_mfma(h, B))
                next_nw = reinterpret_cast<const float *>(h->model + h->final_norm);
            if (!moe_grouped_norm(h, &ml, ffn_norm, c.rms_eps, B, ds.x, ds.xb, routing, next_nw,
                                  next_nw ? ds.xh : nullptr, next_nw ? ds.xl : nullptr))
                return 0;
            xb_ready = next_nw != nullptr;
        } else {
            STEP_LAUNCH(kProfFfnNorm, launch_rmsnorm(L, ds.x, ffn_norm, D, c.rms_eps, ds.xb, B));
            if (!rbt_hip_moe_dev(h, &ml, ds.xb, B, ds.x, nullptr, routing, nullptr)) return 0;
        }
    }
    if (h->rhist)  // the step's routing into each sequence's history, at the position not yet advanced
        STEP_LAUNCH(-1, launch_record_routing(L, ds.st, ds.routing, c.n_layers, c.top_k, B, ds.ctx, h->rhist));
    if (final) {
        const void *W[3] = {h->model + h->lm_head, nullptr, nullptr};
        float *const out[3] = {ds.logits, nullptr, nullptr};
        const int rows[3] = {c.vocab, 0, 0};
        const float *fn = reinterpret_cast<const float *>(h->model + h->final_norm);
        const bool dense = dense_supported(c.dtype, D, W, rows);
        const bool sample = h->sampling.temperature > 0.0f;
        if (B == 1 && dense && !sample) {  // lm_head with per-block argmax candidates, then the argmax
            STEP_LAUNCH(kProfLmHead, launch_dense_argmax(L, c.dtype, ds.x, fn, c.rms_eps, D, W[0], c.vocab, ds.logits,
                                                         ds.cand, ds.st, ds.seq, ds.ctx));
        } else {
            if (dense && B == 1) {
                STEP_LAUNCH(kProfLmHead, launch_dense_norm(L, c.dtype, ds.x, fn, c.rms_eps, D, W, out, rows));
            } else if (lm_head_mfma(h, B)) {
                if (!xb_ready)
                    STEP_LAUNCH(kProfAttnNorm, launch_rmsnorm(L, ds.x, fn, D, c.rms_eps, ds.xb, B, ds.xh, ds.xl));
                STEP_LAUNCH(kProfLmHead, launch_dense_mfma(L, ds.xh, ds.xl, B, D, W, out, rows, nullptr));
            } else if (dense) {
                STEP_LAUNCH(kProfAttnNorm, launch_rmsnorm(L, ds.x, fn, D, c.rms_eps, ds.xb, B));
                STEP_LAUNCH(kProfLmHead, launch_dense_batch(L, c.dtype, ds.xb, B, D, W, out, rows, nullptr));
            } else {
                for (int b = 0; b < B; b++) {
                    float *const ob[3] = {ds.logits + (size_t)b * c.vocab, nullptr, nullptr};
                    STEP_LAUNCH(kProfLmHead, launch_norm_matvec(L, c.dtype, ds.x + (size_t)b * D, fn, c.rms_eps, D, W,
                                                                ob, rows));
                }
            }
            if (sample)
                STEP_LAUNCH(kProfArgmax, launch_sample(L, ds.logits, c.vocab, h->sampling, ds.sprob, ds.sidx, ds.st,
                                                       ds.seq, ds.ctx, B));
            else
                STEP_LAUNCH(kProfArgmax, launch_argmax(L, ds.logits, c.vocab, ds.st, ds.seq, ds.ctx, B));
        }
    } else {
        STEP_LAUNCH(-1, launch_advance(L, ds.st, B));
    }
#undef STEP_LAUNCH
    return 1;
}

// The environment variable through which a ROCm profiler tool announces itself to this process, or
// nullptr. rocprofv3's launcher exports ROCPROFILER_LIBRARY_CTOR and ROCPROF_OUTPUT_PATH to the program
// it starts; the older rocprof tools load through HSA_TOOLS_LIB / ROCP_TOOL_LIB.
const char *profiler_var() {
    static const char *const vars[] = {"ROCPROFILER_LIBRARY_CTOR", "ROCPROF_OUTPUT_PATH", "HSA_TOOLS_LIB",
                                       "ROCP_TOOL_LIB"};
    for (const char *v : vars) {
        const char *val = getenv(v);
        if (val && *val) return v;
    }
    return nullptr;
}

// Captures `n` enqueued steps of one kind into an executable graph. Graph replay is refused while a
// profiler tool is attached: replays traced by rocprofv3 have ended in a host SIGSEGV inside the
// tool's interception of hipGraphLaunch, so a profiled run must take the eager paths.
int capture_step(rbt_hip *h, bool final, hipGraphExec_t *exec) {
    if (const char *v = profiler_var())
        return fail(h, "HIP graph replay is off while a profiler tool is attached (%s is set): profile the "
                       "eager calls (rbt_hip_forward, rbt_hip_forward_batch, rbt_hip_moe_dev) instead", v);
    hipGraph_t g = nullptr;
    HIP_OK(h, hipStreamBeginCapture(h->stream, hipStreamCaptureModeRelaxed));
    const int ok = enqueue_step(h, final);
    const hipError_t e = hipStreamEndCapture(h->stream, &g);
    if (!ok) {
        if (g) (void)hipGraphDestroy(g);
        return 0;
    }
    if (e != hipSuccess) return fail(h, "hipStreamEndCapture failed: %s", hipGetErrorString(e));
    const hipError_t e2 = hipGraphInstantiate(exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e2 != hipSuccess) return fail(h, "hipGraphInstantiate failed: %s", hipGetErrorString(e2));
    return 1;
}

// The form the MoE block takes for a call: the batch-1 kernels with the top-k inside gate/up, the
// grouped GEMM path, or the per-pair GEMVs. (Both workspaces give the h buffer 256-byte alignment, so
// the decode kernels' alignment test sees xb's, which it also checks.)
enum MoeForm { kMoeFastDecode, kMoeGrouped, kMoeGeneral };
MoeForm moe_form(const rbt_hip *h, const rbt_moe_layer *L, int T, const float *xb) {
    if (T == 1 && h->fused_decode && L->n_experts <= kTopkInGateupMaxE &&
        experts_decode_supported(L->dtype, T, L->top_k, L->dim, L->expert_hidden, L->experts, L->expert_stride, xb,
                                 xb))
        return kMoeFastDecode;
    if (prefill_supported(L->dtype, T, h->prefill_min_tokens, L->n_experts, L->top_k, L->dim, L->expert_hidden,
                          L->experts, L->expert_stride, xb))
        return kMoeGrouped;
    return kMoeGeneral;
}

size_t up256(size_t b) { return (b + 255) / 256 * 256; }

// Scratch bytes of one MoE call: probs [T][E], routing and weights [T][K], hbuf [T*K][H], and the
// grouped path's lists, down outputs and activation planes.
size_t moe_scratch_bytes(int T, int E, int K, int H, int D, bool grouped) {
    const size_t t = (size_t)T;
    return up256(4 * t * E) + 2 * up256(4 * t * K) + up256(4 * t * K * H) +
           (grouped ? prefill_workspace_bytes(T, E, K, D) : 0);
}

// A workspace view of the scratch array (device address `base`), in moe_scratch_bytes' order.
Workspace scratch_view(void *base, int T, int E, int K, int H, int D, bool grouped) {
    uint8_t *p = static_cast<uint8_t *>(base);
    const size_t t = (size_t)T;
    Workspace w;
    w.tokens = T;
    w.E = E;
    w.K = K;
    w.H = H;
    w.probs = reinterpret_cast<float *>(p);
    p += up256(4 * t * E);
    w.routing = reinterpret_cast<int32_t *>(p);
    p += up256(4 * t * K);
    w.weights = reinterpret_cast<float *>(p);
    p += up256(4 * t * K);
    w.hbuf = reinterpret_cast<float *>(p);
    p += up256(4 * t * K * H);
    w.pre = grouped ? p : nullptr;
    w.pre_bytes = grouped ? prefill_workspace_bytes(T, E, K, D) : 0;
    return w;
}

// The MoE block (rabbit2.c:513-542) on a workspace w sized for this call by the caller: probs, routing,
// weights, hbuf, and for the grouped form pre. timed: launches take profiling events (the handle
// workspace path); the scratch path takes none.
int moe_block(rbt_hip *h, const rbt_moe_layer *L, const float *xb_dev, int T, float *x_dev, float *moe_dev,
              int32_t *routing_dev, float *weights_dev, Workspace &w, MoeForm form, bool timed) {
    auto lc = [timed](rbt_hip *hh, int k) {
        if (timed) return lc_timed(hh, k);
        Launch plain;
        plain.s = hh->stream;
        return plain;
    };
    int32_t *routing = routing_dev ? routing_dev : w.routing;
    float *weights = weights_dev ? weights_dev : w.weights;
    const bool decode_kernels = experts_decode_supported(L->dtype, T, L->top_k, L->dim, L->expert_hidden, L->experts,
                                                         L->expert_stride, xb_dev, w.hbuf);
    auto done = [&]() { return timed ? prof_collect(h) : 1; };
    if (form == kMoeFastDecode) {
        // batch 1: router logits, then gate/up (with the top-k in every block), then down + combine
        HIP_OK(h, launch_router_logits(lc(h, kProfRouter), h->order, L->dtype, xb_dev, L->router, L->router_bias, T,
                                       L->n_experts, L->dim, w.probs));
        HIP_OK(h, launch_experts_decode(lc(h, kProfGateup), lc(h, kProfDown), L->dtype, L->experts, L->expert_stride,
                                        routing, weights, xb_dev, w.hbuf, T, L->top_k, L->dim, L->expert_hidden, x_dev,
                                        moe_dev, w.probs, L->n_experts, L->norm_topk));
        return done();
    }
    if (form == kMoeGrouped) {
        // router, top-k and the activation split in one launch when it applies, else the two router
        // kernels (the grouped path then splits the activations itself)
        const bool fused = router_prefill_supported(h->order, L->dtype, T, L->n_experts, L->dim, L->top_k,
                                                    L->router, xb_dev);
        if (fused && T <= kRouterDecodeMaxT) {  // few tokens: decode router kernel, then top-k + split
            uint16_t *x_hi = nullptr, *x_lo = nullptr;
            prefill_x_planes(w.pre, T, L->n_experts, L->top_k, L->dim, &x_hi, &x_lo);
            HIP_OK(h, launch_router_logits(lc(h, kProfRouter), h->order, L->dtype, xb_dev, L->router, L->router_bias, T,
                                           L->n_experts, L->dim, w.probs));
            HIP_OK(h, launch_topk_split(lc(h, kProfTopk), w.probs, T, L->n_experts, L->top_k, L->norm_topk, xb_dev, L->dim,
                                        routing, weights, x_hi, x_lo));
        } else if (fused) {
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
                                 L->expert_hidden, routing, weights, w.hbuf, w.pre, x_dev, moe_dev, &counts, fused,
                                 true, h->prefill_tile_rows, tiled_for(h, L), h->prefill_wide));
        h->expert_counts = counts;
        return done();
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
    return done();
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
    if (device >= kMaxDevices) return fail(nullptr, "init: device %d beyond the %d supported", device, kMaxDevices);
    rbt_hip *h = new rbt_hip();
    h->device = device;
    e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        fail(nullptr, "init: %s", hipGetErrorString(e));
        delete h;
        return 0;
    }
    {  // the scratch array's address on this device, looked up once per device with the device current
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (!g_scratch_ptr[device]) {
            void *p = nullptr;
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p) {
                fail(nullptr, "init: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
                (void)hipStreamDestroy(h->stream);
                delete h;
                return 0;
            }
            g_scratch_ptr[device] = p;
        }
        h->scratch = g_scratch_ptr[device];
    }
    *out = h;
    return 1;
}

void rbt_hip_free(rbt_hip *h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    ws_release(h->ws);
    (void)hipFree(h->ds.block);
    for (int k = 0; k < kProfCount; k++) {
        for (int j = 0; j < 2; j++)
            if (h->prof.ev[k][j]) (void)hipEventDestroy(h->prof.ev[k][j]);
        for (hipEvent_t ev : h->prof.pool[k]) (void)hipEventDestroy(ev);
    }
    (void)hipFree(h->stage);
    if (h->pin) (void)hipHostFree(h->pin);
    (void)hipFree(h->rhist);
    if (h->tok_host) (void)hipHostFree(h->tok_host);
    tiled_drop(h, nullptr, nullptr);
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

// The tiled copies of every layer of the loaded model (rbt_hip_prefill_layout with L NULL).
int tiled_build_model(rbt_hip *h) {
    const rbt_config &c = h->cfg;
    for (int l = 0; l < c.n_layers; l++) {
        rbt_moe_layer ml;
        if (!rbt_hip_layer(h, l, &ml) || !tiled_build(h, &ml)) return 0;
    }
    return 1;
}

int rbt_hip_upload(rbt_hip *h, const void *file, uint64_t file_size, rbt_config *cfg) {
    if (!h) return fail(nullptr, "upload: handle is NULL");
    ModelLayout m;
    if (!parse_header(&m, static_cast<const unsigned char *>(file), file_size, h)) return 0;
    if (!model_alloc(h, m)) return 0;
    const hipError_t e = HIP_TRY(hipMemcpy(h->model, file, m.layout_end, hipMemcpyHostToDevice));
    if (e != hipSuccess) {
        model_drop(h);
        return fail(h, "upload: hipMemcpy failed: %s", hipGetErrorString(e));
    }
    const rbt_config c = m.cfg;
    adopt_layout(h, std::move(m));
    h->cache_hits = 0;
    h->cache_misses = (uint64_t)c.n_layers * c.n_experts;
    if (cfg) *cfg = c;
    return 1;
}

int rbt_hip_upload_file(rbt_hip *h, const char *path, rbt_config *cfg) {
    if (!h) return fail(nullptr, "upload_file: handle is NULL");
    if (!path) return fail(h, "upload_file: path is NULL");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(h, "cannot open %s", path);  // rabbit2.c:201
    struct FdCloser {
        int fd;
        ~FdCloser() { close(fd); }
    } closer{fd};
    struct stat st;
    if (fstat(fd, &st) != 0) return fail(h, "cannot stat %s", path);
    const uint64_t file_size = (uint64_t)st.st_size;
    unsigned char hdr[kHeader];
    if (file_size < kHeader || pread(fd, hdr, kHeader, 0) != (ssize_t)kHeader)
        return fail(h, "bad magic: not a .rbt2 file");
    ModelLayout m;
    if (!parse_header(&m, hdr, file_size, h)) return 0;
    // the file mapped read-only (rabbit2.c:141-147) and copied in one call: the runtime pipelines a
    // pageable source through its own pinned staging (measured ~29 GB/s from the page cache, three
    // times a pread loop over pinned buffers)
    void *map = mmap(nullptr, (size_t)m.layout_end, PROT_READ, MAP_SHARED, fd, 0);
    if (map == MAP_FAILED) return fail(h, "cannot map %s", path);
    struct Unmap {
        void *p;
        size_t n;
        ~Unmap() { munmap(p, n); }
    } unmap{map, (size_t)m.layout_end};
    if (!model_alloc(h, m)) return 0;
    (void)madvise(map, (size_t)m.layout_end, MADV_SEQUENTIAL);
    const hipError_t e = HIP_TRY(hipMemcpy(h->model, map, m.layout_end, hipMemcpyHostToDevice));
    if (e != hipSuccess) {
        model_drop(h);
        return fail(h, "upload_file: hipMemcpy failed: %s", hipGetErrorString(e));
    }
    const rbt_config c = m.cfg;
    adopt_layout(h, std::move(m));
    h->cache_hits = 0;
    h->cache_misses = (uint64_t)c.n_layers * c.n_experts;
    if (cfg) *cfg = c;
    return 1;
}

int rbt_hip_file_info(const char *path, rbt_config *cfg, uint64_t info[7]) {
    if (!path) return fail(nullptr, "file_info: path is NULL");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(nullptr, "cannot open %s", path);  // rabbit2.c:200
    struct FdCloser {
        int fd;
        ~FdCloser() { close(fd); }
    } closer{fd};
    struct stat st;
    if (fstat(fd, &st) != 0) return fail(nullptr, "cannot stat %s", path);
    const uint64_t file_size = (uint64_t)st.st_size;
    unsigned char hdr[kHeader];
    if (file_size < kHeader || pread(fd, hdr, kHeader, 0) != (ssize_t)kHeader)
        return fail(nullptr, "bad magic: not a .rbt2 file");
    ModelLayout tmp;  // host-only: no device, no stream
    if (!parse_header(&tmp, hdr, file_size, nullptr)) return 0;
    if (cfg) *cfg = tmp.cfg;
    if (info) {
        info[0] = tmp.tok_emb;
        info[1] = tmp.layers.front().experts;
        info[2] = tmp.layers.back().experts;
        info[3] = tmp.expert_stride;
        info[4] = tmp.lm_head;
        info[5] = tmp.layout_end;
        info[6] = file_size;
    }
    return 1;
}

int rbt_hip_expert_stats(rbt_hip *h, uint64_t stats[6]) {
    if (!h || !stats) return fail(h, "expert_stats: NULL argument");
    if (!h->model) return fail(h, "expert_stats: no model");
    const uint64_t all = (uint64_t)h->cfg.n_layers * h->cfg.n_experts;
    stats[0] = h->cache_hits;
    stats[1] = h->cache_misses;
    stats[2] = 0;  // evictions: everything stays resident
    stats[3] = h->cache_misses * h->expert_stride;  // bytes_read == misses * expert_stride
    stats[4] = all * h->expert_stride;             // resident_bytes
    stats[5] = all * h->expert_stride;             // capacity_bytes
    return 1;
}

int rbt_hip_prefill_layout(rbt_hip *h, const rbt_moe_layer *L) {
    if (!h) return fail(nullptr, "prefill_layout: handle is NULL");
    if (!set_device(h)) return 0;
    if (L) return tiled_build(h, L);
    if (!h->model) return fail(h, "prefill_layout: no model (pass a layer, or upload a model first)");
    return tiled_build_model(h);
}

int rbt_hip_prefill_layout_drop(rbt_hip *h, const rbt_moe_layer *L) {
    if (!h) return fail(nullptr, "prefill_layout_drop: handle is NULL");
    if (!set_device(h)) return 0;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    if (!L) {
        tiled_drop(h, nullptr, nullptr);
        return 1;
    }
    const uint8_t *p = static_cast<const uint8_t *>(L->experts);
    tiled_drop(h, p, p + 1);
    return 1;
}

int rbt_hip_model_create(rbt_hip *h, const rbt_config *cfg, void **model_dev) {
    if (!h) return fail(nullptr, "model_create: handle is NULL");
    if (!cfg || !model_dev) return fail(h, "model_create: NULL argument");
    *model_dev = nullptr;
    if (!config_ok(*cfg)) return fail(h, "model_create: invalid config");
    ModelLayout m;
    uint64_t end = 0, limit = kMaxImageBytes;
    if (!set_device(h)) return 0;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) == hipSuccess && total_b < limit) limit = total_b;
    const int r = layout_of(*cfg, limit, &m, &end);
    if (r < 0) return fail(h, "model_create: no host memory for the layout of %d layers", cfg->n_layers);
    if (!r)
        return fail(h, "model_create: the image of this config (%llu bytes) exceeds the device's %llu bytes",
                    (unsigned long long)end, (unsigned long long)limit);
    if (!model_alloc(h, m)) return 0;
    adopt_layout(h, std::move(m));
    h->cache_hits = 0;
    h->cache_misses = (uint64_t)cfg->n_layers * cfg->n_experts;
    *model_dev = h->model;
    return 1;
}

int rbt_hip_tensor(rbt_hip *h, const char *name, int layer, uint64_t *offset, uint64_t *bytes) {
    if (!h || !name) return fail(h, "tensor: NULL argument");
    if (!h->model) return fail(h, "tensor: no model");
    const rbt_config &c = h->cfg;
    const uint64_t E = c.dtype == RBT_DT_BF16 ? 2 : 4, D = (uint64_t)c.dim;
    const uint64_t qd = (uint64_t)c.n_heads * c.head_dim, kvd = (uint64_t)c.n_kv_heads * c.head_dim;
    uint64_t off = 0, n = 0;
    if (!strcmp(name, "tok_emb")) {
        off = h->tok_emb, n = (uint64_t)c.vocab * D * E;
    } else if (!strcmp(name, "final_norm")) {
        off = h->final_norm, n = D * 4;
    } else if (!strcmp(name, "lm_head")) {
        off = h->lm_head, n = (uint64_t)c.vocab * D * E;
    } else {
        if (layer < 0 || layer >= c.n_layers) return fail(h, "tensor: layer %d out of range", layer);
        const LayerOff &ly = h->layers[(size_t)layer];
        if (!strcmp(name, "attn_norm")) off = ly.attn_norm, n = D * 4;
        else if (!strcmp(name, "wq")) off = ly.wq, n = qd * D * E;
        else if (!strcmp(name, "wk")) off = ly.wk, n = kvd * D * E;
        else if (!strcmp(name, "wv")) off = ly.wv, n = kvd * D * E;
        else if (!strcmp(name, "wo")) off = ly.wo, n = D * qd * E;
        else if (!strcmp(name, "q_norm") && c.qk_norm) off = ly.q_norm, n = qd * 4;
        else if (!strcmp(name, "k_norm") && c.qk_norm) off = ly.k_norm, n = kvd * 4;
        else if (!strcmp(name, "ffn_norm")) off = ly.ffn_norm, n = D * 4;
        else if (!strcmp(name, "router")) off = ly.router, n = (uint64_t)c.n_experts * D * E;
        else if (!strcmp(name, "experts")) off = ly.experts, n = (uint64_t)c.n_experts * h->expert_stride;
        else return fail(h, "tensor: unknown tensor '%s'", name);
    }
    if (offset) *offset = off;
    if (bytes) *bytes = n;
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
    const MoeForm form = moe_form(h, L, T, xb_dev);
    if (form == kMoeGrouped && !pre_reserve(h, prefill_workspace_bytes(T, L->n_experts, L->top_k, L->dim))) return 0;
    return moe_block(h, L, xb_dev, T, x_dev, moe_dev, routing_dev, weights_dev, h->ws, form, true);
}

int rbt_hip_moe_dev_noalloc(rbt_hip *h, const rbt_moe_layer *L, const float *xb_dev, int T, float *x_dev,
                            float *moe_dev, int32_t *routing_dev, float *weights_dev) {
    if (!h) return fail(nullptr, "moe_noalloc: handle is NULL");
    if (T < 0) return fail(h, "moe_noalloc: negative token count");
    if (!check_layer(h, L)) return 0;
    if (T == 0) return 1;
    if (!xb_dev) return fail(h, "moe_noalloc: xb is NULL");
    if (!h->scratch) return fail(h, "moe_noalloc: no scratch address for device %d", h->device);
    const MoeForm form = moe_form(h, L, T, xb_dev);
    const size_t need = moe_scratch_bytes(T, L->n_experts, L->top_k, L->expert_hidden, L->dim, form == kMoeGrouped);
    if (need > kScratchBytes)
        return fail(h, "moe_noalloc: %d tokens of this layer need %zu bytes of scratch, above its %zu bytes", T, need,
                    (size_t)kScratchBytes);
    if (!set_device(h)) return 0;
    Workspace w = scratch_view(h->scratch, T, L->n_experts, L->top_k, L->expert_hidden, L->dim, form == kMoeGrouped);
    return moe_block(h, L, xb_dev, T, x_dev, moe_dev, routing_dev, weights_dev, w, form, false);
}

const int32_t *rbt_hip_expert_counts_dev(rbt_hip *h) { return h ? h->expert_counts : nullptr; }

int rbt_hip_moe(rbt_hip *h, int layer, const float *xb, int T, float *x_inout, int32_t *routing_out) {
    if (!h) return fail(nullptr, "moe: handle is NULL");
    rbt_moe_layer L;
    if (!rbt_hip_layer(h, layer, &L)) return 0;
    if (T < 0) return fail(h, "moe: negative token count");
    if (T == 0) return 1;
    if (!xb) return fail(h, "moe: xb is NULL");
    // one region [xb | x | routing] on the device and its pinned host twin: the inputs go up in one copy,
    // x and the routing come back in one, and the call waits once
    const uint64_t nx = (uint64_t)T * L.dim, nr = (uint64_t)T * L.top_k;
    const uint64_t x_off = align_up(nx * 4, 256), r_off = x_off + align_up(nx * 4, 256), total = r_off + nr * 4;
    if (!set_device(h) || !stage_reserve(h, total) || !pin_reserve(h, total)) return 0;
    uint8_t *st = static_cast<uint8_t *>(h->stage), *pn = static_cast<uint8_t *>(h->pin);
    float *x_d = x_inout ? reinterpret_cast<float *>(st + x_off) : nullptr;
    int32_t *r_d = reinterpret_cast<int32_t *>(st + r_off);
    memcpy(pn, xb, nx * 4);
    if (x_inout) memcpy(pn + x_off, x_inout, nx * 4);
    HIP_OK(h, hipMemcpyAsync(st, pn, x_inout ? x_off + nx * 4 : nx * 4, hipMemcpyHostToDevice, h->stream));
    if (!rbt_hip_moe_dev(h, &L, reinterpret_cast<float *>(st), T, x_d, nullptr, r_d, nullptr)) return 0;
    const uint64_t back = x_inout ? x_off : r_off;  // x (if any) and the routing, one contiguous copy
    HIP_OK(h, hipMemcpyAsync(pn + back, st + back, total - back, hipMemcpyDeviceToHost, h->stream));
    HIP_OK(h, hipStreamSynchronize(h->stream));
    if (x_inout) memcpy(x_inout, pn + x_off, nx * 4);
    if (routing_out) memcpy(routing_out, pn + r_off, nr * 4);
    h->cache_hits += nr;  // every selected expert was resident
    return prof_harvest(h);
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
    const uint8_t *p = static_cast<const uint8_t *>(*dev);
    for (const TiledLayer &t : h->tiled)
        if (static_cast<const uint8_t *>(t.experts) >= p && static_cast<const uint8_t *>(t.experts) < p + bytes) {
            // copies of blobs freed earlier (their memory is this allocation now): drop them
            HIP_OK(h, hipStreamSynchronize(h->stream));
            tiled_drop(h, p, p + bytes);
            break;
        }
    return 1;
}

int rbt_hip_free_dev(rbt_hip *h, void *dev) {
    if (!h) return fail(nullptr, "free_dev: handle is NULL");
    if (!dev) return 1;
    if (!set_device(h)) return 0;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    // tiled copies of blobs inside the freed allocation go with it
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (!h->tiled.empty() && hipMemGetAddressRange(&base, &size, static_cast<hipDeviceptr_t>(dev)) == hipSuccess)
        tiled_drop(h, static_cast<const uint8_t *>(base), static_cast<const uint8_t *>(base) + size);
    HIP_OK(h, hipFree(dev));
    return 1;
}

int rbt_hip_h2d(rbt_hip *h, void *dst_dev, const void *src, uint64_t bytes) {
    if (!h) return fail(nullptr, "h2d: handle is NULL");
    if (!bytes) return 1;
    if (!dst_dev || !src) return fail(h, "h2d: NULL pointer");
    if (!set_device(h)) return 0;
    HIP_OK(h, hipMemcpyAsync(dst_dev, src, bytes, hipMemcpyHostToDevice, h->stream));
    if (!tiled_follow_write(h, dst_dev, bytes)) return 0;
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
    return tiled_follow_write(h, dst_dev, bytes);
}

int rbt_hip_synchronize(rbt_hip *h) {
    if (!h) return fail(nullptr, "synchronize: handle is NULL");
    if (!set_device(h)) return 0;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    return 1;
}

int rbt_hip_set_sampling(rbt_hip *h, float temperature, int top_k, float top_p, uint64_t seed) {
    if (!h) return fail(nullptr, "set_sampling: handle is NULL");
    if (temperature != temperature || top_p != top_p) return fail(h, "set_sampling: NaN argument");
    h->sampling.temperature = temperature;
    h->sampling.top_k = top_k;
    h->sampling.top_p = top_p;
    h->seed = seed;
    return 1;
}

int rbt_hip_set_option(rbt_hip *h, const char *name, int64_t value) {
    if (!h || !name) return fail(h, "set_option: NULL argument");
    if (strcmp(name, "fused_decode") == 0) {
        h->fused_decode = value != 0;
    } else if (strcmp(name, "batch_mfma") == 0) {
        h->batch_mfma = value != 0;
    } else if (strcmp(name, "prefill_layout") == 0) {
        h->prefill_layout = value != 0;
    } else if (strcmp(name, "routing_history") == 0) {
        h->routing_history = value != 0;  // takes effect at the next rbt_hip_state_init / batch_init
    } else if (strcmp(name, "prefill_min_tokens") == 0) {
        if (value < 1 || value > 65536) return fail(h, "set_option: prefill_min_tokens must be in [1, 65536]");
        h->prefill_min_tokens = (int)value;
    } else if (strcmp(name, "prefill_tile_rows") == 0) {
        if (value != 0 && value != 32 && value != 64 && value != 128)
            return fail(h, "set_option: prefill_tile_rows must be 0, 32, 64 or 128");
        h->prefill_tile_rows = (int)value;
    } else if (strcmp(name, "prefill_wide") == 0) {
        h->prefill_wide = value != 0;
    } else if (strcmp(name, "generate_timed_from") == 0) {
        if (value < 1 || value > (1 << 30)) return fail(h, "set_option: generate_timed_from must be in [1, 2^30]");
        h->gen_timed_from = (int)value;
    } else {
        return fail(h, "set_option: unknown option '%s'", name);
    }
    return 1;
}

void *rbt_hip_stream(rbt_hip *h) { return h ? static_cast<void *>(h->stream) : nullptr; }

int rbt_hip_profiler_attached(void) { return profiler_var() != nullptr; }

int rbt_hip_profile_enable(rbt_hip *h, int on) {
    if (!h) return fail(nullptr, "profile: handle is NULL");
    if (!set_device(h)) return 0;
    if (on < 0 || on > 2) return fail(h, "profile: mode must be 0, 1 or 2");
    if (on == 1 && !h->prof.ev[0][0]) {
        for (int k = 0; k < kProfCount; k++)
            for (int j = 0; j < 2; j++) HIP_OK(h, hipEventCreate(&h->prof.ev[k][j]));
    }
    if (on) {
        for (int k = 0; k < kProfCount; k++) {
            h->prof.total_ms[k] = 0.0;
            h->prof.launches[k] = 0;
            h->prof.used[k] = false;
            h->prof.next[k] = 0;
        }
    }
    h->prof.mode = on;
    return 1;
}

int rbt_hip_profile_get(rbt_hip *h, const char *kernel, double *total_ms, uint64_t *launches) {
    if (!h || !kernel) return fail(h, "profile_get: NULL argument");
    for (int k = 0; k < kProfCount; k++) {
        if (strcmp(kernel, kProfNames[k]) != 0) continue;
        if (h->prof.mode == 2 && (!set_device(h) || !prof_harvest(h))) return 0;
        if (total_ms) *total_ms = h->prof.total_ms[k];
        if (launches) *launches = h->prof.launches[k];
        return 1;
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
    return tiled_follow_write(h, dst_dev, n * (dtype == RBT_DT_BF16 ? 2 : 4));
}

int rbt_hip_state_init(rbt_hip *h, int ctx) { return rbt_hip_batch_init(h, 1, ctx); }

int rbt_hip_batch_init(rbt_hip *h, int n_seq, int ctx) {
    if (!h) return fail(nullptr, "state_init: handle is NULL");
    if (!h->model) return fail(h, "state_init: no model");
    const rbt_config &c = h->cfg;
    if (ctx < 0) return fail(h, "state_init: negative context");
    if (n_seq < 1 || n_seq > 1024) return fail(h, "state_init: n_seq must be in [1, 1024]");
    if (ctx == 0) ctx = c.max_seq < 512 ? c.max_seq : 512;  // rabbit2.c:684
    if (ctx > c.max_seq) ctx = c.max_seq;                   // rabbit2.c:685
    if (!set_device(h)) return 0;
    HIP_OK(h, hipStreamSynchronize(h->stream));
    (void)hipFree(h->ds.block);
    h->ds = DecodeState{};
    (void)hipFree(h->rhist);
    h->rhist = nullptr;
    DecodeState ds;
    ds.n_seq = n_seq;
    ds.ctx = ctx;
    // attention splits over positions (<= 64): a split per 24 positions of the context, at most 16 (OLMoE
    // shape, 384 positions: 731 us per token with 16 splits against 736 with 12 and 743 with 24)
    ds.S = ctx / 24 < 1 ? 1 : (ctx / 24 > 16 ? 16 : ctx / 24);
    // (sequence, head) blocks enough to fill the chip twice: one split, and the attention kernel writes
    // its output itself (32 sequences x 16 heads at 2080 positions: 178 us against 187 + 5 us for 16
    // splits and the merge)
    if ((long long)n_seq * c.n_heads >= kAttnDirectBlocks) ds.S = 1;
    const uint64_t D = (uint64_t)c.dim, hd = (uint64_t)c.head_dim, qd = (uint64_t)c.n_heads * hd,
                   kvd = (uint64_t)c.n_kv_heads * hd;
    uint64_t off = 0;
    auto carve = [&](uint64_t bytes) {
        const uint64_t at = off;
        off = align_up(off + bytes, 256);
        return at;
    };
    const uint64_t B = (uint64_t)n_seq;
    const uint64_t o_kc = carve(4 * B * c.n_layers * ctx * kvd), o_vc = carve(4 * B * c.n_layers * ctx * kvd);
    const uint64_t o_x = carve(4 * B * D), o_xb = carve(4 * B * D), o_q = carve(4 * B * qd), o_k = carve(4 * B * kvd),
                   o_v = carve(4 * B * kvd), o_ao = carve(4 * B * qd);
    const uint64_t o_part = carve(4 * B * c.n_heads * ds.S * (hd + 2));
    const uint64_t plane = B <= 64 ? (uint64_t)mfma_plane_elems((int)B, (int)(D > qd ? D : qd)) : 0;
    const uint64_t o_xh = carve(2 * plane), o_xl = carve(2 * plane);
    const uint64_t o_rope = carve(8 * (uint64_t)ctx * (hd / 2));
    const uint64_t o_cand = carve(8 * (uint64_t)dense_argmax_blocks(c.vocab));
    const uint64_t o_sp = carve(4 * B * c.vocab), o_si = carve(4 * B * c.vocab);
    const uint64_t o_lg = carve(4 * B * c.vocab), o_rt = carve(4 * B * c.n_layers * c.top_k);
    const uint64_t o_seq = carve(4 * B * ctx), o_st = carve(sizeof(StepState) * B);
    if (c.head_dim > 256 || 4 * D > 64 * 1024 || 4 * qd > 64 * 1024)
        return fail(h, "state_init: head_dim above 256 or dim above 16384 is not supported");
    HIP_OK(h, hipMalloc(&ds.block, off));
    uint8_t *b = ds.block;
    ds.kc = reinterpret_cast<float *>(b + o_kc);
    ds.vc = reinterpret_cast<float *>(b + o_vc);
    ds.x = reinterpret_cast<float *>(b + o_x);
    ds.xb = reinterpret_cast<float *>(b + o_xb);
    ds.q = reinterpret_cast<float *>(b + o_q);
    ds.k = reinterpret_cast<float *>(b + o_k);
    ds.v = reinterpret_cast<float *>(b + o_v);
    ds.ao = reinterpret_cast<float *>(b + o_ao);
    ds.part = reinterpret_cast<float *>(b + o_part);
    ds.xh = reinterpret_cast<uint16_t *>(b + o_xh);
    ds.xl = reinterpret_cast<uint16_t *>(b + o_xl);
    ds.rope_cs = reinterpret_cast<float2 *>(b + o_rope);
    ds.cand = reinterpret_cast<float2 *>(b + o_cand);
    ds.sprob = reinterpret_cast<float *>(b + o_sp);
    ds.sidx = reinterpret_cast<int32_t *>(b + o_si);
    ds.logits = reinterpret_cast<float *>(b + o_lg);
    ds.routing = reinterpret_cast<int32_t *>(b + o_rt);
    ds.seq = reinterpret_cast<int32_t *>(b + o_seq);
    ds.st = reinterpret_cast<StepState *>(b + o_st);
    HIP_OK(h, hipMemset(ds.block, 0, off));
    // RoPE (cos, sin) of every position and pair, with the engine's own expressions in double and the
    // host's libm (rabbit2.c:414-417), so the rotation uses the same floats as the engine
    {
        const int half = c.head_dim / 2;
        std::vector<float2> cs((size_t)ctx * half);
        for (int p = 0; p < ctx; p++)
            for (int i = 0; i < half; i++) {
                const double freq = pow((double)c.rope_theta, -2.0 * i / c.head_dim);
                const double ang = p * freq;
                cs[(size_t)p * half + i] = make_float2((float)cos(ang), (float)sin(ang));
            }
        const hipError_t e = hipMemcpy(ds.rope_cs, cs.data(), cs.size() * sizeof(float2), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(ds.block);
            return fail(h, "state_init: hipMemcpy failed: %s", hipGetErrorString(e));
        }
    }
    if (h->routing_history) {
        const size_t hb = sizeof(int32_t) * (size_t)n_seq * ctx * c.n_layers * c.top_k;
        hipError_t e = HIP_TRY(hipMalloc(&h->rhist, hb));
        if (e == hipSuccess) e = HIP_TRY(hipMemset(h->rhist, 0, hb));
        if (e != hipSuccess) {
            (void)hipFree(h->rhist);
            (void)hipFree(ds.block);
            h->rhist = nullptr;
            return fail(h, "state_init: hipMalloc of the routing history failed: %s", hipGetErrorString(e));
        }
    }
    h->ds = ds;
    // the MoE workspace for n_seq tokens per layer call, so that no step allocates
    rbt_moe_layer ml;
    if (!rbt_hip_layer(h, 0, &ml) || !rbt_hip_reserve(h, &ml, n_seq)) return 0;
    return 1;
}

int rbt_hip_forward(rbt_hip *h, int token, int pos, float *logits, int32_t *routing_out) {
    if (!h) return fail(nullptr, "forward: handle is NULL");
    if (!h->ds.block) return fail(h, "forward: no decode state (rbt_hip_state_init)");
    if (h->ds.n_seq != 1) return fail(h, "forward: the state holds %d sequences (rbt_hip_forward_batch)", h->ds.n_seq);
    const rbt_config &c = h->cfg;
    if (token < 0 || token >= c.vocab) return fail(h, "token %d out of range", token);
    if (pos < 0 || pos >= h->ds.ctx) return fail(h, "forward: position %d outside the context of %d", pos, h->ds.ctx);
    if (!set_device(h)) return 0;
    const StepState st{pos, 0x7FFFFFFF, 0, 0, 0, 0};
    HIP_OK(h, hipMemcpyAsync(h->ds.seq + pos, &token, 4, hipMemcpyHostToDevice, h->stream));
    HIP_OK(h, hipMemcpyAsync(h->ds.st, &st, sizeof st, hipMemcpyHostToDevice, h->stream));
    const Sampling sp = h->sampling;
    h->sampling = Sampling{};  // a forward returns logits; its tail is the (cheap) greedy argmax
    const int ok = enqueue_step(h, true);
    h->sampling = sp;
    if (!ok) return 0;
    if (logits) HIP_OK(h, hipMemcpyAsync(logits, h->ds.logits, 4 * (size_t)c.vocab, hipMemcpyDeviceToHost, h->stream));
    if (routing_out)
        HIP_OK(h, hipMemcpyAsync(routing_out, h->ds.routing, 4 * (size_t)c.n_layers * c.top_k, hipMemcpyDeviceToHost,
                                 h->stream));
    HIP_OK(h, hipStreamSynchronize(h->stream));
    h->cache_hits += (uint64_t)c.n_layers * c.top_k;
    return prof_harvest(h);
}

int rbt_hip_generate(rbt_hip *h, const int32_t *prompt, int n_prompt, int n_gen, int32_t eos, int32_t *out,
                     int *n_out, double *ms_out) {
    return rbt_hip_generate_stream(h, prompt, n_prompt, n_gen, eos, nullptr, nullptr, out, n_out, ms_out);
}

int rbt_hip_generate_stream(rbt_hip *h, const int32_t *prompt, int n_prompt, int n_gen, int32_t eos,
                            rbt_token_fn on_token, void *user, int32_t *out, int *n_out, double *ms_out) {
    if (!h) return fail(nullptr, "generate: handle is NULL");
    if (n_out) *n_out = 0;
    if (!h->ds.block) return fail(h, "generate: no decode state (rbt_hip_state_init)");
    if (h->ds.n_seq != 1) return fail(h, "generate: the state holds %d sequences (rbt_hip_generate_batch)", h->ds.n_seq);
    const rbt_config &c = h->cfg;
    const int ctx = h->ds.ctx;
    if (!prompt || n_prompt < 1) return fail(h, "generate: empty prompt");
    if (n_prompt > ctx)
        return fail(h, "prompt has %d tokens but context is %d (use --ctx)", n_prompt, ctx);  // rabbit2.c:687
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= c.vocab) return fail(h, "token %d out of range", prompt[i]);
    if (n_gen < 0) return fail(h, "generate: negative n_gen");
    if (n_gen > ctx - n_prompt) n_gen = ctx - n_prompt;  // rabbit2.c:717
    if (n_gen > 0 && !out) return fail(h, "generate: out is NULL");
    if (!set_device(h)) return 0;
    if (on_token && n_gen > h->tok_host_n) {  // the pinned ring the device's tokens are copied into
        HIP_OK(h, hipStreamSynchronize(h->stream));
        if (h->tok_host) (void)hipHostFree(h->tok_host);
        h->tok_host = nullptr;
        h->tok_host_n = 0;
        HIP_OK(h, hipHostMalloc(&h->tok_host, sizeof(int32_t) * (size_t)n_gen, hipHostMallocDefault));
        h->tok_host_n = n_gen;
    }
    const StepState st{0, n_prompt, 0, 0, h->seed ? h->seed : 0x9E3779B97F4A7C15ull, 0};  // rabbit2.c:723
    HIP_OK(h, hipMemcpyAsync(h->ds.seq, prompt, 4 * (size_t)n_prompt, hipMemcpyHostToDevice, h->stream));
    HIP_OK(h, hipMemcpyAsync(h->ds.st, &st, sizeof st, hipMemcpyHostToDevice, h->stream));
    const int prof = h->prof.mode;
    h->prof.mode = 0;
    hipGraphExec_t g_adv = nullptr, g_fin = nullptr;
    // ev: start, after the first generated token, end, start of the timed window (ms_out[1])
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
    const int t0 = h->gen_timed_from;
    // streaming: one event per step in flight; the host keeps at most kStreamAhead steps queued past
    // the last token it has reported, and stops queueing at the eos token
    constexpr int kStreamAhead = 32;
    hipEvent_t ring[kStreamAhead] = {};
    int ok = capture_step(h, false, &g_adv) && capture_step(h, true, &g_fin);
    h->prof.mode = prof;
    auto cleanup = [&]() {
        if (g_adv) (void)hipGraphExecDestroy(g_adv);
        if (g_fin) (void)hipGraphExecDestroy(g_fin);
        for (hipEvent_t e : ev)
            if (e) (void)hipEventDestroy(e);
        for (hipEvent_t e : ring)
            if (e) (void)hipEventDestroy(e);
    };
    if (!ok) {
        cleanup();
        return 0;
    }
    hipError_t e = hipSuccess;
    for (int i = 0; i < 4 && e == hipSuccess; i++) e = HIP_TRY(hipEventCreate(&ev[i]));
    if (e == hipSuccess) e = HIP_TRY(hipEventRecord(ev[0], h->stream));
    // the prompt: n_prompt forwards, the last one with lm_head + argmax (the first generated token)
    for (int p = 0; p + 1 < n_prompt && e == hipSuccess; p++) e = HIP_TRY(hipGraphLaunch(g_adv, h->stream));
    int n = n_gen;
    bool window = false;  // ev[3] recorded: before generated step t0, else with ev[2]
    auto mark_window = [&](int g) -> hipError_t {
        if (window || g < t0) return hipSuccess;
        window = true;
        return HIP_TRY(hipEventRecord(ev[3], h->stream));
    };
    if (!on_token) {
        if (e == hipSuccess && n_gen > 0) e = HIP_TRY(hipGraphLaunch(g_fin, h->stream));
        if (e == hipSuccess) e = HIP_TRY(hipEventRecord(ev[1], h->stream));
        // each further token: one forward of the previous one (rabbit2.c:733)
        for (int g = 1; g < n_gen && e == hipSuccess; g++) {
            e = mark_window(g);
            if (e == hipSuccess) e = HIP_TRY(hipGraphLaunch(g_fin, h->stream));
        }
        if (e == hipSuccess) e = mark_window(INT32_MAX);
        if (e == hipSuccess) e = HIP_TRY(hipEventRecord(ev[2], h->stream));
        if (e == hipSuccess && n_gen > 0)
            e = HIP_TRY(hipMemcpyAsync(out, h->ds.seq + n_prompt, 4 * (size_t)n_gen, hipMemcpyDeviceToHost, h->stream));
        if (e == hipSuccess) e = HIP_TRY(hipStreamSynchronize(h->stream));
        for (int g = 0; g < n_gen && e == hipSuccess; g++)
            if (out[g] == eos) {  // the engine prints the eos token, then stops (rabbit2.c:729-730)
                n = g + 1;
                break;
            }
    } else {
        for (int i = 0; i < kStreamAhead && e == hipSuccess; i++) e = HIP_TRY(hipEventCreate(&ring[i]));
        int queued = 0, reported = 0;
        bool more = n_gen > 0, report = true;
        auto queue_step = [&](int g) -> hipError_t {
            hipError_t r = g > 0 ? mark_window(g) : hipSuccess;
            if (r == hipSuccess) r = HIP_TRY(hipGraphLaunch(g_fin, h->stream));
            if (r == hipSuccess && g == 0) r = HIP_TRY(hipEventRecord(ev[1], h->stream));
            if (r == hipSuccess)
                r = HIP_TRY(hipMemcpyAsync(h->tok_host + g, h->ds.seq + n_prompt + g, 4, hipMemcpyDeviceToHost,
                                           h->stream));
            if (r == hipSuccess) r = HIP_TRY(hipEventRecord(ring[g % kStreamAhead], h->stream));
            return r;
        };
        n = 0;
        while (e == hipSuccess && reported < queued + (more ? 1 : 0)) {
            while (e == hipSuccess && more && queued < reported + kStreamAhead) {
                e = queue_step(queued++);
                if (queued == n_gen) more = false;
                if (!more && e == hipSuccess) e = mark_window(INT32_MAX);
                if (!more && e == hipSuccess) e = HIP_TRY(hipEventRecord(ev[2], h->stream));
            }
            if (e != hipSuccess || reported == queued) break;
            e = HIP_TRY(hipEventSynchronize(ring[reported % kStreamAhead]));
            if (e != hipSuccess) break;
            const int32_t tok = h->tok_host[reported];
            out[reported++] = tok;
            n = reported;
            if (report && !on_token(user, tok)) report = false;  // the caller wants no more tokens
            if (tok == eos || !report) {  // nothing more is queued; the queued steps run to their end
                if (more) {
                    more = false;
                    e = mark_window(INT32_MAX);
                    if (e == hipSuccess) e = HIP_TRY(hipEventRecord(ev[2], h->stream));
                }
                break;
            }
        }
        if (e == hipSuccess) e = HIP_TRY(hipStreamSynchronize(h->stream));
        if (n_gen == 0 && e == hipSuccess) e = HIP_TRY(hipEventRecord(ev[1], h->stream));
        if (n_gen == 0 && e == hipSuccess) e = mark_window(INT32_MAX);
        if (n_gen == 0 && e == hipSuccess) e = HIP_TRY(hipEventRecord(ev[2], h->stream));
        if (e == hipSuccess) e = HIP_TRY(hipStreamSynchronize(h->stream));
    }
    if (e == hipSuccess && ms_out) {
        float a = 0.0f, b = 0.0f;
        e = HIP_TRY(hipEventElapsedTime(&a, ev[0], ev[1]));
        if (e == hipSuccess) e = HIP_TRY(hipEventElapsedTime(&b, ev[3], ev[2]));
        ms_out[0] = a;
        ms_out[1] = b;
    }
    cleanup();
    if (e != hipSuccess) return fail(h, "generate: %s failed: %s", failed_call(), hipGetErrorString(e));
    if (n_out) *n_out = n;
    return 1;
}

int rbt_hip_forward_batch(rbt_hip *h, const int32_t *tokens, const int32_t *pos, float *logits, int32_t *routing_out) {
    if (!h) return fail(nullptr, "forward_batch: handle is NULL");
    if (!h->ds.block) return fail(h, "forward_batch: no decode state (rbt_hip_batch_init)");
    if (!tokens || !pos) return fail(h, "forward_batch: NULL argument");
    const rbt_config &c = h->cfg;
    const int B = h->ds.n_seq;
    std::vector<StepState> st((size_t)B);
    for (int b = 0; b < B; b++) {
        if (tokens[b] < 0 || tokens[b] >= c.vocab) return fail(h, "token %d out of range", tokens[b]);
        if (pos[b] < 0 || pos[b] >= h->ds.ctx)
            return fail(h, "forward_batch: position %d outside the context of %d", pos[b], h->ds.ctx);
        st[(size_t)b] = StepState{pos[b], 0x7FFFFFFF, 0, 0, 0, 0};
    }
    if (!set_device(h)) return 0;
    for (int b = 0; b < B; b++)
        HIP_OK(h, hipMemcpyAsync(h->ds.seq + (size_t)b * h->ds.ctx + pos[b], tokens + b, 4, hipMemcpyHostToDevice,
                                 h->stream));
    HIP_OK(h, hipMemcpyAsync(h->ds.st, st.data(), sizeof(StepState) * B, hipMemcpyHostToDevice, h->stream));
    const Sampling sp = h->sampling;
    h->sampling = Sampling{};
    const int ok = enqueue_step(h, true);
    h->sampling = sp;
    if (!ok) return 0;
    if (logits)
        HIP_OK(h, hipMemcpyAsync(logits, h->ds.logits, 4 * (size_t)B * c.vocab, hipMemcpyDeviceToHost, h->stream));
    if (routing_out)
        HIP_OK(h, hipMemcpyAsync(routing_out, h->ds.routing, 4 * (size_t)c.n_layers * B * c.top_k,
                                 hipMemcpyDeviceToHost, h->stream));
    HIP_OK(h, hipStreamSynchronize(h->stream));
    h->cache_hits += (uint64_t)c.n_layers * B * c.top_k;
    return prof_harvest(h);
}

int rbt_hip_generate_batch(rbt_hip *h, const int32_t *prompts, int n_prompt, int n_gen, int32_t *out, double *ms_out) {
    if (!h) return fail(nullptr, "generate_batch: handle is NULL");
    if (!h->ds.block) return fail(h, "generate_batch: no decode state (rbt_hip_batch_init)");
    const rbt_config &c = h->cfg;
    const int B = h->ds.n_seq, ctx = h->ds.ctx;
    if (!prompts || n_prompt < 1) return fail(h, "generate_batch: empty prompts");
    if (n_prompt > ctx) return fail(h, "prompt has %d tokens but context is %d (use --ctx)", n_prompt, ctx);
    for (size_t i = 0; i < (size_t)B * n_prompt; i++)
        if (prompts[i] < 0 || prompts[i] >= c.vocab) return fail(h, "token %d out of range", prompts[i]);
    if (n_gen < 0 || n_gen > ctx - n_prompt)
        return fail(h, "generate_batch: n_gen %d outside [0, ctx - n_prompt = %d]", n_gen, ctx - n_prompt);
    if (n_gen > 0 && !out) return fail(h, "generate_batch: out is NULL");
    if (!set_device(h)) return 0;
    std::vector<StepState> st((size_t)B, StepState{0, n_prompt, 0, 0, h->seed ? h->seed : 0x9E3779B97F4A7C15ull, 0});
    for (int b = 0; b < B; b++)
        HIP_OK(h, hipMemcpyAsync(h->ds.seq + (size_t)b * ctx, prompts + (size_t)b * n_prompt, 4 * (size_t)n_prompt,
                                 hipMemcpyHostToDevice, h->stream));
    HIP_OK(h, hipMemcpyAsync(h->ds.st, st.data(), sizeof(StepState) * B, hipMemcpyHostToDevice, h->stream));
    const int prof = h->prof.mode;
    h->prof.mode = 0;
    hipGraphExec_t g_adv = nullptr, g_fin = nullptr;
    // ev: start, after the first generated step, end, start of the timed window (ms_out[1])
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
    const int t0 = h->gen_timed_from;
    int ok = capture_step(h, false, &g_adv) && capture_step(h, true, &g_fin);
    h->prof.mode = prof;
    hipError_t e = hipSuccess;
    if (ok) {
        for (int i = 0; i < 4 && e == hipSuccess; i++) e = HIP_TRY(hipEventCreate(&ev[i]));
        if (e == hipSuccess) e = HIP_TRY(hipEventRecord(ev[0], h->stream));
        for (int p = 0; p + 1 < n_prompt && e == hipSuccess; p++) e = HIP_TRY(hipGraphLaunch(g_adv, h->stream));
        if (e == hipSuccess && n_gen > 0) e = HIP_TRY(hipGraphLaunch(g_fin, h->stream));
        if (e == hipSuccess) e = HIP_TRY(hipEventRecord(ev[1], h->stream));
        bool window = false;
        for (int g = 1; g < n_gen && e == hipSuccess; g++) {
            if (!window && g >= t0) {
                window = true;
                e = HIP_TRY(hipEventRecord(ev[3], h->stream));
            }
            if (e == hipSuccess) e = HIP_TRY(hipGraphLaunch(g_fin, h->stream));
        }
        if (e == hipSuccess && !window) e = HIP_TRY(hipEventRecord(ev[3], h->stream));
        if (e == hipSuccess) e = HIP_TRY(hipEventRecord(ev[2], h->stream));
        for (int b = 0; b < B && e == hipSuccess && n_gen > 0; b++)
            e = HIP_TRY(hipMemcpyAsync(out + (size_t)b * n_gen, h->ds.seq + (size_t)b * ctx + n_prompt,
                                       4 * (size_t)n_gen, hipMemcpyDeviceToHost, h->stream));
        if (e == hipSuccess) e = HIP_TRY(hipStreamSynchronize(h->stream));
        if (e == hipSuccess && ms_out) {
            float a = 0.0f, bms = 0.0f;
            e = HIP_TRY(hipEventElapsedTime(&a, ev[0], ev[1]));
            if (e == hipSuccess) e = HIP_TRY(hipEventElapsedTime(&bms, ev[3], ev[2]));
            ms_out[0] = a;
            ms_out[1] = bms;
        }
    }
    if (g_adv) (void)hipGraphExecDestroy(g_adv);
    if (g_fin) (void)hipGraphExecDestroy(g_fin);
    for (hipEvent_t ei : ev)
        if (ei) (void)hipEventDestroy(ei);
    if (!ok) return 0;
    if (e != hipSuccess) return fail(h, "generate_batch: %s failed: %s", failed_call(), hipGetErrorString(e));
    return 1;
}

int rbt_hip_routing_history(rbt_hip *h, int seq, int first_pos, int n_pos, int32_t *out) {
    if (!h) return fail(nullptr, "routing_history: handle is NULL");
    if (!h->ds.block) return fail(h, "routing_history: no decode state");
    if (!h->rhist) return fail(h, "routing_history: option \"routing_history\" was off at rbt_hip_state_init");
    if (seq < 0 || seq >= h->ds.n_seq) return fail(h, "routing_history: sequence %d out of range", seq);
    if (first_pos < 0 || n_pos < 0 || first_pos > h->ds.ctx - n_pos)
        return fail(h, "routing_history: positions [%d, %d) outside the context of %d", first_pos, first_pos + n_pos,
                    h->ds.ctx);
    if (n_pos == 0) return 1;
    if (!out) return fail(h, "routing_history: out is NULL");
    if (!set_device(h)) return 0;
    const size_t per = (size_t)h->cfg.n_layers * h->cfg.top_k;
    HIP_OK(h, hipMemcpyAsync(out, h->rhist + ((size_t)seq * h->ds.ctx + first_pos) * per, 4 * per * (size_t)n_pos,
                             hipMemcpyDeviceToHost, h->stream));
    HIP_OK(h, hipStreamSynchronize(h->stream));
    return 1;
}

int rbt_hip_expert_cache_replay(uint64_t budget_bytes, uint64_t expert_stride, int n_layers, int n_experts, int top_k,
                                const int32_t *routing, uint64_t n_tokens, uint64_t stats[6]) {
    if (!stats || (n_tokens && !routing)) return fail(nullptr, "expert_cache_replay: NULL argument");
    if (expert_stride == 0 || n_layers <= 0 || n_experts <= 0 || top_k <= 0)
        return fail(nullptr, "expert_cache_replay: invalid shape");
    if (budget_bytes < expert_stride)  // rabbit2.c:238-242
        return fail(nullptr, "expert cache budget too small: need at least %llu bytes for one expert",
                    (unsigned long long)expert_stride);
    // expert_cache_init (rabbit2.c:243-245): as many whole slots as the budget holds, at most every expert
    uint64_t cap = budget_bytes / expert_stride;
    const uint64_t total = (uint64_t)n_layers * (uint64_t)n_experts;
    if (cap > total) cap = total;
    struct Slot {
        int layer = -1, expert = -1;
        uint64_t last_used = 0;
        bool valid = false, has_data = false;
    };
    std::vector<Slot> slots((size_t)cap);
    uint64_t clock = 0, hits = 0, misses = 0, evictions = 0, resident = 0;
    // get_expert (rabbit2.c:261-300) for every selection in the engine's order: token, layer, slot
    for (uint64_t t = 0; t < n_tokens; t++)
        for (int l = 0; l < n_layers; l++)
            for (int k = 0; k < top_k; k++) {
                const int e = routing[(t * (uint64_t)n_layers + (uint64_t)l) * (uint64_t)top_k + (uint64_t)k];
                if (e < 0 || e >= n_experts)
                    return fail(nullptr, "expert_cache_replay: expert %d out of range (token %llu, layer %d)", e,
                                (unsigned long long)t, l);
                Slot *victim = nullptr;
                bool hit = false;
                for (Slot &sl : slots) {
                    if (sl.valid && sl.layer == l && sl.expert == e) {
                        sl.last_used = ++clock;
                        hits++;
                        hit = true;
                        break;
                    }
                    // the first never-filled slot, else the least recently used one
                    if (!victim || (!sl.valid && victim->valid) ||
                        (sl.valid == victim->valid && sl.last_used < victim->last_used))
                        victim = &sl;
                }
                if (hit) continue;
                misses++;
                if (!victim->has_data) {
                    victim->has_data = true;
                    resident++;
                }
                if (victim->valid) evictions++;
                victim->layer = l;
                victim->expert = e;
                victim->last_used = ++clock;
                victim->valid = true;
            }
    stats[0] = hits;
    stats[1] = misses;
    stats[2] = evictions;
    stats[3] = misses * expert_stride;    // bytes_read: one stride per miss
    stats[4] = resident * expert_stride;  // resident_bytes
    stats[5] = cap * expert_stride;       // capacity_bytes
    return 1;
}

}  // extern "C"
