/*
 * ORACLE -- test infrastructure, not product code. See rbt2_oracle.h for the scope and for how
 * each function is pinned. Built with `gcc -O2 -std=c99 -ffp-contract=off` (oracle/Makefile),
 * the reference engine's own floating-point regime (rabbit2/Makefile:2).
 */
#define _POSIX_C_SOURCE 200809L
#define _FILE_OFFSET_BITS 64
#include "rbt2_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#if defined(__GNUC__) && (defined(__x86_64__) || defined(__i386__))
#define ORC_X86 1
#include <immintrin.h>
#else
#define ORC_X86 0
#endif

#define ORC_ALIGN 4096u /* header and expert blobs (rabbit2.c:56) */
#define ORC_TALIGN 64u  /* every other tensor (rabbit2.c:57) */
#define ORC_HEADER 68u  /* rabbit2.c:58 */
#define ORC_MAX_TOPK 64 /* rabbit2.c:59 */

static char g_err[256];
const char *orc_last_error(void) { return g_err; }
static int fail(const char *msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return 0;
}

/* ------------------------------------------------------------------ layout (rabbit2.c:158-193) */

static uint64_t align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

static uint64_t take(uint64_t *off, uint64_t nbytes) {
    *off = align_up(*off, ORC_TALIGN);
    uint64_t at = *off;
    *off += nbytes;
    return at;
}

void orc_layout(const orc_config *c, orc_model_off *m, orc_layer_off *layers) {
    const uint64_t E = c->dtype == ORC_DT_BF16 ? 2 : 4, F = 4;
    const uint64_t D = (uint64_t)c->dim;
    const uint64_t qd = (uint64_t)c->n_heads * c->head_dim, kvd = (uint64_t)c->n_kv_heads * c->head_dim;
    uint64_t off = ORC_ALIGN;
    m->tok_emb = take(&off, (uint64_t)c->vocab * D * E);
    m->expert_stride = align_up(3 * (uint64_t)c->expert_hidden * D * E, ORC_ALIGN);
    for (int l = 0; l < c->n_layers; l++) {
        orc_layer_off *ly = &layers[l];
        memset(ly, 0, sizeof *ly);
        ly->attn_norm = take(&off, D * F);
        ly->wq = take(&off, qd * D * E);
        ly->wk = take(&off, kvd * D * E);
        ly->wv = take(&off, kvd * D * E);
        ly->wo = take(&off, D * qd * E);
        if (c->qk_norm) {
            ly->q_norm = take(&off, qd * F);
            ly->k_norm = take(&off, kvd * F);
        }
        ly->ffn_norm = take(&off, D * F);
        ly->router = take(&off, (uint64_t)c->n_experts * D * E);
        off = align_up(off, ORC_ALIGN);
        ly->experts = off;
        off += (uint64_t)c->n_experts * m->expert_stride;
    }
    m->final_norm = take(&off, D * F);
    m->lm_head = take(&off, (uint64_t)c->vocab * D * E);
    m->end = m->lm_head + (uint64_t)c->vocab * D * E; /* layout_end(), rabbit2.c:195-197 */
}

/* ------------------------------------------------------------------ bf16 (rabbit2.c:304-309, rbt2.py:106-113) */

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_f32_to_bf16(float f) {
    if (f != f) return 0x7FC0;
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u); /* round to nearest, ties to even (wraps like uint32 numpy) */
    return (uint16_t)(u >> 16);
}

void orc_f32_to_bf16_n(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_bf16(src[i]);
}

/* ------------------------------------------------------------------ matvec */

/* Scalar order, rabbit2.c:356-390: partials s0..s3 over columns i = 4m+j, tail into s0,
 * result (s0+s1)+(s2+s3). */
static void matvec_scalar(float *out, const void *W, int dtype, const float *x, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
        int i = 0;
        if (dtype == ORC_DT_F32) {
            const float *w = (const float *)W + (size_t)r * cols;
            for (; i + 3 < cols; i += 4) {
                s0 += w[i] * x[i];
                s1 += w[i + 1] * x[i + 1];
                s2 += w[i + 2] * x[i + 2];
                s3 += w[i + 3] * x[i + 3];
            }
            for (; i < cols; i++) s0 += w[i] * x[i];
        } else {
            const uint16_t *w = (const uint16_t *)W + (size_t)r * cols;
            for (; i + 3 < cols; i += 4) {
                s0 += orc_bf16_to_f32(w[i]) * x[i];
                s1 += orc_bf16_to_f32(w[i + 1]) * x[i + 1];
                s2 += orc_bf16_to_f32(w[i + 2]) * x[i + 2];
                s3 += orc_bf16_to_f32(w[i + 3]) * x[i + 3];
            }
            for (; i < cols; i++) s0 += orc_bf16_to_f32(w[i]) * x[i];
        }
        out[r] = (s0 + s1) + (s2 + s3);
    }
}

static inline float welem(const void *W, int dtype, size_t k) {
    return dtype == ORC_DT_F32 ? ((const float *)W)[k] : orc_bf16_to_f32(((const uint16_t *)W)[k]);
}

/* AVX2 order, rabbit2.c:323-353, written lane by lane: accumulator a[j] takes column 16m+j,
 * b[j] takes 16m+8+j (each step adds the rounded product); then lanes = a+b, a sequential sum of
 * the 8 lanes starting from 0, then the scalar tail. Portable form of the same order. */
static void matvec_lane16(float *out, const void *W, int dtype, const float *x, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        const size_t base = (size_t)r * cols;
        float a[8] = {0, 0, 0, 0, 0, 0, 0, 0}, b[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int i = 0;
        for (; i + 15 < cols; i += 16) {
            for (int j = 0; j < 8; j++) {
                float p = welem(W, dtype, base + i + j) * x[i + j];
                float q = welem(W, dtype, base + i + 8 + j) * x[i + 8 + j];
                a[j] = a[j] + p;
                b[j] = b[j] + q;
            }
        }
        float sum = 0.0f;
        for (int j = 0; j < 8; j++) sum += a[j] + b[j];
        for (; i < cols; i++) sum += welem(W, dtype, base + i) * x[i];
        out[r] = sum;
    }
}

#if ORC_X86
/* The same order with AVX2 registers (no FMA), so the CPU baseline runs at the speed of the
 * reference's vector kernel. Bitwise equal to matvec_lane16 (tested). */
__attribute__((target("avx2,no-fma"))) static void matvec_avx2(float *out, const void *W, int dtype, const float *x,
                                                                int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        const size_t base = (size_t)r * cols;
        __m256 a = _mm256_setzero_ps(), b = _mm256_setzero_ps();
        int i = 0;
        if (dtype == ORC_DT_F32) {
            const float *w = (const float *)W + base;
            for (; i + 15 < cols; i += 16) {
                a = _mm256_add_ps(a, _mm256_mul_ps(_mm256_loadu_ps(w + i), _mm256_loadu_ps(x + i)));
                b = _mm256_add_ps(b, _mm256_mul_ps(_mm256_loadu_ps(w + i + 8), _mm256_loadu_ps(x + i + 8)));
            }
        } else {
            const uint16_t *w = (const uint16_t *)W + base;
            for (; i + 15 < cols; i += 16) {
                __m256i lo = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)(const void *)(w + i)));
                __m256i hi = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)(const void *)(w + i + 8)));
                __m256 w0 = _mm256_castsi256_ps(_mm256_slli_epi32(lo, 16));
                __m256 w1 = _mm256_castsi256_ps(_mm256_slli_epi32(hi, 16));
                a = _mm256_add_ps(a, _mm256_mul_ps(w0, _mm256_loadu_ps(x + i)));
                b = _mm256_add_ps(b, _mm256_mul_ps(w1, _mm256_loadu_ps(x + i + 8)));
            }
        }
        float lanes[8];
        _mm256_storeu_ps(lanes, _mm256_add_ps(a, b));
        float sum = 0.0f;
        for (int j = 0; j < 8; j++) sum += lanes[j];
        for (; i < cols; i++) sum += welem(W, dtype, base + i) * x[i];
        out[r] = sum;
    }
}

static int have_avx2(void) {
    static int cached = -1;
    if (cached < 0) {
        __builtin_cpu_init();
        cached = __builtin_cpu_supports("avx2") != 0;
    }
    return cached;
}
#endif

/* order 2 = the portable lane-by-lane form of the AVX2 order (for testing the vector form). */
void orc_matvec(float *out, const void *W, int dtype, const float *x, int rows, int cols, int order) {
    if (order == ORC_ORDER_SCALAR) {
        matvec_scalar(out, W, dtype, x, rows, cols);
        return;
    }
#if ORC_X86
    if (order == ORC_ORDER_AVX2 && have_avx2()) {
        matvec_avx2(out, W, dtype, x, rows, cols);
        return;
    }
#endif
    matvec_lane16(out, W, dtype, x, rows, cols);
}

/* ------------------------------------------------------------------ elementwise (rabbit2.c:392-407) */

void orc_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

void orc_softmax(float *x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    for (int i = 0; i < n; i++) x[i] /= sum;
}

float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* rabbit2.c:516-528 */
void orc_topk(const float *probs, int n, int k, unsigned char *used, int32_t *idx, float *wt, float *wsum) {
    float s = 0.0f;
    memset(used, 0, (size_t)n);
    for (int j = 0; j < k; j++) {
        int best = -1;
        for (int e = 0; e < n; e++)
            if (!used[e] && (best < 0 || probs[e] > probs[best])) best = e;
        used[best] = 1;
        idx[j] = best;
        wt[j] = probs[best];
        s += wt[j];
    }
    *wsum = s;
}

/* rope, rabbit2.c:409-423 (attention half; used by orc_run only) */
static void rope(float *v, int heads, int head_dim, int pos, float theta) {
    int half = head_dim / 2;
    for (int h = 0; h < heads; h++) {
        float *p = v + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            double freq = pow((double)theta, -2.0 * i / head_dim);
            double ang = pos * freq;
            float cs = (float)cos(ang), sn = (float)sin(ang);
            float a = p[i], b = p[i + half];
            p[i] = a * cs - b * sn;
            p[i + half] = b * cs + a * sn;
        }
    }
}

/* ------------------------------------------------------------------ MoE block (rabbit2.c:513-542) */

typedef struct {
    float *probs, *h1, *h3, *tmp, *moe;
    unsigned char *used;
} moe_scratch;

static int scratch_alloc(moe_scratch *s, int E, int H, int D) {
    s->probs = (float *)malloc(sizeof(float) * (size_t)E);
    s->h1 = (float *)malloc(sizeof(float) * (size_t)H);
    s->h3 = (float *)malloc(sizeof(float) * (size_t)H);
    s->tmp = (float *)malloc(sizeof(float) * (size_t)D);
    s->moe = (float *)malloc(sizeof(float) * (size_t)D);
    s->used = (unsigned char *)malloc((size_t)E);
    return s->probs && s->h1 && s->h3 && s->tmp && s->moe && s->used;
}

static void scratch_free(moe_scratch *s) {
    free(s->probs);
    free(s->h1);
    free(s->h3);
    free(s->tmp);
    free(s->moe);
    free(s->used);
}

/* One token. Leaves the block output in s->moe; routing/weights receive top_k entries. */
static void moe_token(const orc_moe_desc *d, const float *xb, int order, moe_scratch *s, int32_t *routing,
                      float *weights) {
    const int D = d->dim, E = d->n_experts, K = d->top_k, H = d->expert_hidden;
    const size_t esz = d->dtype == ORC_DT_BF16 ? 2 : 4;
    orc_matvec(s->probs, d->router, d->dtype, xb, E, D, order);
    if (d->router_bias)
        for (int e = 0; e < E; e++) s->probs[e] += d->router_bias[e];
    orc_softmax(s->probs, E);
    int32_t idx[ORC_MAX_TOPK];
    float wt[ORC_MAX_TOPK], wsum;
    orc_topk(s->probs, E, K, s->used, idx, wt, &wsum);
    memset(s->moe, 0, sizeof(float) * (size_t)D);
    for (int k = 0; k < K; k++) {
        const unsigned char *eb = d->experts + (size_t)idx[k] * d->expert_stride;
        const size_t mat = (size_t)H * D * esz;
        orc_matvec(s->h1, eb, d->dtype, xb, H, D, order);
        orc_matvec(s->h3, eb + mat, d->dtype, xb, H, D, order);
        for (int i = 0; i < H; i++) s->h1[i] = orc_silu(s->h1[i]) * s->h3[i];
        orc_matvec(s->tmp, eb + 2 * mat, d->dtype, s->h1, D, H, order);
        const float wk = d->norm_topk ? wt[k] / wsum : wt[k];
        for (int i = 0; i < D; i++) s->moe[i] += wk * s->tmp[i];
        if (routing) routing[k] = idx[k];
        if (weights) weights[k] = wk;
    }
}

int orc_moe_layer(const orc_moe_desc *d, const float *xb, int T, int order, float *x_inout, float *moe_out,
                  int32_t *routing, float *weights, float *probs_out) {
    if (!d || d->dim <= 0 || d->n_experts <= 0 || d->top_k <= 0 || d->top_k > d->n_experts ||
        d->top_k > ORC_MAX_TOPK || d->expert_hidden <= 0 || (d->dtype != ORC_DT_F32 && d->dtype != ORC_DT_BF16) ||
        T < 0)
        return fail("orc_moe_layer: bad descriptor");
    moe_scratch s;
    if (!scratch_alloc(&s, d->n_experts, d->expert_hidden, d->dim)) {
        scratch_free(&s);
        return fail("orc_moe_layer: out of memory");
    }
    const int D = d->dim, K = d->top_k, E = d->n_experts;
    for (int t = 0; t < T; t++) {
        moe_token(d, xb + (size_t)t * D, order, &s, routing ? routing + (size_t)t * K : NULL,
                  weights ? weights + (size_t)t * K : NULL);
        if (probs_out) memcpy(probs_out + (size_t)t * E, s.probs, sizeof(float) * (size_t)E);
        if (moe_out) memcpy(moe_out + (size_t)t * D, s.moe, sizeof(float) * (size_t)D);
        if (x_inout)
            for (int i = 0; i < D; i++) x_inout[(size_t)t * D + i] += s.moe[i];
    }
    scratch_free(&s);
    return 1;
}

/* ------------------------------------------------------------------ full engine (rabbit2.c:199-228, 425-548, 684-740) */

int orc_parse_header(const unsigned char *file, uint64_t file_size, orc_config *c) {
    if (file_size < ORC_HEADER || memcmp(file, "RBT2", 4) != 0) return fail("bad magic: not a .rbt2 file");
    uint32_t version;
    memcpy(&version, file + 4, 4);
    if (version != 2) return fail("unsupported .rbt2 version");
    memcpy(c, file + 8, sizeof *c);
    if (c->vocab <= 0 || c->dim <= 0 || c->n_layers <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 ||
        c->head_dim <= 0 || c->n_experts <= 0 || c->expert_hidden <= 0 || c->max_seq <= 0 || c->top_k <= 0 ||
        c->top_k > c->n_experts || c->top_k > ORC_MAX_TOPK || c->head_dim % 2 != 0 ||
        c->n_heads % c->n_kv_heads != 0 || (c->dtype != ORC_DT_F32 && c->dtype != ORC_DT_BF16))
        return fail("invalid config in header");
    return 1;
}

typedef struct {
    orc_config c;
    orc_model_off m;
    orc_layer_off *ly;
    const unsigned char *base;
    int ctx;
    float *x, *xb, *q, *k, *v, *att, *attn_out, *logits, *kcache, *vcache;
    moe_scratch ms;
} engine;

static const float *VEC(const engine *g, uint64_t off) { return (const float *)(const void *)(g->base + off); }

static int forward(engine *g, int token, int pos, int32_t *routing_out, int order) {
    const orc_config *c = &g->c;
    const int hd = c->head_dim, qd = c->n_heads * hd, kvd = c->n_kv_heads * hd;
    const int group = c->n_heads / c->n_kv_heads, D = c->dim;
    if (c->dtype == ORC_DT_F32) {
        memcpy(g->x, g->base + g->m.tok_emb + (size_t)token * D * 4, (size_t)D * 4);
    } else {
        const uint16_t *row = (const uint16_t *)(const void *)(g->base + g->m.tok_emb) + (size_t)token * D;
        for (int i = 0; i < D; i++) g->x[i] = orc_bf16_to_f32(row[i]);
    }
    for (int l = 0; l < c->n_layers; l++) {
        const orc_layer_off *ly = &g->ly[l];
        orc_rmsnorm(g->xb, g->x, VEC(g, ly->attn_norm), D, c->rms_eps);
        orc_matvec(g->q, g->base + ly->wq, c->dtype, g->xb, qd, D, order);
        orc_matvec(g->k, g->base + ly->wk, c->dtype, g->xb, kvd, D, order);
        orc_matvec(g->v, g->base + ly->wv, c->dtype, g->xb, kvd, D, order);
        if (c->qk_norm) {
            orc_rmsnorm(g->q, g->q, VEC(g, ly->q_norm), qd, c->rms_eps);
            orc_rmsnorm(g->k, g->k, VEC(g, ly->k_norm), kvd, c->rms_eps);
        }
        rope(g->q, c->n_heads, hd, pos, c->rope_theta);
        rope(g->k, c->n_kv_heads, hd, pos, c->rope_theta);
        float *kc = g->kcache + (size_t)l * g->ctx * kvd;
        float *vc = g->vcache + (size_t)l * g->ctx * kvd;
        memcpy(kc + (size_t)pos * kvd, g->k, (size_t)kvd * 4);
        memcpy(vc + (size_t)pos * kvd, g->v, (size_t)kvd * 4);
        const float scale = 1.0f / sqrtf((float)hd);
        for (int h = 0; h < c->n_heads; h++) {
            const float *qh = g->q + (size_t)h * hd;
            const int kvh = h / group;
            for (int t = 0; t <= pos; t++) {
                const float *kt = kc + (size_t)t * kvd + (size_t)kvh * hd;
                float dot = 0.0f;
                for (int i = 0; i < hd; i++) dot += qh[i] * kt[i];
                g->att[t] = dot * scale;
            }
            orc_softmax(g->att, pos + 1);
            float *out = g->attn_out + (size_t)h * hd;
            memset(out, 0, (size_t)hd * 4);
            for (int t = 0; t <= pos; t++) {
                const float *vt = vc + (size_t)t * kvd + (size_t)kvh * hd;
                const float a = g->att[t];
                for (int i = 0; i < hd; i++) out[i] += a * vt[i];
            }
        }
        orc_matvec(g->xb, g->base + ly->wo, c->dtype, g->attn_out, D, qd, order);
        for (int i = 0; i < D; i++) g->x[i] += g->xb[i];

        orc_rmsnorm(g->xb, g->x, VEC(g, ly->ffn_norm), D, c->rms_eps);
        orc_moe_desc d = {c->dim, c->n_experts, c->top_k, c->expert_hidden, c->dtype, c->norm_topk,
                          g->base + ly->router, g->base + ly->experts, g->m.expert_stride, NULL};
        moe_token(&d, g->xb, order, &g->ms, routing_out + (size_t)l * c->top_k, NULL);
        for (int i = 0; i < D; i++) g->x[i] += g->ms.moe[i];
    }
    orc_rmsnorm(g->xb, g->x, VEC(g, g->m.final_norm), D, c->rms_eps);
    orc_matvec(g->logits, g->base + g->m.lm_head, c->dtype, g->xb, c->vocab, D, order);
    return 1;
}

static int argmax(const float *v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* ---- sampling, rabbit2.c:558-610: xorshift64* state (a zero state counts as the golden-ratio
 * constant), uniform doubles from its top 53 bits, and sample_logits: temperature, top-k by K rounds
 * of "largest remaining, first index on ties" swapped to the front, softmax over the kept values
 * (max-subtract, expf, sequential sum, divide), top-p over the kept order, then the first position
 * whose running double sum exceeds the draw. */
uint64_t orc_rng_next(uint64_t *s) {
    uint64_t x = *s ? *s : 0x9E3779B97F4A7C15ULL;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *s = x;
    return x * 2685821657736338717ULL;
}

double orc_rng_uniform(uint64_t *s) { return (double)(orc_rng_next(s) >> 11) * (1.0 / 9007199254740992.0); }

int orc_sample(const float *logits, int n, float temperature, int top_k, float top_p, uint64_t *rng, int32_t *idx,
               float *prob) {
    if (temperature <= 0.0f) return argmax(logits, n);
    for (int i = 0; i < n; i++) {
        idx[i] = i;
        prob[i] = logits[i] / temperature;
    }
    const int use_k = top_k > 0 && top_k < n;
    if (use_k) {
        for (int i = 0; i < top_k; i++) {
            int best = i;
            for (int j = i + 1; j < n; j++)
                if (prob[j] > prob[best]) best = j;
            const float tp = prob[i];
            prob[i] = prob[best];
            prob[best] = tp;
            const int32_t ti = idx[i];
            idx[i] = idx[best];
            idx[best] = ti;
        }
        for (int i = top_k; i < n; i++) prob[i] = -INFINITY;
    }
    float mx = -INFINITY;
    for (int i = 0; i < n; i++)
        if (prob[i] > mx) mx = prob[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        if (isfinite(prob[i])) {
            prob[i] = expf(prob[i] - mx);
            sum += prob[i];
        } else {
            prob[i] = 0.0f;
        }
    }
    if (!(sum > 0.0f)) return argmax(logits, n);
    for (int i = 0; i < n; i++) prob[i] /= sum;
    if (top_p > 0.0f && top_p < 1.0f) {
        const int m = use_k ? top_k : n;
        float cum = 0.0f;
        int keep = m;
        for (int i = 0; i < m; i++) {
            cum += prob[i];
            if (cum >= top_p) {
                keep = i + 1;
                break;
            }
        }
        for (int i = keep; i < n; i++) prob[i] = 0.0f;
        sum = 0.0f;
        for (int i = 0; i < n; i++) sum += prob[i];
        if (!(sum > 0.0f)) return idx[0];
        for (int i = 0; i < n; i++) prob[i] /= sum;
    }
    const double r = orc_rng_uniform(rng);
    double cum = 0.0;
    for (int i = 0; i < n; i++) {
        cum += prob[i];
        if (r < cum) return idx[i];
    }
    for (int i = n - 1; i >= 0; i--)
        if (prob[i] > 0.0f) return idx[i];
    return argmax(logits, n);
}

static void engine_free(engine *g) {
    free(g->ly);
    free(g->x);
    free(g->xb);
    free(g->q);
    free(g->k);
    free(g->v);
    free(g->att);
    free(g->attn_out);
    free(g->logits);
    free(g->kcache);
    free(g->vcache);
    scratch_free(&g->ms);
}

int orc_run(const unsigned char *file, uint64_t file_size, const int32_t *tokens, int nt, int ctx, int order,
            float *logits, int32_t *routing, int gen, int32_t eos, int32_t *gen_out, int *n_gen) {
    return orc_run_sampled(file, file_size, tokens, nt, ctx, order, logits, routing, gen, eos, gen_out, n_gen, 0.0f, 0,
                           1.0f, 0);
}

int orc_run_sampled(const unsigned char *file, uint64_t file_size, const int32_t *tokens, int nt, int ctx, int order,
                    float *logits, int32_t *routing, int gen, int32_t eos, int32_t *gen_out, int *n_gen,
                    float temperature, int top_k, float top_p, uint64_t seed) {
    engine g;
    memset(&g, 0, sizeof g);
    if (n_gen) *n_gen = 0;
    if (!orc_parse_header(file, file_size, &g.c)) return 0;
    const orc_config *c = &g.c;
    g.ly = (orc_layer_off *)calloc((size_t)c->n_layers, sizeof *g.ly);
    if (!g.ly) return fail("out of memory");
    orc_layout(c, &g.m, g.ly);
    if (g.m.end > file_size) {
        free(g.ly);
        return fail("file too small for its own config");
    }
    g.base = file;
    if (ctx <= 0) ctx = c->max_seq < 512 ? c->max_seq : 512;
    if (ctx > c->max_seq) ctx = c->max_seq;
    if (nt < 1 || nt > ctx) {
        free(g.ly);
        return fail("prompt longer than context");
    }
    for (int i = 0; i < nt; i++)
        if (tokens[i] < 0 || tokens[i] >= c->vocab) {
            free(g.ly);
            return fail("token out of range");
        }
    g.ctx = ctx;
    const int qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
    g.x = (float *)calloc((size_t)c->dim, 4);
    g.xb = (float *)calloc((size_t)c->dim, 4);
    g.q = (float *)calloc((size_t)qd, 4);
    g.k = (float *)calloc((size_t)kvd, 4);
    g.v = (float *)calloc((size_t)kvd, 4);
    g.att = (float *)calloc((size_t)ctx, 4);
    g.attn_out = (float *)calloc((size_t)qd, 4);
    g.logits = (float *)calloc((size_t)c->vocab, 4);
    g.kcache = (float *)calloc((size_t)c->n_layers * ctx * kvd, 4);
    g.vcache = (float *)calloc((size_t)c->n_layers * ctx * kvd, 4);
    int ok = scratch_alloc(&g.ms, c->n_experts, c->expert_hidden, c->dim);
    if (!ok || !g.x || !g.xb || !g.q || !g.k || !g.v || !g.att || !g.attn_out || !g.logits || !g.kcache ||
        !g.vcache) {
        engine_free(&g);
        return fail("out of memory");
    }
    const size_t LK = (size_t)c->n_layers * c->top_k;
    int32_t *rt = (int32_t *)calloc(LK, sizeof(int32_t));
    if (!rt) {
        engine_free(&g);
        return fail("out of memory");
    }
    for (int i = 0; i < nt; i++) {
        forward(&g, tokens[i], i, rt, order);
        if (logits) memcpy(logits + (size_t)i * c->vocab, g.logits, (size_t)c->vocab * 4);
        if (routing) memcpy(routing + (size_t)i * LK, rt, LK * sizeof(int32_t));
    }
    if (gen > 0) {
        if (gen > ctx - nt) gen = ctx - nt;
        int pos = nt, produced = 0;
        uint64_t rng = seed ? seed : 0x9E3779B97F4A7C15ULL; /* rabbit2.c:723 */
        int32_t *sidx = (int32_t *)malloc(sizeof(int32_t) * (size_t)c->vocab);
        float *sprob = (float *)malloc(sizeof(float) * (size_t)c->vocab);
        if (!sidx || !sprob) {
            free(sidx);
            free(sprob);
            free(rt);
            engine_free(&g);
            return fail("out of memory");
        }
        for (int j = 0; j < gen; j++) {
            int next = orc_sample(g.logits, c->vocab, temperature, top_k, top_p, &rng, sidx, sprob);
            if (gen_out) gen_out[produced] = next;
            produced++;
            if (next == eos) break;
            if (j + 1 == gen) break;
            forward(&g, next, pos++, rt, order);
        }
        if (n_gen) *n_gen = produced;
        free(sidx);
        free(sprob);
    }
    free(rt);
    engine_free(&g);
    return 1;
}

/* ------------------------------------------------------------------ generator + writer */

#define GOLDEN 0x9E3779B97F4A7C15ULL

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t orc_splitmix64_next(uint64_t *state) {
    *state += GOLDEN;
    return mix64(*state);
}

/* Both samples of pair p of a stream: z[0] = r cos(th) (even index), z[1] = r sin(th) (odd). */
static void normal_pair(uint64_t key, uint64_t p, double z[2]) {
    const uint64_t o1 = mix64(key + (2 * p + 1) * GOLDEN); /* output 2p of the sequence at key */
    const uint64_t o2 = mix64(key + (2 * p + 2) * GOLDEN); /* output 2p+1 */
    const double u1 = ((double)(o1 >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(o2 >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    const double th = 6.283185307179586 * u2;
    z[0] = r * cos(th);
    z[1] = r * sin(th);
}

static uint64_t stream_key(uint64_t seed, uint64_t stream) {
    uint64_t s = seed ^ (stream * GOLDEN);
    return orc_splitmix64_next(&s);
}

double orc_normal(uint64_t seed, uint64_t stream, uint64_t i) {
    double z[2];
    normal_pair(stream_key(seed, stream), i >> 1, z);
    return z[i & 1];
}

static void store_one(void *dst, int dtype, uint64_t i, double z, float scale, float offset) {
    const float v = (float)((double)offset + (double)scale * z);
    if (dtype == ORC_DT_F32)
        ((float *)dst)[i] = v;
    else
        ((uint16_t *)dst)[i] = orc_f32_to_bf16(v);
}

void orc_fill_normal(void *dst, int dtype, uint64_t n, uint64_t seed, uint64_t stream, uint64_t first, float scale,
                     float offset) {
    const uint64_t key = stream_key(seed, stream);
    double z[2];
    uint64_t i = 0;
    while (i < n) {
        const uint64_t g = first + i;
        normal_pair(key, g >> 1, z);
        store_one(dst, dtype, i, z[g & 1], scale, offset);
        i++;
        if ((g & 1) == 0 && i < n) {
            store_one(dst, dtype, i, z[1], scale, offset);
            i++;
        }
    }
}

uint64_t orc_layer_stream(int layer, int which) { return 16u + 16u * (uint64_t)layer + (uint64_t)which; }

uint64_t orc_expert_stream(const orc_config *c, int layer, int e, int which) {
    return (1ULL << 32) | (((uint64_t)layer * (uint64_t)c->n_experts + (uint64_t)e) * 3u + (uint64_t)which);
}

uint64_t orc_model_file_size(const orc_config *c) {
    orc_layer_off *ly = (orc_layer_off *)calloc((size_t)(c->n_layers > 0 ? c->n_layers : 1), sizeof *ly);
    orc_model_off m;
    if (!ly) return 0;
    orc_layout(c, &m, ly);
    free(ly);
    return align_up(m.end, ORC_ALIGN);
}

typedef int (*put_fn)(void *ctx, uint64_t off, const void *data, uint64_t n);

static int put_buf(void *ctx, uint64_t off, const void *data, uint64_t n) {
    unsigned char **b = (unsigned char **)ctx;
    memcpy(*b + off, data, (size_t)n);
    return 1;
}

static int put_file(void *ctx, uint64_t off, const void *data, uint64_t n) {
    FILE *f = (FILE *)ctx;
    if (fseeko(f, (off_t)off, SEEK_SET) != 0) return 0;
    return fwrite(data, 1, (size_t)n, f) == (size_t)n;
}

/* Writes one tensor in chunks so large matrices never need a full host copy. */
static int put_tensor(put_fn put, void *ctx, uint64_t off, int dtype, uint64_t n, uint64_t seed, uint64_t stream,
                      float scale, float offset) {
    enum { CH = 1 << 16 };
    static float fbuf[CH];
    const uint64_t esz = dtype == ORC_DT_BF16 ? 2 : 4;
    for (uint64_t i = 0; i < n; i += CH) {
        const uint64_t m = n - i < CH ? n - i : CH;
        orc_fill_normal(fbuf, dtype, m, seed, stream, i, scale, offset);
        if (!put(ctx, off + i * esz, fbuf, m * esz)) return 0;
    }
    return 1;
}

static int build_any(put_fn put, void *ctx, const orc_config *c, const orc_gen_params *g) {
    orc_layer_off *ly = (orc_layer_off *)calloc((size_t)c->n_layers, sizeof *ly);
    orc_model_off m;
    if (!ly) return fail("out of memory");
    orc_layout(c, &m, ly);
    unsigned char hdr[ORC_HEADER];
    memcpy(hdr, "RBT2", 4);
    const uint32_t version = 2;
    memcpy(hdr + 4, &version, 4);
    memcpy(hdr + 8, c, sizeof *c);
    int ok = put(ctx, 0, hdr, ORC_HEADER);
    const int dt = c->dtype;
    const uint64_t D = (uint64_t)c->dim, H = (uint64_t)c->expert_hidden;
    const uint64_t qd = (uint64_t)c->n_heads * c->head_dim, kvd = (uint64_t)c->n_kv_heads * c->head_dim;
#define MSCALE(cols) (g->fan_in_scale ? (float)((double)g->w_scale / sqrt((double)(cols))) : g->w_scale)
    ok = ok && put_tensor(put, ctx, m.tok_emb, dt, (uint64_t)c->vocab * D, g->seed, 1, g->emb_scale, 0.0f);
    for (int l = 0; l < c->n_layers && ok; l++) {
        const orc_layer_off *o = &ly[l];
        ok = ok && put_tensor(put, ctx, o->attn_norm, ORC_DT_F32, D, g->seed, orc_layer_stream(l, 0), g->norm_jitter, 1.0f);
        ok = ok && put_tensor(put, ctx, o->wq, dt, qd * D, g->seed, orc_layer_stream(l, 1), MSCALE(D), 0.0f);
        ok = ok && put_tensor(put, ctx, o->wk, dt, kvd * D, g->seed, orc_layer_stream(l, 2), MSCALE(D), 0.0f);
        ok = ok && put_tensor(put, ctx, o->wv, dt, kvd * D, g->seed, orc_layer_stream(l, 3), MSCALE(D), 0.0f);
        ok = ok && put_tensor(put, ctx, o->wo, dt, D * qd, g->seed, orc_layer_stream(l, 4), MSCALE(qd), 0.0f);
        if (c->qk_norm) {
            ok = ok && put_tensor(put, ctx, o->q_norm, ORC_DT_F32, qd, g->seed, orc_layer_stream(l, 5), g->norm_jitter, 1.0f);
            ok = ok && put_tensor(put, ctx, o->k_norm, ORC_DT_F32, kvd, g->seed, orc_layer_stream(l, 6), g->norm_jitter, 1.0f);
        }
        ok = ok && put_tensor(put, ctx, o->ffn_norm, ORC_DT_F32, D, g->seed, orc_layer_stream(l, 7), g->norm_jitter, 1.0f);
        ok = ok && put_tensor(put, ctx, o->router, dt, (uint64_t)c->n_experts * D, g->seed, orc_layer_stream(l, 8),
                              MSCALE(D), 0.0f);
        const uint64_t esz = dt == ORC_DT_BF16 ? 2 : 4;
        for (int e = 0; e < c->n_experts && ok; e++) {
            const uint64_t eb = o->experts + (uint64_t)e * m.expert_stride;
            ok = ok && put_tensor(put, ctx, eb, dt, H * D, g->seed, orc_expert_stream(c, l, e, 0), MSCALE(D), 0.0f);
            ok = ok && put_tensor(put, ctx, eb + H * D * esz, dt, H * D, g->seed, orc_expert_stream(c, l, e, 1), MSCALE(D), 0.0f);
            ok = ok && put_tensor(put, ctx, eb + 2 * H * D * esz, dt, D * H, g->seed, orc_expert_stream(c, l, e, 2),
                                  MSCALE(H), 0.0f);
        }
    }
    ok = ok && put_tensor(put, ctx, m.final_norm, ORC_DT_F32, D, g->seed, 2, g->norm_jitter, 1.0f);
    ok = ok && put_tensor(put, ctx, m.lm_head, dt, (uint64_t)c->vocab * D, g->seed, 3, MSCALE(D), 0.0f);
#undef MSCALE
    free(ly);
    return ok ? 1 : fail("cannot write model");
}

int orc_build_model(unsigned char *buf, uint64_t size, const orc_config *c, const orc_gen_params *g) {
    if (size < orc_model_file_size(c)) return fail("buffer too small");
    unsigned char *b = buf;
    return build_any(put_buf, &b, c, g);
}

int orc_write_model(const char *path, const orc_config *c, const orc_gen_params *g) {
    FILE *f = fopen(path, "wb");
    if (!f) return fail("cannot open output file");
    int ok = build_any(put_file, f, c, g);
    if (fclose(f) != 0) ok = 0;
    /* extend to the 4 KiB-rounded size with zeros, as the reference writer's truncate() does (rbt2.py:141) */
    if (ok && truncate(path, (off_t)orc_model_file_size(c)) != 0) ok = 0;
    return ok ? 1 : fail("cannot write model");
}
