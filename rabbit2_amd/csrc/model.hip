// The rest of the engine's per-token forward pass on the GPU, around the MoE block: token embedding,
// RMSNorm, the q/k/v, wo and lm_head matvecs, QK-norm, RoPE, the KV cache in HBM, attention, and the
// greedy argmax. Reference: rabbit2/src/rabbit2.c:453-548 (forward), :392-397 (rmsnorm), :399-405
// (softmax), :410-423 (rope), :552-556 (argmax), :703-740 (the prompt and --gen loops).
//
// Every kernel reads the token and position of the step from a small device record (StepState), so
// one captured step replays unchanged for every position: the prompt's tokens sit in seq[] before the
// first step, and the argmax kernel appends each generated token to seq[] and advances pos.
//
// Arithmetic follows the engine's formulas (rmsnorm as x * inv * w with inv = 1/sqrtf(ss/n + eps);
// RoPE angles in double, rounded to float; softmax with max-subtract and expf; strict '>' argmax). Sums
// run in parallel orders, so results agree with the engine to rounding, not bit for bit; the MoE router
// keeps its exact order (router.hip).
#include <math.h>

#include "rbt2_internal.h"

namespace rbt {
namespace {

// block-wide sum of one float per thread (blockDim.x a multiple of 64, at most 1024)
__device__ __forceinline__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_sum(v);
    __syncthreads();  // red may still be read by a previous call
    if (lane == 0) red[wv] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}

// inv = 1 / sqrtf(sum(x^2) / n + eps), rabbit2.c:394-395
__device__ __forceinline__ float rms_inv(const float *__restrict__ x, int n, float eps, float *red) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum(ss, red);
    return 1.0f / sqrtf(ss / (float)n + eps);
}

template <int DT>
__device__ __forceinline__ float elem(const uint8_t *W, size_t i) {
    return load_w<DT>(W, i);
}

// dot of one weight row (cols elements of DT) with x in LDS, summed over the wave
template <int DT, bool VEC>
__device__ __forceinline__ float row_dot(const uint8_t *__restrict__ row, const float *xs, int cols, int lane) {
    float acc = 0.0f;
    if constexpr (VEC) {
        constexpr int per = DT == RBT_DT_BF16 ? 8 : 4;
        for (int c = lane * per; c < cols; c += kWave * per) {
            const u32x4 w = ld_stream_u4(row + (size_t)c * (DT == RBT_DT_BF16 ? 2 : 4));
            if constexpr (DT == RBT_DT_BF16) {
                const f32x4 x0 = *reinterpret_cast<const f32x4 *>(xs + c);
                const f32x4 x1 = *reinterpret_cast<const f32x4 *>(xs + c + 4);
                acc += bf16_lo(w.x) * x0.x + bf16_hi(w.x) * x0.y + bf16_lo(w.y) * x0.z + bf16_hi(w.y) * x0.w +
                       bf16_lo(w.z) * x1.x + bf16_hi(w.z) * x1.y + bf16_lo(w.w) * x1.z + bf16_hi(w.w) * x1.w;
            } else {
                const f32x4 x0 = *reinterpret_cast<const f32x4 *>(xs + c);
                acc += __uint_as_float(w.x) * x0.x + __uint_as_float(w.y) * x0.y + __uint_as_float(w.z) * x0.z +
                       __uint_as_float(w.w) * x0.w;
            }
        }
    } else {
        for (int c = lane; c < cols; c += kWave) acc += elem<DT>(row, (size_t)c) * xs[c];
    }
    return wave_sum(acc);
}

// ---------------------------------------------------------------- embedding (rabbit2.c:460-466)
template <int DT>
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t *__restrict__ emb, int D, int vocab,
                                                    const StepState *__restrict__ st, const int32_t *__restrict__ seq,
                                                    float *__restrict__ x) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= D) return;
    int tok = seq[st->pos];
    tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);  // ids are checked on the host; generated ids are in range
    x[i] = elem<DT>(emb, (size_t)tok * D + i);
}

// ---------------------------------------------------------------- RMSNorm + matvec
// out_s[r] = W_s[r] . (x * inv * w) for up to three weight segments (q, k, v share one launch).
// One row per wave; every block recomputes the norm of x (D floats from L2) into LDS.
struct Segs {
    const uint8_t *W[3];
    float *out[3];
    int rows[3];
};

template <int DT, bool VEC>
__global__ __launch_bounds__(256) void norm_matvec_kernel(const float *__restrict__ x, const float *__restrict__ nw,
                                                          float eps, int D, Segs sg, int total_rows) {
    extern __shared__ __align__(16) float xs[];
    __shared__ float red[16];
    const float inv = rms_inv(x, D, eps, red);
    for (int i = threadIdx.x; i < D; i += blockDim.x) xs[i] = x[i] * inv * nw[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    int r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (r >= total_rows) return;
    int s = 0;
    while (s < 2 && r >= sg.rows[s]) {
        r -= sg.rows[s];
        ++s;
    }
    constexpr size_t esz = DT == RBT_DT_BF16 ? 2 : 4;
    const float v = row_dot<DT, VEC>(sg.W[s] + (size_t)r * D * esz, xs, D, lane);
    if (lane == 0) sg.out[s][r] = v;
}

// ---------------------------------------------------------------- attention, split over positions
// grid (n_heads, S). Block (h, s): QK-norm over the whole q and k projections (rabbit2.c:475-478),
// RoPE of head h's q and of its kv head's k at pos (:479-480), then positions t in its share of
// [0, pos]: scores q.k_t / sqrt(hd) (:486-492), local max m, l = sum exp(score - m), o = sum exp(score -
// m) v_t. The current position's k and v are used from registers; block (h, 0) of the first query head
// of each kv head appends them to the cache (:482-484). part[(h*S + s)*(hd + 2)]: m, l, o[hd].
__device__ __forceinline__ void rope_pair(float *p, int i, int half, int hd, int pos, float theta) {
#pragma clang fp contract(off)
    const double freq = pow((double)theta, -2.0 * i / hd);
    const double ang = pos * freq;
    const float cs = (float)cos(ang), sn = (float)sin(ang);
    const float a = p[i], b = p[i + half];
    p[i] = a * cs - b * sn;
    p[i + half] = b * cs + a * sn;
}

__global__ __launch_bounds__(256) void attn_kernel(const float *__restrict__ q_raw, const float *__restrict__ k_raw,
                                                   const float *__restrict__ v_raw, const float *__restrict__ qw,
                                                   const float *__restrict__ kw, int qk_norm, float eps, float theta,
                                                   int n_heads, int n_kv, int hd, int S, int ctx,
                                                   const StepState *__restrict__ st, float *__restrict__ kc,
                                                   float *__restrict__ vc, float *__restrict__ part) {
    extern __shared__ __align__(16) float sm[];  // q[hd], k[hd], v[hd], scores[chunk]
    __shared__ float red[16];
    float *qh = sm, *kh = sm + hd, *vh = sm + 2 * hd, *sc = sm + 3 * hd;
    const int h = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
    const int group = n_heads / n_kv, kvh = h / group;
    const int q_dim = n_heads * hd, kv_dim = n_kv * hd, half = hd / 2;
    const int pos = st->pos;
    float inv_q = 1.0f, inv_k = 1.0f;
    if (qk_norm) {
        inv_q = rms_inv(q_raw, q_dim, eps, red);
        inv_k = rms_inv(k_raw, kv_dim, eps, red);
    }
    for (int i = tid; i < hd; i += blockDim.x) {
        const int qi = h * hd + i, ki = kvh * hd + i;
        qh[i] = qk_norm ? q_raw[qi] * inv_q * qw[qi] : q_raw[qi];
        kh[i] = qk_norm ? k_raw[ki] * inv_k * kw[ki] : k_raw[ki];
        vh[i] = v_raw[ki];
    }
    __syncthreads();
    for (int i = tid; i < half; i += blockDim.x) {
        rope_pair(qh, i, half, hd, pos, theta);
        rope_pair(kh, i, half, hd, pos, theta);
    }
    __syncthreads();
    if (s == 0 && h % group == 0) {
        float *kd = kc + (size_t)pos * kv_dim + (size_t)kvh * hd, *vd = vc + (size_t)pos * kv_dim + (size_t)kvh * hd;
        for (int i = tid; i < hd; i += blockDim.x) {
            kd[i] = kh[i];
            vd[i] = vh[i];
        }
    }
    const int n = pos + 1;
    const int chunk = (n + S - 1) / S;
    const int t0 = s * chunk, t1 = min(n, t0 + chunk);
    float *po = part + ((size_t)h * S + s) * (hd + 2);
    if (t0 >= t1) {  // block-uniform: this split has no positions
        if (tid == 0) {
            po[0] = -INFINITY;
            po[1] = 0.0f;
        }
        for (int i = tid; i < hd; i += blockDim.x) po[2 + i] = 0.0f;
        return;
    }
    const float scale = 1.0f / sqrtf((float)hd);
    const int lane = tid & 63, wv = tid >> 6, nwv = blockDim.x >> 6;
    for (int t = t0 + wv; t < t1; t += nwv) {
        const float *kt = t == pos ? kh : kc + (size_t)t * kv_dim + (size_t)kvh * hd;
        float d = 0.0f;
        for (int i = lane; i < hd; i += kWave) d += qh[i] * kt[i];
        d = wave_sum(d);
        if (lane == 0) sc[t - t0] = d * scale;
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int t = tid; t < t1 - t0; t += blockDim.x) mx = fmaxf(mx, sc[t]);
    mx = wave_max(mx);
    __syncthreads();
    if (lane == 0) red[wv] = mx;
    __syncthreads();
    mx = red[0];
    for (int i = 1; i < nwv; ++i) mx = fmaxf(mx, red[i]);
    float l = 0.0f;
    for (int t = tid; t < t1 - t0; t += blockDim.x) {
        const float e = expf(sc[t] - mx);
        sc[t] = e;
        l += e;
    }
    l = block_sum(l, red);  // its leading barrier also publishes sc[]
    for (int i = tid; i < hd; i += blockDim.x) {
        float o = 0.0f;
        for (int t = t0; t < t1; ++t) {
            const float vt = t == pos ? vh[i] : vc[(size_t)t * kv_dim + (size_t)kvh * hd + i];
            o += sc[t - t0] * vt;
        }
        po[2 + i] = o;
    }
    if (tid == 0) {
        po[0] = mx;
        po[1] = l;
    }
}

// ---------------------------------------------------------------- attention combine
// Block h merges the S split partials of head h: M = max m_s, L = sum exp(m_s - M) l_s,
// attn_out[h*hd + i] = sum exp(m_s - M) o_s[i] / L (the engine's softmax-weighted sum, :493-498).
__global__ __launch_bounds__(256) void attn_combine_kernel(const float *__restrict__ part, int hd, int S,
                                                           float *__restrict__ ao) {
    const int h = blockIdx.x;
    const float *ph = part + (size_t)h * S * (hd + 2);
    float M = -INFINITY;
    for (int s = 0; s < S; ++s) M = fmaxf(M, ph[(size_t)s * (hd + 2)]);
    float L = 0.0f;
    for (int s = 0; s < S; ++s) {
        const float *p = ph + (size_t)s * (hd + 2);
        if (p[1] > 0.0f) L += expf(p[0] - M) * p[1];
    }
    const float invL = 1.0f / L;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) {
        float o = 0.0f;
        for (int s = 0; s < S; ++s) {
            const float *p = ph + (size_t)s * (hd + 2);
            if (p[1] > 0.0f) o += expf(p[0] - M) * p[2 + i];
        }
        ao[(size_t)h * hd + i] = o * invL;
    }
}

// ---------------------------------------------------------------- wo + residual
// x[r] += wo[r] . attn_out, one row per wave (rabbit2.c:500-501); attn_out staged in LDS per block.
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void wo_kernel(const float *__restrict__ ao, int q_dim, const uint8_t *__restrict__ Wo,
                                                 int D, float *__restrict__ x) {
    extern __shared__ __align__(16) float sm[];
    for (int j = threadIdx.x; j < q_dim; j += blockDim.x) sm[j] = ao[j];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (r >= D) return;
    constexpr size_t esz = DT == RBT_DT_BF16 ? 2 : 4;
    const float v = row_dot<DT, VEC>(Wo + (size_t)r * q_dim * esz, sm, q_dim, lane);
    if (lane == 0) x[r] = x[r] + v;
}

// ---------------------------------------------------------------- RMSNorm (one block)
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ w, int n,
                                                       float eps, float *__restrict__ out) {
    __shared__ float red[16];
    const float inv = rms_inv(x, n, eps, red);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * inv * w[i];
}

// ---------------------------------------------------------------- greedy argmax (rabbit2.c:552-556)
// best = 0; for i: if v[i] > v[best] best = i -- the first index of the largest value; a NaN never
// wins, and a NaN at index 0 is never beaten. Then the step advances: seq[pos + 1] = best when that
// slot is past the prompt (generation), pos += 1.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ v, int n, StepState *st,
                                                      int32_t *__restrict__ seq, int ctx) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    float best = -INFINITY;
    int idx = n;  // n: nothing found yet
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float a = v[i];
        if (a == a && (idx == n || a > best)) {  // first non-NaN, then strictly larger
            best = a;
            idx = i;
        }
    }
    // wave then block reduction on (value, index): larger value wins, equal values keep the lower index
    for (int off = 32; off > 0; off >>= 1) {
        const float ob = __shfl_down(best, off, 64);
        const int oi = __shfl_down(idx, off, 64);
        if (oi < n && (idx == n || ob > best || (ob == best && oi < idx))) {
            best = ob;
            idx = oi;
        }
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (lane == 0) {
        bv[wv] = best;
        bi[wv] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = -INFINITY;
        int k = n;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
            if (bi[w] < n && (k == n || bv[w] > b || (bv[w] == b && bi[w] < k))) {
                b = bv[w];
                k = bi[w];
            }
        }
        const float v0 = v[0];
        if (k == n || v0 != v0) k = 0;  // all NaN, or v[0] NaN: the engine's scan keeps index 0
        const int p = st->pos;
        st->last = k;
        if (p + 1 < ctx && p + 1 >= st->n_prompt) seq[p + 1] = k;
        st->pos = p + 1;
    }
}

// advances the step record without an argmax (prompt positions whose logits nobody reads)
__global__ void advance_kernel(StepState *st) {
    if (threadIdx.x == 0) st->pos = st->pos + 1;
}

inline bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

hipError_t launch_embed(const Launch &L, int dtype, const void *emb, int D, int vocab, const StepState *st,
                        const int32_t *seq, float *x) {
    const dim3 g((unsigned)((D + 255) / 256)), b(256);
    const uint8_t *e = static_cast<const uint8_t *>(emb);
    return dtype == RBT_DT_BF16 ? launch(L, embed_kernel<RBT_DT_BF16>, g, b, 0, e, D, vocab, st, seq, x)
                                : launch(L, embed_kernel<RBT_DT_F32>, g, b, 0, e, D, vocab, st, seq, x);
}

hipError_t launch_norm_matvec(const Launch &L, int dtype, const float *x, const float *nw, float eps, int D,
                              const void *const W[3], float *const out[3], const int rows[3]) {
    Segs sg;
    int total = 0;
    bool vec = dtype == RBT_DT_BF16 ? D % 8 == 0 : D % 4 == 0;
    for (int i = 0; i < 3; ++i) {
        sg.W[i] = static_cast<const uint8_t *>(W[i]);
        sg.out[i] = out[i];
        sg.rows[i] = rows[i];
        total += rows[i];
        if (rows[i] > 0) vec = vec && al16(W[i]);
    }
    if (total == 0) return hipSuccess;
    const dim3 g((unsigned)((total + 3) / 4)), b(256);
    const uint32_t lds = (uint32_t)(4 * (size_t)D);
    if (dtype == RBT_DT_BF16)
        return vec ? launch(L, norm_matvec_kernel<RBT_DT_BF16, true>, g, b, lds, x, nw, eps, D, sg, total)
                   : launch(L, norm_matvec_kernel<RBT_DT_BF16, false>, g, b, lds, x, nw, eps, D, sg, total);
    return vec ? launch(L, norm_matvec_kernel<RBT_DT_F32, true>, g, b, lds, x, nw, eps, D, sg, total)
               : launch(L, norm_matvec_kernel<RBT_DT_F32, false>, g, b, lds, x, nw, eps, D, sg, total);
}

size_t attn_lds_bytes(int hd, int ctx, int S) { return 4 * (3 * (size_t)hd + (size_t)((ctx + S - 1) / S)); }

hipError_t launch_attention(const Launch &L, const float *q, const float *k, const float *v, const float *qw,
                            const float *kw, int qk_norm, float eps, float theta, int n_heads, int n_kv, int hd, int S,
                            int ctx, const StepState *st, float *kc, float *vc, float *part) {
    return launch(L, attn_kernel, dim3((unsigned)n_heads, (unsigned)S), dim3(256), (uint32_t)attn_lds_bytes(hd, ctx, S),
                  q, k, v, qw, kw, qk_norm, eps, theta, n_heads, n_kv, hd, S, ctx, st, kc, vc, part);
}

hipError_t launch_attn_combine(const Launch &L, const float *part, int n_heads, int hd, int S, float *ao) {
    return launch(L, attn_combine_kernel, dim3((unsigned)n_heads), dim3(256), 0, part, hd, S, ao);
}

hipError_t launch_wo(const Launch &L, int dtype, const float *ao, int q_dim, const void *Wo, int D, float *x) {
    const bool vec = (dtype == RBT_DT_BF16 ? q_dim % 8 == 0 : q_dim % 4 == 0) && al16(Wo);
    const dim3 g((unsigned)((D + 3) / 4)), b(256);
    const uint32_t lds = (uint32_t)(4 * (size_t)q_dim);
    const uint8_t *W = static_cast<const uint8_t *>(Wo);
    if (dtype == RBT_DT_BF16)
        return vec ? launch(L, wo_kernel<RBT_DT_BF16, true>, g, b, lds, ao, q_dim, W, D, x)
                   : launch(L, wo_kernel<RBT_DT_BF16, false>, g, b, lds, ao, q_dim, W, D, x);
    return vec ? launch(L, wo_kernel<RBT_DT_F32, true>, g, b, lds, ao, q_dim, W, D, x)
               : launch(L, wo_kernel<RBT_DT_F32, false>, g, b, lds, ao, q_dim, W, D, x);
}

hipError_t launch_rmsnorm(const Launch &L, const float *x, const float *w, int n, float eps, float *out) {
    return launch(L, rmsnorm_kernel, dim3(1), dim3(1024), 0, x, w, n, eps, out);
}

hipError_t launch_argmax(const Launch &L, const float *v, int n, StepState *st, int32_t *seq, int ctx) {
    return launch(L, argmax_kernel, dim3(1), dim3(1024), 0, v, n, st, seq, ctx);
}

hipError_t launch_advance(const Launch &L, StepState *st) {
    return launch(L, advance_kernel, dim3(1), dim3(64), 0, st);
}

}  // namespace rbt
