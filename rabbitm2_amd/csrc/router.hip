// Router: gate logits in the engine's exact fp32 order, softmax, top-k, combine weights.
//
// Reference: rabbit2/src/rabbit2.c:513-528 (router matvec, softmax :399-405, iterative top-k with
// strict '>' so the lowest index wins ties) and :539 (norm_topk weights).
//
// Why exact order: the engine selects experts by comparing fp32 probabilities. A different
// summation order for the logits moves them by an ulp or so, which can swap two experts whose
// logits are merely close. Reproducing the engine's order makes the logits bit-identical, so the
// selection is identical unless the engine itself sees an exact tie.
//   RBT_ORDER_AVX2   (rabbit2.c:323-353): 16 independent chains; chain c sums, in column order,
//                    the rounded products of columns 16m+c (c<8: register a lane c, c>=8:
//                    register b lane c-8); then lanes a[j]+b[j], summed j=0..7 onto 0.0f; then
//                    the < 16-column tail in order.
//   RBT_ORDER_SCALAR (rabbit2.c:356-390): 4 chains over columns 4m+j, tail into chain 0, result
//                    (s0+s1)+(s2+s3).
// Each chain is one thread. A block owns `rpb` router rows of one token; their columns are staged
// through LDS a chunk at a time with 16-byte loads (every load of a chunk in flight at once), and
// the chains then run out of LDS. A token's E rows are spread over ceil(E/rpb) blocks so the 256 KiB
// router streams through many CUs. A second kernel (one block per token) does the softmax and the
// top-k; the kernel boundary is the only synchronisation (no device-scope fences or atomics, whose
// L2 write-back/invalidate costs more than a launch inside a graph).
// No multiply-add contraction anywhere in this file: every product is rounded before its add,
// exactly as the engine's `-std=c99` build does.
#pragma clang fp contract(off)

#include <math.h>

#include "rbt2_internal.h"

namespace rbt {
namespace {

constexpr int kLdsProbsMax = 4096;  // tokens with E <= this keep probabilities in LDS
constexpr int kRankMax = 1024;      // top-k by rank counting up to this many experts
constexpr int kPad = 16;            // elements of padding per staged row (spreads rows over LDS banks)

// WIDE: blocks of at most 4 rows stage 2048 columns per chunk (one round trip for the OLMoE
// width); blocks of up to 16 rows stage 1024 (bf16) / 512 (f32), keeping LDS under 40 KiB.
template <int DT, bool WIDE = false>
struct RouterTile {
    using W = typename std::conditional<DT == RBT_DT_F32, float, uint16_t>::type;
    static constexpr int kCols = WIDE ? 2048 : (DT == RBT_DT_F32 ? 512 : 1024);  // multiple of 16
    static constexpr int kPitch = kCols + kPad;
    static constexpr int kEsz = (int)sizeof(W);
};

template <int DT>
__device__ __forceinline__ float widen(typename RouterTile<DT, false>::W w) {
    if constexpr (DT == RBT_DT_F32)
        return w;
    else
        return __uint_as_float((uint32_t)w << 16);
}

__device__ float block_max_f(float v, float *red) {
    v = wave_max(v);
    const int nw = blockDim.x / kWave;
    if (nw == 1) return v;
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < nw; ++i) r = fmaxf(r, red[i]);
    return r;
}

__device__ unsigned long long block_max_u64(unsigned long long v, unsigned long long *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long u = __shfl_xor(v, o, kWave);
        v = u > v ? u : v;
    }
    const int nw = blockDim.x / kWave;
    if (nw == 1) return v;
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
    __syncthreads();
    unsigned long long r = red[0];
    for (int i = 1; i < nw; ++i) r = red[i] > r ? red[i] : r;
    return r;
}

// grid (ceil(E/rpb), T); block rpb*NCH threads (64 or 256). Dynamic LDS (host computes the size):
//   wt [rpb][kPitch] W | xt [kCols] f32 | part [blockDim] f32
template <int NCH, int DT, bool WIDE>
__global__ __launch_bounds__(256) void router_logits_kernel(const float *__restrict__ xb,
                                                            const void *__restrict__ Wv,
                                                            const float *__restrict__ bias, int E, int D, int rpb,
                                                            int vec, float *__restrict__ logits) {
    using Tile = RouterTile<DT, WIDE>;
    using W = typename Tile::W;
    extern __shared__ __align__(16) unsigned char smem[];
    W *wt = reinterpret_cast<W *>(smem);
    float *xt = reinterpret_cast<float *>(smem + (size_t)rpb * Tile::kPitch * Tile::kEsz);
    float *part = xt + Tile::kCols;

    const W *Wg = static_cast<const W *>(Wv);
    const int t = blockIdx.y;
    const int tid = threadIdx.x, nt = blockDim.x;
    const int rr = tid / NCH, c = tid - rr * NCH;
    const int r0 = blockIdx.x * rpb;
    const int nrows = E - r0 < rpb ? E - r0 : rpb;
    const float *x = xb + (size_t)t * D;
    float *prow = logits + (size_t)t * E;
    const int nfull = D / NCH;
    const int body = nfull * NCH;  // columns the chains cover; the rest is the tail

    // ---- chains over LDS-staged chunks (chunk boundaries are multiples of NCH, so each chain's
    // column order is unchanged)
    float acc = 0.0f;
    for (int c0 = 0; c0 < body; c0 += Tile::kCols) {
        const int cn = body - c0 < Tile::kCols ? body - c0 : Tile::kCols;
        if (vec) {
            // 16-byte units: rows are 16-byte aligned and cn*esz is a multiple of 16 (host-checked).
            // Addresses are clamped into range so every load of a batch is issued before any wait.
            constexpr int per = 16 / Tile::kEsz;
            constexpr int UB = 16;  // 4 rows x 2048 bf16 by 64 threads: one batch
            const int upr = cn / per, total = nrows * upr;
            for (int b0 = tid; b0 < total; b0 += nt * UB) {
                u32x4 v[UB];
#pragma unroll
                for (int i = 0; i < UB; ++i) {
                    const int u = min(b0 + i * nt, total - 1);
                    const int rl = u / upr, k = u - rl * upr;
                    v[i] = *reinterpret_cast<const u32x4 *>(Wg + (size_t)(r0 + rl) * D + c0 + k * per);
                }
#pragma unroll
                for (int i = 0; i < UB; ++i) {
                    const int u = b0 + i * nt;
                    if (u < total) {
                        const int rl = u / upr, k = u - rl * upr;
                        *reinterpret_cast<u32x4 *>(wt + rl * Tile::kPitch + k * per) = v[i];
                    }
                }
            }
            const int xu = cn / 4;
            for (int b0 = tid; b0 < xu; b0 += nt * 4) {
                f32x4 v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const f32x4 *>(x + c0 + 4 * min(b0 + i * nt, xu - 1));
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (b0 + i * nt < xu) *reinterpret_cast<f32x4 *>(xt + 4 * (b0 + i * nt)) = v[i];
            }
        } else {
            for (int i = tid; i < nrows * cn; i += nt) {
                const int rl = i / cn, cc = i - rl * cn;
                wt[rl * Tile::kPitch + cc] = Wg[(size_t)(r0 + rl) * D + c0 + cc];
            }
            for (int i = tid; i < cn; i += nt) xt[i] = x[c0 + i];
        }
        __syncthreads();
        if (rr < nrows) {
            const W *wr = wt + rr * Tile::kPitch;
            const int steps = cn / NCH;
#pragma unroll 8
            for (int m = 0; m < steps; ++m) {
                const int cc = m * NCH + c;
                acc = acc + widen<DT>(wr[cc]) * xt[cc];
            }
        }
        __syncthreads();
    }
    part[tid] = acc;
    __syncthreads();
    if (c == 0 && rr < nrows) {
        const int r = r0 + rr;
        const W *wrow = Wg + (size_t)r * D;
        float res;
        if constexpr (NCH == 16) {
            float sum = 0.0f;
            for (int j = 0; j < 8; ++j) sum = sum + (part[tid + j] + part[tid + 8 + j]);
            for (int i = body; i < D; ++i) sum = sum + widen<DT>(wrow[i]) * x[i];
            res = sum;
        } else {
            float s0 = part[tid], s1 = part[tid + 1], s2 = part[tid + 2], s3 = part[tid + 3];
            for (int i = body; i < D; ++i) s0 = s0 + widen<DT>(wrow[i]) * x[i];
            res = (s0 + s1) + (s2 + s3);
        }
        if (bias) res = res + bias[r];
        prow[r] = res;
    }

}

// Few tokens (decode), AVX2 order, bf16 weights, D a multiple of 128: one 64-thread block per DR router
// rows of one token, thread (row rr, chain c). DR = 2 while the blocks fit the CUs once (each block
// stages x plus fewer weight bytes before its chains start; one OLMoE MoE layer 24.4 against 24.7 us
// with 4 rows), lanes 32-63 then staging only; DR = 4 for more tokens (at 32 tokens 5.5 against
// 7.2 us: every block stages its token's x). Chain c's operands are staged transposed in LDS, both as
// f32 -- wt[rr][c][m] = W[r][16m + c], xt[c][m] = x[16m + c] -- so two 16-byte reads of each carry 4
// steps of one chain, and a step is one rounded multiply and one add (the bf16 weights are widened
// once, while staging, not in the chain): the chain's dependent adds are the only long pole.
// Staging: a thread takes 8 consecutive steps of 8 chains (eight 16-byte loads of the row), widens
// and transposes them in registers into sixteen 16-byte LDS stores. The 16 chains of a row sit in
// 16 consecutive lanes: (chain j) + (chain 8+j) via a
// DPP row rotation, then the sequential sum over j, as the engine's lanes a[j] + b[j].
// NORM: the kernel also runs the RMSNorm in front of the router (rabbit2.c:512): x is the residual
// stream, xb = x * inv * nw with inv = 1/sqrtf(sum x^2 / D + eps) from the block's own staging loads,
// and block (0, t) writes token t's xb to xb_out for the expert kernels.
template <int M, bool NORM = false, int DR = 4>  // steps per chain = D / 16, a multiple of 8
__global__ __launch_bounds__(64) void router_decode_kernel(const float *__restrict__ xb, const uint16_t *__restrict__ W,
                                                          const float *__restrict__ bias, int E,
                                                          float *__restrict__ logits, const float *__restrict__ nw = nullptr,
                                                          float eps = 0.0f, float *__restrict__ xb_out = nullptr) {
    constexpr int D = 16 * M;
    constexpr int WP = M + 4;  // f32 per (row, chain) line: 16-byte pad, lanes of one read hit distinct banks
    constexpr int XP = M + 4;  // f32 per chain line
    constexpr int G = M / 8;   // 8-step groups per chain
    constexpr int kDRows = DR;
    static_assert(DR == 2 || DR == 4, "rows per block");
    __shared__ __align__(16) float wt[kDRows * 16 * WP];  // the weights widened to f32 (exact)
    __shared__ __align__(16) float xt[16 * XP];
    const int tid = threadIdx.x, rr = tid >> 4, c = tid & 15;
    const int t = blockIdx.y, r0 = blockIdx.x * kDRows;
    const float *x = xb + (size_t)t * D;

    // ---- staging tasks: (row, half h, group g) for W, (half h, group g) for x; all loads first
    constexpr int WT = kDRows * 2 * G, XT = 2 * G;
    constexpr int WPER = (WT + 63) / 64, XPER = (XT + 63) / 64;
    u32x4 wv[WPER][8];
    f32x4 xv[XPER][8][2], nv[NORM ? XPER : 1][8][2];
    auto load_w = [&]() {
#pragma unroll
        for (int q = 0; q < WPER; ++q) {
            const int task = min(tid + 64 * q, WT - 1);
            const int row = task / (2 * G), h = (task / G) & 1, g = task % G;
            const int r = min(r0 + row, E - 1);
            const uint16_t *src = W + (size_t)r * D + 8 * h;
#pragma unroll
            for (int i = 0; i < 8; ++i) wv[q][i] = *reinterpret_cast<const u32x4 *>(src + 16 * (8 * g + i));
        }
    };
    // With NORM, x and the norm weights go before W: loads return in issue order, so the norm below
    // waits for these only, while the router rows are still in flight. Without it W goes first.
    if constexpr (!NORM) load_w();
#pragma unroll
    for (int q = 0; q < XPER; ++q) {
        const int task = min(tid + 64 * q, XT - 1);
        const int h = task / G, g = task % G;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int off = 16 * (8 * g + i) + 8 * h;
            xv[q][i][0] = *reinterpret_cast<const f32x4 *>(x + off);
            xv[q][i][1] = *reinterpret_cast<const f32x4 *>(x + off + 4);
            if constexpr (NORM) {
                nv[q][i][0] = *reinterpret_cast<const f32x4 *>(nw + off);
                nv[q][i][1] = *reinterpret_cast<const f32x4 *>(nw + off + 4);
            }
        }
    }
    if constexpr (NORM) {
        __builtin_amdgcn_sched_barrier(0);
        load_w();
    }
    if constexpr (NORM) {
        // sum of squares over the token's x (every element once: tasks past XT repeat the last one)
        float ss = 0.0f;
#pragma unroll
        for (int q = 0; q < XPER; ++q) {
            if (tid + 64 * q < XT) {
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        ss += xv[q][i][j].x * xv[q][i][j].x + xv[q][i][j].y * xv[q][i][j].y +
                              xv[q][i][j].z * xv[q][i][j].z + xv[q][i][j].w * xv[q][i][j].w;
            }
        }
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
        for (int q = 0; q < XPER; ++q) {
            const int task = min(tid + 64 * q, XT - 1);
            const int h = task / G, g = task % G;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int off = 16 * (8 * g + i) + 8 * h;
                const f32x4 w0 = nv[q][i][0], w1 = nv[q][i][1];
                f32x4 &a = xv[q][i][0], &b = xv[q][i][1];
                a = f32x4{a.x * inv * w0.x, a.y * inv * w0.y, a.z * inv * w0.z, a.w * inv * w0.w};
                b = f32x4{b.x * inv * w1.x, b.y * inv * w1.y, b.z * inv * w1.z, b.w * inv * w1.w};
                if (blockIdx.x == 0 && tid + 64 * q < XT) {
                    float *dst = xb_out + (size_t)t * D + off;
                    *reinterpret_cast<f32x4 *>(dst) = a;
                    *reinterpret_cast<f32x4 *>(dst + 4) = b;
                }
            }
        }
    }
    // transposed stores (clamped tasks rewrite the last task's identical data)
#pragma unroll
    for (int q = 0; q < WPER; ++q) {
        const int task = min(tid + 64 * q, WT - 1);
        const int row = task / (2 * G), h = (task / G) & 1, g = task % G;
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) {
            // chain 8h+ch, steps 8g..8g+7: bf16 #ch of units i = 0..7, widened here once by all lanes
            // instead of in every step of the chain (ch odd: the high halves)
            uint32_t d[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t u = wv[q][i][ch >> 1];
                d[i] = (ch & 1) ? (u & 0xFFFF0000u) : (u << 16);
            }
            float *dst = &wt[(row * 16 + 8 * h + ch) * WP + 8 * g];
            *reinterpret_cast<u32x4 *>(dst) = u32x4{d[0], d[1], d[2], d[3]};
            *reinterpret_cast<u32x4 *>(dst + 4) = u32x4{d[4], d[5], d[6], d[7]};
        }
    }
#pragma unroll
    for (int q = 0; q < XPER; ++q) {
        const int task = min(tid + 64 * q, XT - 1);
        const int h = task / G, g = task % G;
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) {
            f32x4 lo, hi;
            lo.x = xv[q][0][ch >> 2][ch & 3]; lo.y = xv[q][1][ch >> 2][ch & 3];
            lo.z = xv[q][2][ch >> 2][ch & 3]; lo.w = xv[q][3][ch >> 2][ch & 3];
            hi.x = xv[q][4][ch >> 2][ch & 3]; hi.y = xv[q][5][ch >> 2][ch & 3];
            hi.z = xv[q][6][ch >> 2][ch & 3]; hi.w = xv[q][7][ch >> 2][ch & 3];
            float *dst = &xt[(8 * h + ch) * XP + 8 * g];
            *reinterpret_cast<f32x4 *>(dst) = lo;
            *reinterpret_cast<f32x4 *>(dst + 4) = hi;
        }
    }
    __syncthreads();

    // ---- chain c of row rr, 128 steps in column order (rounded product, then add)
    const float *wl = &wt[(min(rr, kDRows - 1) * 16 + c) * WP];  // lanes past the rows: clamped, no write
    const float *xl = &xt[c * XP];
    float acc = 0.0f;
#pragma unroll 4
    for (int g = 0; g < G; ++g) {
        const f32x4 wa = *reinterpret_cast<const f32x4 *>(wl + 8 * g);
        const f32x4 wc = *reinterpret_cast<const f32x4 *>(wl + 8 * g + 4);
        const f32x4 xa = *reinterpret_cast<const f32x4 *>(xl + 8 * g);
        const f32x4 xc = *reinterpret_cast<const f32x4 *>(xl + 8 * g + 4);
        acc = acc + wa.x * xa.x;
        acc = acc + wa.y * xa.y;
        acc = acc + wa.z * xa.z;
        acc = acc + wa.w * xa.w;
        acc = acc + wc.x * xc.x;
        acc = acc + wc.y * xc.y;
        acc = acc + wc.z * xc.z;
        acc = acc + wc.w * xc.w;
    }
    // lanes c and c+8 of the row: row_ror:8 brings chain c+8 to lane c
    const float other = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x128, 0xF, 0xF, false));
    const float pair = acc + other;  // lanes c < 8: a[c] + b[c]
    float rs[kDRows];  // each row's sum over j, in order, from wave-uniform lanes
#pragma unroll
    for (int R = 0; R < kDRows; ++R) {
        rs[R] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) rs[R] = rs[R] + lane_value(pair, 16 * R + j);
    }
    float sum = rs[0];
#pragma unroll
    for (int R = 1; R < kDRows; ++R) sum = rr == R ? rs[R] : sum;
    const int r = r0 + rr;
    if (c == 0 && rr < kDRows && r < E) {
        if (bias) sum = sum + bias[r];
        logits[(size_t)t * E + r] = sum;
    }
}

// Softmax + top-k of one token's E <= 64 logits by one wave (lane = expert), the engine's arithmetic
// (rabbit2.c:399-405 softmax with max-subtract, exp, sequential sum, divide; :516-528 K rounds of
// "largest unused, lowest index on ties" = the first K places of a stable descending sort; :539
// norm_topk). s_v: this wave's 64-float LDS scratch. NaN: as the engine's '>' scans (a NaN logit
// never wins a comparison, except that element 0 starts the max scan).
__device__ __forceinline__ void wave_softmax_topk(float v, int E, int K, int norm_topk, float *s_v, float *s_p,
                                                  int32_t *routing_t, float *weights_t) {
    const int lane = threadIdx.x & (kWave - 1);
    if (lane >= E) v = -INFINITY;
    float mx = wave_max(v);
    const float first = lane_value(v, 0);
    if (first != first) mx = first;
    const float e = lane < E ? (float)exp((double)(v - mx)) : 0.0f;
    s_v[lane] = e;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const f32x4 *p4 = reinterpret_cast<const f32x4 *>(s_v);
    float sum = 0.0f;  // every lane, sequentially in the engine's order (entries past E are 0, last)
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const f32x4 v4 = p4[q];
        sum = sum + v4.x;
        sum = sum + v4.y;
        sum = sum + v4.z;
        sum = sum + v4.w;
    }
    const float p = e / sum;
    if (sum != sum) {
        if (lane < K) {  // all NaN: each round keeps the first unused index
            routing_t[lane] = lane;
            s_p[lane] = p;
        }
    } else {
        // K rounds of the selection: the largest remaining probability, the lowest index among equal
        // ones; a wave maximum and a ballot per round. Probabilities are finite and >= 0 here, so
        // lanes past E (-1) never win and a taken lane (-2) is out for good.
        float cand = lane < E ? p : -1.0f;
        for (int k = 0; k < K; ++k) {
            const float m = wave_max(cand);
            const int w = __builtin_ctzll(__ballot(cand == m));
            if (lane == w) {
                routing_t[k] = lane;
                s_p[k] = p;
                cand = -2.0f;
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float wsum = 0.0f;
    for (int k = 0; k < K; ++k) wsum = wsum + s_p[k];
    if (lane < K) weights_t[lane] = norm_topk ? s_p[lane] / wsum : s_p[lane];
}

// Softmax + top-k of token t's E <= 64 logits (wave 0 of block t, the engine's arithmetic as above) and
// the bf16 hi/lo split of its activation row (every thread, 8 elements per 16-byte pair): the grouped
// expert path's front end for a few tokens whose logits and normalised rows router_decode_kernel<M,
// true> has just written (E / 2 or E / 4 x T blocks for the chains instead of the fused prefill kernel's one
// block per two tokens).
__global__ __launch_bounds__(256) void topk_split_kernel(const float *__restrict__ logits, int E, int K, int norm_topk,
                                                         const float *__restrict__ xb, int D,
                                                         int32_t *__restrict__ routing, float *__restrict__ weights,
                                                         uint16_t *__restrict__ x_hi, uint16_t *__restrict__ x_lo) {
    __shared__ __align__(16) float s_v[64];
    __shared__ float s_p[64];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float v = tid < E ? logits[(size_t)t * E + tid] : 0.0f;
    const size_t row = (size_t)t * D;
    for (int u = tid; u < D / 8; u += blockDim.x) {
        const f32x4 a = ld_f4(xb + row + 8 * u), b = ld_f4(xb + row + 8 * u + 4);
        const float x8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t hb[8], lb[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            hb[k] = f32_to_bf16_rne(x8[k]);
            lb[k] = f32_to_bf16_rne(x8[k] - __uint_as_float(hb[k] << 16));
        }
        *reinterpret_cast<u32x4 *>(x_hi + row + 8 * u) =
            u32x4{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16), hb[4] | (hb[5] << 16), hb[6] | (hb[7] << 16)};
        *reinterpret_cast<u32x4 *>(x_lo + row + 8 * u) =
            u32x4{lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16), lb[4] | (lb[5] << 16), lb[6] | (lb[7] << 16)};
    }
    if (tid < kWave) wave_softmax_topk(v, E, K, norm_topk, s_v, s_p, routing + (size_t)t * K, weights + (size_t)t * K);
}

// Prefill front end in one launch (AVX2 order, E <= 64, bf16): router logits, softmax + top-k, and the
// bf16 hi/lo split of x for the grouped GEMMs. One block per kPTok tokens covers all router rows, so the
// top-k runs in the block. Wave (token tl, quarter q) holds the 64 router rows in its lanes and runs
// chains 4q..4q+3 of each: eight waves per block, two per SIMD, since a SIMD issues two waves' VALU
// operations in the time one wave issues one. Router columns stream through LDS in double-buffered
// chunks of kPCols (coalesced global reads; each lane then reads its row's 8-byte slice per step). x is
// the same for the whole wave: it is read with scalar loads, kPGroup steps at a time and one group
// ahead, and enters the multiplies as a scalar operand, so no lane-by-lane copy of it returns from
// memory. What bounds it at 512 tokens is the staging: every block pulls the whole 256 KiB router from
// L2, and a CU's outstanding misses at L2 latency give it ~26 GB/s (about 10 of the kernel's 16 us);
// the VALU work (a widen, a rounded multiply and a rounded add per weight) runs under that.
constexpr int kPTok = 2, kPCols = 512, kPGroup = 8, kPThreads = kPTok * 64 * 4;
template <int DT>
__global__ __launch_bounds__(kPThreads) void router_prefill_kernel(const float *__restrict__ xb,
                                                                   const void *__restrict__ Wv,
                                                                   const float *__restrict__ bias, int T, int E, int D,
                                                                   int K, int norm_topk, int32_t *__restrict__ routing,
                                                                   float *__restrict__ weights,
                                                                   uint16_t *__restrict__ x_hi,
                                                                   uint16_t *__restrict__ x_lo) {
    static_assert(DT == RBT_DT_BF16, "bf16 router rows");
    constexpr int CW = kPCols;                // columns per chunk (1 KiB per row)
    constexpr int WP = CW * 2 + 16;           // row pitch in bytes
    constexpr int UPR = CW * 2 / 16;          // 16-byte units per row per chunk
    constexpr int WU = 64 * UPR / kPThreads;  // per thread per chunk
    constexpr int G = kPGroup;
    constexpr int SU = 2;                     // split: 16-byte loads in flight per thread
    __shared__ __align__(16) unsigned char wt[2][64 * WP];
    __shared__ __align__(16) float s_part[kPTok][16][64];  // the 16 chains of each (token, row)
    __shared__ __align__(16) float s_log[kPTok][64];
    __shared__ __align__(16) float s_v[kPTok][64];
    __shared__ float s_p[kPTok][64];
    const uint16_t *Wg = static_cast<const uint16_t *>(Wv);
    const int tid = threadIdx.x, r = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int q = wv & 3, tl = wv >> 2;
    const int t0 = blockIdx.x * kPTok;
    const int ntok = min(kPTok, T - t0);
    const int body = (D / 16) * 16;
    const int nch = (body + CW - 1) / CW;
    const bool live = tl < ntok;  // wave-uniform
    const float *xrow = xb + (size_t)(t0 + (live ? tl : 0)) * D + 4 * q;  // wave-uniform: scalar loads
    const float bias_r = bias ? bias[min(r, E - 1)] : 0.0f;  // read now, used at the end

    u32x4 wv4[WU];
    auto load = [&](int c) {
        const int c0 = c * CW, upr = min(CW, body - c0) / 8;
#pragma unroll
        for (int i = 0; i < WU; ++i) {
            const int u = tid + i * kPThreads, row = u / UPR, k = min(u % UPR, upr - 1);
            wv4[i] = *reinterpret_cast<const u32x4 *>(Wg + (size_t)min(row, E - 1) * D + c0 + 8 * k);
        }
    };
    auto store = [&](int c) {
        const int upr = min(CW, body - c * CW) / 8;
#pragma unroll
        for (int i = 0; i < WU; ++i) {
            const int u = tid + i * kPThreads, row = u / UPR, k = min(u % UPR, upr - 1);
            *reinterpret_cast<u32x4 *>(wt[c & 1] + row * WP + k * 16) = wv4[i];
        }
    };
    if (nch > 0) load(0);  // in flight during the split

    // the hi/lo split of this block's x rows (contiguous): SU 16-byte loads in flight per thread; a
    // unit past the rows is clamped to the last one, which is then written twice with the same bytes
    if (x_hi) {
        const int units = ntok * D / 4;
        const size_t base = (size_t)t0 * D;
        for (int u0 = tid; u0 < units; u0 += SU * kPThreads) {
            f32x4 v[SU];
#pragma unroll
            for (int i = 0; i < SU; ++i) v[i] = ld_f4(xb + base + 4 * (size_t)min(u0 + i * kPThreads, units - 1));
#pragma unroll
            for (int i = 0; i < SU; ++i) {
                const size_t o = base + 4 * (size_t)min(u0 + i * kPThreads, units - 1);
                uint32_t hb[4], lb[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    hb[j] = f32_to_bf16_rne(v[i][j]);
                    lb[j] = f32_to_bf16_rne(v[i][j] - __uint_as_float(hb[j] << 16));
                }
                *reinterpret_cast<uint2 *>(x_hi + o) = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
                *reinterpret_cast<uint2 *>(x_lo + o) = make_uint2(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16));
            }
        }
    }

    float acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = 0.0f;
    auto step = [&](const uint2 a, const float *xs) {
        acc[0] = acc[0] + bf16_lo(a.x) * xs[0];
        acc[1] = acc[1] + bf16_hi(a.x) * xs[1];
        acc[2] = acc[2] + bf16_lo(a.y) * xs[2];
        acc[3] = acc[3] + bf16_hi(a.y) * xs[3];
    };
    if (nch > 0) store(0);
    __syncthreads();
    for (int c = 0; c < nch; ++c) {
        const bool more = c + 1 < nch;
        if (more) load(c + 1);  // in flight during this chunk's chains
        const int c0 = c * CW, steps = min(CW, body - c0) / 16, full = steps / (2 * G) * (2 * G);
        if (live) {  // every lane (rows past E repeat row E - 1 and are not used): uniform control flow
            const unsigned char *wr = wt[c & 1] + r * WP + 8 * q;
            const float *xc = xrow + c0;
            // groups of G steps in two register sets: while one set's group multiplies, the other set
            // takes the next group's router slices (LDS) and x (scalar loads at constant offsets from
            // one base, so few address registers). The fetch after the last group is clamped into the
            // chunk and its values are not used. A scalar-load wait cannot skip the newest loads (they
            // return out of order), so each fetch is issued only once the set about to multiply has
            // arrived: its offset takes a register-only dependence on that set's first value (an empty
            // asm), which places the wait before it; scheduling barriers keep each fetch ahead of the
            // other set's multiplies.
            uint2 wa[G], wb[G];
            float xa[G * 4], xb4[G * 4];
            auto fetch = [&](uint2 (&w)[G], float (&x)[G * 4], int g, float after) {
                g = min(g, steps - G);
                int xo = 16 * g;
                asm volatile("" : "+s"(xo) : "s"(after));
                const unsigned char *wp = wr + 32 * g;
                const float *xp = xc + xo;
#pragma unroll
                for (int i = 0; i < G; ++i) w[i] = *reinterpret_cast<const uint2 *>(wp + 32 * i);
#pragma unroll
                for (int k = 0; k < G * 4; ++k) x[k] = xp[16 * (k / 4) + k % 4];
            };
            // all of a group's products first, then its adds in step order: dependent operations sit
            // far apart, so neither wave of a SIMD waits on a result
            auto run = [&](const uint2 (&w)[G], const float (&x)[G * 4]) {
                float pr[G][4];
#pragma unroll
                for (int i = 0; i < G; ++i) {
                    pr[i][0] = bf16_lo(w[i].x) * x[4 * i];
                    pr[i][1] = bf16_hi(w[i].x) * x[4 * i + 1];
                    pr[i][2] = bf16_lo(w[i].y) * x[4 * i + 2];
                    pr[i][3] = bf16_hi(w[i].y) * x[4 * i + 3];
                }
#pragma unroll
                for (int i = 0; i < G; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[j] = acc[j] + pr[i][j];
            };
            if (full > 0) fetch(wa, xa, 0, 0.0f);
            for (int g = 0; g < full; g += 2 * G) {
                fetch(wb, xb4, g + G, xa[0]);
                __builtin_amdgcn_sched_barrier(0);
                run(wa, xa);
                __builtin_amdgcn_sched_barrier(0);
                fetch(wa, xa, g + 2 * G, xb4[0]);
                __builtin_amdgcn_sched_barrier(0);
                run(wb, xb4);
                __builtin_amdgcn_sched_barrier(0);
            }
            for (int m = full; m < steps; ++m) step(*reinterpret_cast<const uint2 *>(wr + 32 * m), xc + 16 * m);
        }
        if (more) store(c + 1);  // the other buffer: last read in chunk c-1, before the barrier below
        __syncthreads();
    }
    if (live) {
#pragma unroll
        for (int j = 0; j < 4; ++j) s_part[tl][4 * q + j][r] = acc[j];
    }
    __syncthreads();
    if (q == 0 && live && r < E) {
        float sum = 0.0f;  // the engine's lanes a[j] + b[j] (chains j and 8 + j), summed from j = 0
#pragma unroll
        for (int j = 0; j < 8; ++j) sum = sum + (s_part[tl][j][r] + s_part[tl][8 + j][r]);
        const uint16_t *wrow = Wg + (size_t)r * D;
        const float *x = xb + (size_t)(t0 + tl) * D;
        for (int i = body; i < D; ++i) sum = sum + widen<DT>(wrow[i]) * x[i];
        if (bias) sum = sum + bias_r;
        s_log[tl][r] = sum;
    }
    __syncthreads();
    if (wv < ntok) {
        const int lane = tid & 63;
        wave_softmax_topk(lane < E ? s_log[wv][lane] : 0.0f, E, K, norm_topk, s_v[wv], s_p[wv],
                          routing + (size_t)(t0 + wv) * K, weights + (size_t)(t0 + wv) * K);
    }
}

// Many tokens, AVX2 order: the router tile is shared by a block's tokens instead of re-read per token.
// grid (ceil(E/16), ceil(T/8)), 256 threads: tid -> half h = tid & 1, router row 16*bx + ((tid >> 1) & 15),
// token 8*by + (tid >> 5). Thread (t, r, h) runs chains 8h..8h+7 of row r for token t: step m adds the
// rounded products of columns 16m + 8h + j (j = 0..7), i.e. chain 8h+j, in column order -- a 16-byte
// read of the row and two of x per step, 8 independent chains. The pair (h = 0, 1) sits in adjacent
// lanes; the h = 0 lane combines (chain j) + (chain 8+j) for j = 0..7 onto 0.0f, then the tail.
// LDS per column chunk of kBCols: router rows [16][kBCols] in DT and x [8][kBCols] f32.
constexpr int kBRows = 16, kBTok = 8, kBCols = 512;
template <int DT>
__global__ __launch_bounds__(256) void router_logits_batch_kernel(const float *__restrict__ xb,
                                                                  const void *__restrict__ Wv,
                                                                  const float *__restrict__ bias, int T, int E, int D,
                                                                  float *__restrict__ logits) {
    using W = typename RouterTile<DT, false>::W;
    constexpr int ESZ = (int)sizeof(W);
    constexpr int WP = kBCols * ESZ + 32;  // row pitch in bytes (32-byte pad)
    constexpr int XP = kBCols * 4 + 16;
    __shared__ __align__(16) unsigned char wt[kBRows * WP];
    __shared__ __align__(16) unsigned char xt[kBTok * XP];
    const W *Wg = static_cast<const W *>(Wv);
    const int tid = threadIdx.x, h = tid & 1, rl = (tid >> 1) & 15, tl = tid >> 5;
    const int r0 = blockIdx.x * kBRows, t0 = blockIdx.y * kBTok;
    const int r = r0 + rl, t = t0 + tl;
    const int nrows = min(kBRows, E - r0), ntok = min(kBTok, T - t0);
    const int body = (D / 16) * 16;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    for (int c0 = 0; c0 < body; c0 += kBCols) {
        const int cn = min(kBCols, body - c0);  // a multiple of 16
        // stage: 16-byte units, every load of a batch issued before the stores (clamped addresses)
        {
            constexpr int per = 16 / ESZ;
            const int wu = cn / per, wtot = nrows * wu;
            const int xu = cn / 4, xtot = ntok * xu;
            for (int b0 = tid; b0 < wtot + xtot; b0 += 256 * 8) {
                u32x4 v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int u = min(b0 + i * 256, wtot + xtot - 1);
                    if (u < wtot) {
                        const int rr = u / wu, k = u - rr * wu;
                        v[i] = *reinterpret_cast<const u32x4 *>(Wg + (size_t)(r0 + rr) * D + c0 + k * per);
                    } else {
                        const int q = u - wtot, tt = q / xu, k = q - tt * xu;
                        v[i] = *reinterpret_cast<const u32x4 *>(xb + (size_t)(t0 + tt) * D + c0 + 4 * k);
                    }
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int u = b0 + i * 256;
                    if (u < wtot) {
                        const int rr = u / wu, k = u - rr * wu;
                        *reinterpret_cast<u32x4 *>(wt + rr * WP + k * 16) = v[i];
                    } else if (u < wtot + xtot) {
                        const int q = u - wtot, tt = q / xu, k = q - tt * xu;
                        *reinterpret_cast<u32x4 *>(xt + tt * XP + k * 16) = v[i];
                    }
                }
            }
        }
        __syncthreads();
        if (rl < nrows && tl < ntok) {
            const unsigned char *wr = wt + rl * WP + h * 8 * ESZ;
            const float *xr = reinterpret_cast<const float *>(xt + tl * XP) + 8 * h;
            const int steps = cn / 16;
#pragma unroll 2
            for (int m = 0; m < steps; ++m) {
                float wv[8];
                if constexpr (DT == RBT_DT_F32) {
                    const f32x4 a = *reinterpret_cast<const f32x4 *>(wr + m * 64);
                    const f32x4 b = *reinterpret_cast<const f32x4 *>(wr + m * 64 + 16);
                    wv[0] = a.x; wv[1] = a.y; wv[2] = a.z; wv[3] = a.w;
                    wv[4] = b.x; wv[5] = b.y; wv[6] = b.z; wv[7] = b.w;
                } else {
                    const u32x4 a = *reinterpret_cast<const u32x4 *>(wr + m * 32);
                    wv[0] = bf16_lo(a.x); wv[1] = bf16_hi(a.x); wv[2] = bf16_lo(a.y); wv[3] = bf16_hi(a.y);
                    wv[4] = bf16_lo(a.z); wv[5] = bf16_hi(a.z); wv[6] = bf16_lo(a.w); wv[7] = bf16_hi(a.w);
                }
                const f32x4 xa = *reinterpret_cast<const f32x4 *>(xr + 16 * m);
                const f32x4 xc = *reinterpret_cast<const f32x4 *>(xr + 16 * m + 4);
                acc[0] = acc[0] + wv[0] * xa.x;
                acc[1] = acc[1] + wv[1] * xa.y;
                acc[2] = acc[2] + wv[2] * xa.z;
                acc[3] = acc[3] + wv[3] * xa.w;
                acc[4] = acc[4] + wv[4] * xc.x;
                acc[5] = acc[5] + wv[5] * xc.y;
                acc[6] = acc[6] + wv[6] * xc.z;
                acc[7] = acc[7] + wv[7] * xc.w;
            }
        }
        __syncthreads();
    }
    // chains 8..15 from the partner lane (h = 1), fetched by every lane (the DPP move is wave-wide)
    float other[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) other[j] = dpp_f<kDppXor1>(acc[j]);
    if (h == 0 && rl < nrows && tl < ntok) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) sum = sum + (acc[j] + other[j]);
        const W *wrow = Wg + (size_t)r * D;
        const float *x = xb + (size_t)t * D;
        for (int i = body; i < D; ++i) sum = sum + widen<DT>(wrow[i]) * x[i];
        if (bias) sum = sum + bias[r];
        logits[(size_t)t * E + r] = sum;
    }
}

// grid (T), block 64 or 256 threads; dynamic LDS E floats when E <= kLdsProbsMax. Reads the logits
// row of its token, leaves the probabilities in it, writes routing/weights.
__global__ __launch_bounds__(256) void router_topk_kernel(int E, int K, int norm_topk, float *__restrict__ probs,
                                                          int32_t *__restrict__ routing,
                                                          float *__restrict__ weights) {
    extern __shared__ __align__(16) float pb_lds[];
    __shared__ float red_f[4];
    __shared__ unsigned long long red_u[4];
    __shared__ int32_t s_idx[64];
    __shared__ float s_wt[64];
    __shared__ float s_sum;
    const int t = blockIdx.x;
    const int tid = threadIdx.x, nt = blockDim.x;
    float *prow = probs + (size_t)t * E;
    const bool lds = E <= kLdsProbsMax;
    float *pb = lds ? pb_lds : prow;
    float mx = -INFINITY;
    for (int i = tid; i < E; i += nt) {
        const float v = prow[i];
        if (lds) pb[i] = v;
        mx = fmaxf(mx, v);  // ignores NaN, as the engine's '>' scan does ...
    }
    mx = block_max_f(mx, red_f);
    __syncthreads();
    const float first = pb[0];
    if (first != first) mx = first;  // ... except that a NaN in element 0 is its starting maximum
    for (int i = tid; i < E; i += nt) {
        // expf rounded from a double evaluation: within 0.5 ulp + 2^-29, as glibc's expf (0.502 ulp)
        pb[i] = (float)exp((double)(pb[i] - mx));
    }
    if (!lds) __threadfence();
    __syncthreads();
    if (tid == 0) {
        // the engine's sequential order; 16-byte LDS reads keep several values in flight
        float sum = 0.0f;
        int i = 0;
        if (lds) {
            const f32x4 *p4 = reinterpret_cast<const f32x4 *>(pb);
#pragma unroll 4
            for (; i + 4 <= E; i += 4) {
                const f32x4 v = p4[i / 4];
                sum = sum + v.x;
                sum = sum + v.y;
                sum = sum + v.z;
                sum = sum + v.w;
            }
        }
        for (; i < E; ++i) sum = sum + pb[i];
        s_sum = sum;
    }
    __syncthreads();
    const float sum = s_sum;
    for (int i = tid; i < E; i += nt) pb[i] = pb[i] / sum;
    if (!lds) __threadfence();
    __syncthreads();

    if (sum != sum) {
        // every probability is NaN: the engine's scan keeps the first unused index each round
        if (tid < K) {
            s_idx[tid] = tid;
            s_wt[tid] = pb[tid];
        }
    } else if (lds && E <= kRankMax) {
        // The engine's K rounds of "largest unused, lowest index on ties" are the first K places of a
        // stable descending sort: an element's place is the number of elements that beat it.
        for (int i = tid; i < E; i += nt) {
            const float pi = pb[i];
            int rank = 0;
            for (int j = 0; j < E; ++j) {
                const float pj = pb[j];
                rank += (pj > pi) | ((pj == pi) & (j < i));
            }
            if (rank < K) {
                s_idx[rank] = i;
                s_wt[rank] = pi;
            }
        }
    } else {
        // probabilities are >= +0, so their bit patterns order like the values; the low word makes
        // every key unique and prefers the lower index on equal probability. Round j takes the
        // largest key below round j-1's.
        unsigned long long prev = ~0ull;
        for (int j = 0; j < K; ++j) {
            unsigned long long best = 0;
            for (int i = tid; i < E; i += nt) {
                const unsigned long long key =
                    ((unsigned long long)__float_as_uint(pb[i]) << 32) | (0xFFFFFFFFu - (unsigned)i);
                if (key < prev && key > best) best = key;
            }
            best = block_max_u64(best, red_u);
            prev = best;
            if (tid == 0) {
                const int id = (int)(0xFFFFFFFFu - (unsigned)(best & 0xFFFFFFFFull));
                s_idx[j] = id;
                s_wt[j] = pb[id];
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        float wsum = 0.0f;
        for (int j = 0; j < K; ++j) wsum = wsum + s_wt[j];
        for (int j = 0; j < K; ++j) {
            routing[(size_t)t * K + j] = s_idx[j];
            weights[(size_t)t * K + j] = norm_topk ? s_wt[j] / wsum : s_wt[j];
        }
    }
    if (lds)
        for (int i = tid; i < E; i += nt) prow[i] = pb[i];
}

template <int NCH, int DT, bool WIDE>
hipError_t launch_logits(const Launch &L, const float *xb, const void *W, const float *bias, int T, int E, int D,
                         int threads, float *probs) {
    using Tile = RouterTile<DT, WIDE>;
    const int rpb = threads / NCH;
    const bool vec = (reinterpret_cast<uintptr_t>(W) % 16 == 0) && ((size_t)D * Tile::kEsz) % 16 == 0 &&
                     (reinterpret_cast<uintptr_t>(xb) % 16 == 0) && D % 16 == 0;
    const size_t lds = (size_t)rpb * Tile::kPitch * Tile::kEsz + Tile::kCols * 4 + threads * 4;
    return launch(L, router_logits_kernel<NCH, DT, WIDE>, dim3((E + rpb - 1) / rpb, T), dim3(threads),
                  (uint32_t)lds, xb, W, bias, E, D, rpb, vec ? 1 : 0, probs);
}

// The decode kernel (AVX2 order, bf16) below 16 tokens, for the row lengths instantiated below.
inline bool decode_ok(int T, int D, int dtype, const void *W, const float *xb) {
    const int m = D / 16;
    const bool m_ok = D % 16 == 0 && (m == 8 || m == 16 || m == 32 || m == 48 || m == 64 || m == 96 || m == 128 ||
                                      m == 192 || m == 256);
    return T <= kRouterDecodeMaxT && dtype == RBT_DT_BF16 && m_ok && (reinterpret_cast<uintptr_t>(W) % 16 == 0) &&
           (reinterpret_cast<uintptr_t>(xb) % 16 == 0);
}

constexpr int kRouterTwoRowBlocks = 256;  // blocks up to which the decode router takes 2 rows per block
template <bool NORM>
inline hipError_t launch_router_decode_t(const Launch &L, const float *xb, const void *W, const float *bias, int T,
                                         int E, int D, float *logits, const float *nw, float eps, float *xb_out) {
    const bool two = (long long)((E + 1) / 2) * T <= kRouterTwoRowBlocks;  // rows per block, see the kernel
    const dim3 g((unsigned)(two ? (E + 1) / 2 : (E + 3) / 4), (unsigned)T), b(64);
    const uint16_t *w = static_cast<const uint16_t *>(W);
    switch (D / 16) {
#define RD_CASE(m)                                                                                                \
    case m:                                                                                                       \
        return two ? launch(L, router_decode_kernel<m, NORM, 2>, g, b, 0, xb, w, bias, E, logits, nw, eps, xb_out) \
                   : launch(L, router_decode_kernel<m, NORM, 4>, g, b, 0, xb, w, bias, E, logits, nw, eps, xb_out);
        RD_CASE(8)
        RD_CASE(16)
        RD_CASE(32)
        RD_CASE(48)
        RD_CASE(64)
        RD_CASE(96)
        RD_CASE(128)
        RD_CASE(192)
        RD_CASE(256)
#undef RD_CASE
        default:
            return hipErrorNotSupported;
    }
}

inline hipError_t launch_router_decode(const Launch &L, const float *xb, const void *W, const float *bias, int T, int E,
                                       int D, float *logits) {
    return launch_router_decode_t<false>(L, xb, W, bias, T, E, D, logits, nullptr, 0.0f, nullptr);
}

// The batch kernel (AVX2 order) from 16 tokens on; its 16-byte staging needs 16-byte aligned rows.
inline bool batch_ok(int T, int D, int dtype, const void *W, const float *xb) {
    const int esz = dtype == RBT_DT_BF16 ? 2 : 4;
    return T >= 16 && (reinterpret_cast<uintptr_t>(W) % 16 == 0) && (reinterpret_cast<uintptr_t>(xb) % 16 == 0) &&
           (D * esz) % 16 == 0 && D % 4 == 0;
}

template <int NCH, int DT>
hipError_t launch_t(const Launch &L, const Launch &Lk, const float *xb, const void *W, const float *bias, int T, int E,
                    int D, int K, int norm_topk, float *probs, int32_t *routing, float *weights) {
    hipError_t e;
    if (NCH == 16 && decode_ok(T, D, DT, W, xb)) {
        e = launch_router_decode(L, xb, W, bias, T, E, D, probs);
    } else if (NCH == 16 && batch_ok(T, D, DT, W, xb)) {
        e = launch(L, router_logits_batch_kernel<DT>, dim3((E + kBRows - 1) / kBRows, (T + kBTok - 1) / kBTok),
                   dim3(256), 0, xb, W, bias, T, E, D, probs);
    } else {
        // 64-thread blocks for small batches (4 or 16 rows each, so one token's router spreads over
        // many CUs); 256 threads (16 rows) for larger batches with the AVX2 order.
        const int threads = (NCH == 16 && T > 8) ? 256 : 64;
        const bool wide = threads / NCH <= 4;
        e = wide ? launch_logits<NCH, DT, true>(L, xb, W, bias, T, E, D, threads, probs)
                 : launch_logits<NCH, DT, false>(L, xb, W, bias, T, E, D, threads, probs);
    }
    if (e != hipSuccess) return e;
    const int tk = E <= 64 ? 64 : 256;
    const size_t lds_k = E <= kLdsProbsMax ? (size_t)E * 4 : 0;
    return launch(Lk, router_topk_kernel, dim3(T), dim3(tk), (uint32_t)lds_k, E, K, norm_topk, probs, routing,
                  weights);
}

}  // namespace

hipError_t launch_router_logits(const Launch &L, int order, int dtype, const float *xb, const void *W,
                                const float *bias, int T, int E, int D, float *logits) {
    if (T <= 0) return hipSuccess;
    if (T > 65535) return hipErrorInvalidValue;
    if (order == RBT_ORDER_AVX2) {
        if (decode_ok(T, D, dtype, W, xb)) return launch_router_decode(L, xb, W, bias, T, E, D, logits);
        if (batch_ok(T, D, dtype, W, xb))
            return dtype == RBT_DT_BF16
                       ? launch(L, router_logits_batch_kernel<RBT_DT_BF16>,
                                dim3((E + kBRows - 1) / kBRows, (T + kBTok - 1) / kBTok), dim3(256), 0, xb, W, bias, T,
                                E, D, logits)
                       : launch(L, router_logits_batch_kernel<RBT_DT_F32>,
                                dim3((E + kBRows - 1) / kBRows, (T + kBTok - 1) / kBTok), dim3(256), 0, xb, W, bias, T,
                                E, D, logits);
        const int threads = T > 8 ? 256 : 64;
        if (dtype == RBT_DT_BF16)
            return threads == 64 ? launch_logits<16, RBT_DT_BF16, true>(L, xb, W, bias, T, E, D, 64, logits)
                                 : launch_logits<16, RBT_DT_BF16, false>(L, xb, W, bias, T, E, D, 256, logits);
        return threads == 64 ? launch_logits<16, RBT_DT_F32, true>(L, xb, W, bias, T, E, D, 64, logits)
                             : launch_logits<16, RBT_DT_F32, false>(L, xb, W, bias, T, E, D, 256, logits);
    }
    return dtype == RBT_DT_BF16 ? launch_logits<4, RBT_DT_BF16, false>(L, xb, W, bias, T, E, D, 64, logits)
                                : launch_logits<4, RBT_DT_F32, false>(L, xb, W, bias, T, E, D, 64, logits);
}

bool router_norm_supported(int order, int dtype, int T, int D, const void *W, const float *x, const float *nw) {
    return order == RBT_ORDER_AVX2 && decode_ok(T, D, dtype, W, x) && (reinterpret_cast<uintptr_t>(nw) & 15u) == 0;
}

hipError_t launch_router_norm(const Launch &L, const float *x, const float *nw, float eps, const void *W,
                              const float *bias, int T, int E, int D, float *logits, float *xb_out) {
    return launch_router_decode_t<true>(L, x, W, bias, T, E, D, logits, nw, eps, xb_out);
}

hipError_t launch_topk_split(const Launch &L, const float *logits, int T, int E, int K, int norm_topk, const float *xb,
                             int D, int32_t *routing, float *weights, uint16_t *x_hi, uint16_t *x_lo) {
    if (T <= 0) return hipSuccess;
    if (T > 65535 || E < 1 || E > 64 || K < 1 || K > E || D % 8 != 0 ||
        ((reinterpret_cast<uintptr_t>(xb) | reinterpret_cast<uintptr_t>(x_hi) | reinterpret_cast<uintptr_t>(x_lo)) & 15u))
        return hipErrorInvalidValue;
    return launch(L, topk_split_kernel, dim3((unsigned)T), dim3(256), 0, logits, E, K, norm_topk, xb, D, routing,
                  weights, x_hi, x_lo);
}

bool router_prefill_supported(int order, int dtype, int T, int E, int D, int K, const void *W, const float *xb) {
    return order == RBT_ORDER_AVX2 && dtype == RBT_DT_BF16 && T >= 1 && E >= 1 && E <= 64 && K <= E && D >= 16 &&
           D % 8 == 0 && (reinterpret_cast<uintptr_t>(W) % 16 == 0) && (reinterpret_cast<uintptr_t>(xb) % 16 == 0);
}

hipError_t launch_router_prefill(const Launch &L, int dtype, const float *xb, const void *W, const float *bias, int T,
                                 int E, int D, int K, int norm_topk, int32_t *routing, float *weights,
                                 uint16_t *x_hi, uint16_t *x_lo) {
    if (T <= 0) return hipSuccess;
    if (dtype != RBT_DT_BF16) return hipErrorNotSupported;  // the grouped path is bf16 only
    const dim3 g((unsigned)((T + kPTok - 1) / kPTok)), b(kPThreads);
    return launch(L, router_prefill_kernel<RBT_DT_BF16>, g, b, 0, xb, W, bias, T, E, D, K, norm_topk, routing, weights,
                  x_hi, x_lo);
}

hipError_t launch_router(const Launch &L, const Launch &Lk, int order, int dtype, const float *xb, const void *W,
                         const float *bias, int T, int E, int D, int K, int norm_topk, float *probs,
                         int32_t *routing, float *weights) {
    if (T <= 0) return hipSuccess;
    if (T > 65535) return hipErrorInvalidValue;  // grid.y limit of the logits kernel
    if (order == RBT_ORDER_AVX2) {
        return dtype == RBT_DT_BF16
                   ? launch_t<16, RBT_DT_BF16>(L, Lk, xb, W, bias, T, E, D, K, norm_topk, probs, routing, weights)
                   : launch_t<16, RBT_DT_F32>(L, Lk, xb, W, bias, T, E, D, K, norm_topk, probs, routing, weights);
    }
    return dtype == RBT_DT_BF16
               ? launch_t<4, RBT_DT_BF16>(L, Lk, xb, W, bias, T, E, D, K, norm_topk, probs, routing, weights)
               : launch_t<4, RBT_DT_F32>(L, Lk, xb, W, bias, T, E, D, K, norm_topk, probs, routing, weights);
}

}  // namespace rbt
