// Expert FFN, GEMV form: one (token, slot) pair at a time. Used for decode (T=1: the 8 experts
// the router picked) and for small batches, where every weight row is used by one token and the
// layer is a pure HBM stream.
//
// Reference: rabbit2/src/rabbit2.c:531-541 -- for each selected expert k (in selection order):
//   h1 = W1 xb, h3 = W3 xb (:535-536), h = silu(h1) * h3 (:537, silu :407), tmp = W2 h (:538),
//   moe += w_k * tmp (:539-540); then x += moe (:542).
// The expert blob layout is the .rbt2 one (rabbit2.c:173, rbt2.py:152-156): w1[H][D] | w3[H][D] |
// w2[D][H] at experts + e*stride.
//
// Memory: one wavefront per output row (pair). Each lane loads 16 bytes per step (8 bf16 or 4
// f32 weights) so a wave pulls 1 KiB per instruction, fully coalesced; gate and up rows share the
// x loads. Dots are accumulated in fp32 and reduced across the wave; only the combine (moe += w*tmp
// in selection order) keeps the engine's sequential order.
#include <math.h>

#include "rbt2_internal.h"

namespace rbt {
namespace {

// ---- per-lane partial dots over n columns of one (or two) weight rows against x (f32).
template <int DT, bool VEC>
__device__ __forceinline__ void dot2(const uint8_t *__restrict__ a, const uint8_t *__restrict__ b,
                                     const float *__restrict__ x, int n, int lane, float &sa, float &sb) {
    float pa = 0.0f, pb = 0.0f;
    if constexpr (VEC && DT == RBT_DT_BF16) {
#pragma unroll 4
        for (int c = lane * 8; c < n; c += kWave * 8) {
            const u32x4 wa = ld_stream_u4(a + (size_t)c * 2);
            const u32x4 wb = ld_stream_u4(b + (size_t)c * 2);
            const f32x4 x0 = ld_f4(x + c);
            const f32x4 x1 = ld_f4(x + c + 4);
            pa += bf16_lo(wa.x) * x0.x + bf16_hi(wa.x) * x0.y + bf16_lo(wa.y) * x0.z + bf16_hi(wa.y) * x0.w +
                  bf16_lo(wa.z) * x1.x + bf16_hi(wa.z) * x1.y + bf16_lo(wa.w) * x1.z + bf16_hi(wa.w) * x1.w;
            pb += bf16_lo(wb.x) * x0.x + bf16_hi(wb.x) * x0.y + bf16_lo(wb.y) * x0.z + bf16_hi(wb.y) * x0.w +
                  bf16_lo(wb.z) * x1.x + bf16_hi(wb.z) * x1.y + bf16_lo(wb.w) * x1.z + bf16_hi(wb.w) * x1.w;
        }
    } else if constexpr (VEC && DT == RBT_DT_F32) {
#pragma unroll 4
        for (int c = lane * 4; c < n; c += kWave * 4) {
            const f32x4 wa = ld_stream_f4(a + (size_t)c * 4);
            const f32x4 wb = ld_stream_f4(b + (size_t)c * 4);
            const f32x4 xv = ld_f4(x + c);
            pa += wa.x * xv.x + wa.y * xv.y + wa.z * xv.z + wa.w * xv.w;
            pb += wb.x * xv.x + wb.y * xv.y + wb.z * xv.z + wb.w * xv.w;
        }
    } else {
        for (int c = lane; c < n; c += kWave) {
            pa += load_w<DT>(a, c) * x[c];
            if (b) pb += load_w<DT>(b, c) * x[c];
        }
    }
    sa = pa;
    sb = pb;
}

template <int DT, bool VEC>
__device__ __forceinline__ float dot1(const uint8_t *__restrict__ a, const float *__restrict__ x, int n, int lane) {
    float p = 0.0f;
    if constexpr (VEC && DT == RBT_DT_BF16) {
#pragma unroll 4
        for (int c = lane * 8; c < n; c += kWave * 8) {
            const u32x4 w = ld_stream_u4(a + (size_t)c * 2);
            const f32x4 x0 = ld_f4(x + c);
            const f32x4 x1 = ld_f4(x + c + 4);
            p += bf16_lo(w.x) * x0.x + bf16_hi(w.x) * x0.y + bf16_lo(w.y) * x0.z + bf16_hi(w.y) * x0.w +
                 bf16_lo(w.z) * x1.x + bf16_hi(w.z) * x1.y + bf16_lo(w.w) * x1.z + bf16_hi(w.w) * x1.w;
        }
    } else if constexpr (VEC && DT == RBT_DT_F32) {
#pragma unroll 4
        for (int c = lane * 4; c < n; c += kWave * 4) {
            const f32x4 w = ld_stream_f4(a + (size_t)c * 4);
            const f32x4 xv = ld_f4(x + c);
            p += w.x * xv.x + w.y * xv.y + w.z * xv.z + w.w * xv.w;
        }
    } else {
        for (int c = lane; c < n; c += kWave) p += load_w<DT>(a, c) * x[c];
    }
    return p;
}

// h[p][j] = silu(W1_e[j] . x_t) * (W3_e[j] . x_t) for every pair p = t*K + k, e = routing[p].
// One wave per (p, j); 4 waves per block; grid covers P*H rows.
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void gateup_gemv_kernel(const uint8_t *__restrict__ experts, uint64_t stride,
                                                          const int32_t *__restrict__ routing,
                                                          const float *__restrict__ xb, int K, int D, int H,
                                                          long long rows, float *__restrict__ hbuf) {
    const int lane = threadIdx.x & (kWave - 1);
    const long long item = (long long)blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave);
    if (item >= rows) return;
    const long long p = item / H;
    const int j = (int)(item - p * H);
    const int e = routing[p];
    const int t = (int)(p / K);
    constexpr size_t esz = DT == RBT_DT_F32 ? 4 : 2;
    const uint8_t *w1 = experts + (size_t)e * stride + (size_t)j * D * esz;
    const uint8_t *w3 = w1 + (size_t)H * D * esz;
    float g, u;
    dot2<DT, VEC>(w1, w3, xb + (size_t)t * D, D, lane, g, u);
    g = wave_sum(g);
    u = wave_sum(u);
    if (lane == 0) hbuf[(size_t)p * H + j] = (g / (1.0f + expf(-g))) * u;
}

// moe[t][d] = sum_k w[t][k] * (W2_e[d] . h[t*K+k]) in selection order; x[t][d] += moe.
// One wave per (t, d); the K dots of a chunk of 8 slots are issued together for memory parallelism.
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void down_combine_kernel(const uint8_t *__restrict__ experts, uint64_t stride,
                                                           const int32_t *__restrict__ routing,
                                                           const float *__restrict__ weights,
                                                           const float *__restrict__ hbuf, int K, int D, int H,
                                                           long long rows, float *__restrict__ x_inout,
                                                           float *__restrict__ moe_out) {
    const int lane = threadIdx.x & (kWave - 1);
    const long long item = (long long)blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave);
    if (item >= rows) return;
    const long long t = item / D;
    const int d = (int)(item - t * D);
    constexpr size_t esz = DT == RBT_DT_F32 ? 4 : 2;
    const size_t w2off = 2 * (size_t)H * D * esz + (size_t)d * H * esz;
    float moe = 0.0f;
    for (int k0 = 0; k0 < K; k0 += 8) {
        const int nk = K - k0 < 8 ? K - k0 : 8;
        float acc[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            acc[kk] = 0.0f;
            if (kk < nk) {
                const long long p = t * K + k0 + kk;
                const int e = routing[p];
                acc[kk] = dot1<DT, VEC>(experts + (size_t)e * stride + w2off, hbuf + (size_t)p * H, H, lane);
            }
        }
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            if (kk < nk) {
                const float tmp = wave_sum(acc[kk]);
                const float wk = weights[t * K + k0 + kk];
                {
#pragma clang fp contract(off)
                    moe = moe + wk * tmp;  // rabbit2.c:540, rounded product then add
                }
            }
        }
    }
    if (lane == 0) {
        const size_t o = (size_t)t * D + d;
        if (moe_out) moe_out[o] = moe;
        if (x_inout) x_inout[o] = x_inout[o] + moe;
    }
}

template <int DT, bool VEC>
__global__ __launch_bounds__(256) void matvec_kernel(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                     float *__restrict__ out, int rows, int cols) {
    const int lane = threadIdx.x & (kWave - 1);
    const long long r = (long long)blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave);
    if (r >= rows) return;
    constexpr size_t esz = DT == RBT_DT_F32 ? 4 : 2;
    const float s = wave_sum(dot1<DT, VEC>(W + (size_t)r * cols * esz, x, cols, lane));
    if (lane == 0) out[r] = s;
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Rows of `n` elements of dtype starting at a 16-byte aligned base stay 16-byte aligned, and x
// vectors of n floats too, when n is a multiple of 8 (bf16) or 4 (f32).
inline bool vec_ok(int dtype, int n) { return dtype == RBT_DT_BF16 ? n % 8 == 0 : n % 4 == 0; }

inline unsigned blocks_for(long long rows) { return (unsigned)((rows + 3) / 4); }

}  // namespace

hipError_t launch_gateup_gemv(const Launch &L, int dtype, const void *experts, uint64_t stride, const int32_t *routing,
                              const float *xb, int T, int K, int D, int H, float *hbuf) {
    const long long rows = (long long)T * K * H;
    if (rows == 0) return hipSuccess;
    const bool vec = vec_ok(dtype, D) && aligned16(experts) && stride % 16 == 0 && aligned16(xb);
    const uint8_t *E = static_cast<const uint8_t *>(experts);
    const dim3 g(blocks_for(rows)), b(256);
    if (dtype == RBT_DT_BF16) {
        if (vec)
            return launch(L, gateup_gemv_kernel<RBT_DT_BF16, true>, g, b, 0, E, stride, routing, xb, K, D, H,
                               rows, hbuf);
        else
            return launch(L, gateup_gemv_kernel<RBT_DT_BF16, false>, g, b, 0, E, stride, routing, xb, K, D, H,
                               rows, hbuf);
    } else {
        if (vec)
            return launch(L, gateup_gemv_kernel<RBT_DT_F32, true>, g, b, 0, E, stride, routing, xb, K, D, H,
                               rows, hbuf);
        else
            return launch(L, gateup_gemv_kernel<RBT_DT_F32, false>, g, b, 0, E, stride, routing, xb, K, D, H,
                               rows, hbuf);
    }
    return hipGetLastError();
}

hipError_t launch_down_combine(const Launch &L, int dtype, const void *experts, uint64_t stride, const int32_t *routing,
                               const float *weights, const float *hbuf, int T, int K, int D, int H, float *x_inout,
                               float *moe_out) {
    const long long rows = (long long)T * D;
    if (rows == 0) return hipSuccess;
    const bool vec = vec_ok(dtype, H) && aligned16(experts) && stride % 16 == 0 && aligned16(hbuf);
    const uint8_t *E = static_cast<const uint8_t *>(experts);
    const dim3 g(blocks_for(rows)), b(256);
    if (dtype == RBT_DT_BF16) {
        if (vec)
            return launch(L, down_combine_kernel<RBT_DT_BF16, true>, g, b, 0, E, stride, routing, weights, hbuf, K, D,
                          H, rows, x_inout, moe_out);
        return launch(L, down_combine_kernel<RBT_DT_BF16, false>, g, b, 0, E, stride, routing, weights, hbuf, K, D, H,
                      rows, x_inout, moe_out);
    }
    if (vec)
        return launch(L, down_combine_kernel<RBT_DT_F32, true>, g, b, 0, E, stride, routing, weights, hbuf, K, D, H,
                      rows, x_inout, moe_out);
    return launch(L, down_combine_kernel<RBT_DT_F32, false>, g, b, 0, E, stride, routing, weights, hbuf, K, D, H, rows,
                  x_inout, moe_out);
}

hipError_t launch_matvec(const Launch &L, int dtype, const void *W, const float *x, float *out, int rows, int cols) {
    if (rows <= 0) return hipSuccess;
    const bool vec = vec_ok(dtype, cols) && aligned16(W) && aligned16(x);
    const uint8_t *Wb = static_cast<const uint8_t *>(W);
    const dim3 g(blocks_for(rows)), b(256);
    if (dtype == RBT_DT_BF16) {
        if (vec)
            return launch(L, matvec_kernel<RBT_DT_BF16, true>, g, b, 0, Wb, x, out, rows, cols);
        else
            return launch(L, matvec_kernel<RBT_DT_BF16, false>, g, b, 0, Wb, x, out, rows, cols);
    } else {
        if (vec)
            return launch(L, matvec_kernel<RBT_DT_F32, true>, g, b, 0, Wb, x, out, rows, cols);
        else
            return launch(L, matvec_kernel<RBT_DT_F32, false>, g, b, 0, Wb, x, out, rows, cols);
    }
    return hipGetLastError();
}

}  // namespace rbt
