// Expert FFN for decode and small batches, specialised for the common shapes: every row length is
// a whole number of 1 KiB wave-steps (D and H multiples of 512 bf16 or 256 f32, at most 8 steps),
// so each wavefront knows its exact load list at compile time and issues all of it before the
// first wait. The generic kernels in experts_gemv.hip cover every other shape.
//
// Reference: rabbit2/src/rabbit2.c:531-541 (per selected expert: h1 = W1 xb, h3 = W3 xb,
// h = silu(h1) * h3, tmp = W2 h, moe += w_k * tmp in selection order; x += moe at :542), experts in
// the .rbt2 blob layout w1[H][D] | w3[H][D] | w2[D][H] (rabbit2.c:173, rbt2.py:152-156).
//
// gateup: one wave per JW consecutive hidden units j of one (token, slot) pair; per lane 2*JW*NC
//   16-byte weight loads + NC x loads, then 2*JW wave sums; h[p][j] = silu(g)*u in f32.
// down:   one block per (token, 4*RW output rows); the token's K hidden vectors are staged once in
//   LDS; per wave, KC slots x RW rows x NH 16-byte weight loads in flight, then the K dot products
//   are combined in selection order exactly like the engine's loop.
// Bytes per decode layer at the OLMoE shape: gateup 64 MiB of weights, down 32 MiB.
#include <math.h>

#include "rbt2_internal.h"

namespace rbt {
namespace {

constexpr int KMAX_T = 64;  // selected experts per token (the engine's MAX_TOPK, rabbit2.c:59)
constexpr int kDownThreads = 512, kDownRows = 1;  // down kernel: block size, output rows per wave
constexpr int kDownPrefetch = 3;  // down kernel: weight slots in flight ahead of the dot products
constexpr int kHStageMax = 8;  // 16-byte units of h per thread in the down kernel: K*H <= 16384 floats
constexpr int EMAX_T = 64;  // experts per layer for the in-kernel top-k (one per lane of wave 0)

// Softmax + top-k of one token's logits, the engine's arithmetic (rabbit2.c:399-405, :516-528,
// :539): leaves the expert ids in s_idx[0..nr) (the first nr <= K places; a round's place does not
// depend on the later rounds) and, with all_k, every place and the combine weights in s_w[0..K).
// Called by every thread of the block (it ends with a barrier); wave 0 does the work, exchanging
// values through LDS with wave-scope fences only (a wave's LDS operations execute in order).
__device__ __forceinline__ void wave_lds_sync() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// XS > 0: the block also stages the token's activation row x (xu 16-byte units, at most XS per
// thread, clamped loads and stores) into xs_lds; its loads are issued next to the logits load, so
// they land while wave 0 selects.
template <int XS = 0>
__device__ __forceinline__ void block_topk(const float *__restrict__ logits, int E, int K, int nr, bool all_k,
                                           int norm_topk, float *s_v, int *s_idx, float *s_pw, float *s_w,
                                           const float *__restrict__ x = nullptr, f32x4 *xs_lds = nullptr,
                                           int xu = 0) {
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    f32x4 xv[XS > 0 ? XS : 1];
    if constexpr (XS > 0) {
#pragma unroll
        for (int i = 0; i < XS; ++i) xv[i] = reinterpret_cast<const f32x4 *>(x)[min(tid + i * (int)blockDim.x, xu - 1)];
    }
    const float v0 = (tid < kWave && lane < E) ? logits[lane] : -INFINITY;
    if constexpr (XS > 0) {
#pragma unroll
        for (int i = 0; i < XS; ++i) xs_lds[min(tid + i * (int)blockDim.x, xu - 1)] = xv[i];
    }
    if (tid < kWave) {
        const float v = v0;
        float mx = wave_max(v);  // ignores NaN like the engine's '>' scan ...
        const float first = lane_value(v, 0);
        if (first != first) mx = first;  // ... which starts from element 0
        const float e = lane < E ? (float)exp((double)(v - mx)) : 0.0f;
        s_v[lane] = e;
        wave_lds_sync();
        // every lane forms the sum itself, sequentially in the engine's order (entries past E are 0
        // and come last, so they do not change it)
        const f32x4 *p4 = reinterpret_cast<const f32x4 *>(s_v);
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < EMAX_T / 4; ++q) {
            const f32x4 v4 = p4[q];
            sum = sum + v4.x;
            sum = sum + v4.y;
            sum = sum + v4.z;
            sum = sum + v4.w;
        }
        const float p = e / sum;
        if (sum != sum) {
            if (lane < K) {  // all NaN: the engine keeps the first unused index each round
                s_idx[lane] = lane;
                s_pw[lane] = p;
            }
        } else {
            // K rounds of the engine's selection: the largest remaining probability, the lowest index
            // among equal ones (its strict '>' scan from index 0); a wave maximum and a ballot per
            // round. Probabilities are finite and >= 0 here, so lanes past E (-1) never win and a
            // taken lane (-2) is out for good.
            float cand = lane < E ? p : -1.0f;
            auto round = [&](int k) {
                const float m = wave_max(cand);
                const int w = __builtin_ctzll(__ballot(cand == m));
                if (lane == w) {
                    s_idx[k] = lane;
                    s_pw[k] = p;
                    cand = -2.0f;
                }
            };
            const int n = all_k ? K : nr;
            if (n == 8) {  // the common top-8, unrolled
#pragma unroll
                for (int k = 0; k < 8; ++k) round(k);
            } else {
                for (int k = 0; k < n; ++k) round(k);
            }
        }
        wave_lds_sync();
        if (all_k) {  // the combine weights, for the block that publishes them
            float wsum = 0.0f;
            if (K <= 8) {  // one LDS round trip instead of K dependent ones; the engine's order
                const f32x4 a = reinterpret_cast<const f32x4 *>(s_pw)[0], b = reinterpret_cast<const f32x4 *>(s_pw)[1];
                const float pw[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if (k < K) wsum = wsum + pw[k];
            } else {
                for (int k = 0; k < K; ++k) wsum = wsum + s_pw[k];
            }
            if (lane < K) s_w[lane] = norm_topk ? s_pw[lane] / wsum : s_pw[lane];
        }
    }
    __syncthreads();
}

template <int DT>
struct Elem {
    static constexpr int kEsz = DT == RBT_DT_F32 ? 4 : 2;
    static constexpr int kPer = 16 / kEsz;  // weights per 16-byte load
};

// dot of 16 bytes of weights with the matching kPer floats of x
template <int DT>
__device__ __forceinline__ float dot16(const u32x4 w, const float *x) {
    if constexpr (DT == RBT_DT_BF16) {
        const f32x4 x0 = *reinterpret_cast<const f32x4 *>(x);
        const f32x4 x1 = *reinterpret_cast<const f32x4 *>(x + 4);
        return bf16_lo(w.x) * x0.x + bf16_hi(w.x) * x0.y + bf16_lo(w.y) * x0.z + bf16_hi(w.y) * x0.w +
               bf16_lo(w.z) * x1.x + bf16_hi(w.z) * x1.y + bf16_lo(w.w) * x1.z + bf16_hi(w.w) * x1.w;
    } else {
        const f32x4 x0 = *reinterpret_cast<const f32x4 *>(x);
        return __uint_as_float(w.x) * x0.x + __uint_as_float(w.y) * x0.y + __uint_as_float(w.z) * x0.z +
               __uint_as_float(w.w) * x0.w;
    }
}

template <int DT>
__device__ __forceinline__ float dot16r(const u32x4 w, const f32x4 x0, const f32x4 x1) {
    if constexpr (DT == RBT_DT_BF16) {
        return bf16_lo(w.x) * x0.x + bf16_hi(w.x) * x0.y + bf16_lo(w.y) * x0.z + bf16_hi(w.y) * x0.w +
               bf16_lo(w.z) * x1.x + bf16_hi(w.z) * x1.y + bf16_lo(w.w) * x1.z + bf16_hi(w.w) * x1.w;
    } else {
        (void)x1;
        return __uint_as_float(w.x) * x0.x + __uint_as_float(w.y) * x0.y + __uint_as_float(w.z) * x0.z +
               __uint_as_float(w.w) * x0.w;
    }
}

// grid: ceil(P*H/JW / 4) blocks of 4 waves; requires H % JW == 0 and D == NC * 64 * kPer.
// TOPK (batch 1 only): every block first runs the token's softmax + top-k from the router logits
// (`logits`, E experts) instead of reading `routing`, as far as the slots of its items; the last block
// runs all K places and publishes routing/weights for the down kernel. Saves a launch on the decode
// critical path.
// With TOPK (one token) the block stages x in LDS once (XS units per thread) instead of every wave
// reading all of it from L2.
template <int DT, int NC, int JW, bool TOPK>
__global__ __launch_bounds__(256) void gateup_fast_kernel(const uint8_t *__restrict__ experts, uint64_t stride,
                                                          int32_t *__restrict__ routing,
                                                          const float *__restrict__ xb, int K, int H,
                                                          long long items, float *__restrict__ hbuf,
                                                          const float *__restrict__ logits, int E, int norm_topk,
                                                          float *__restrict__ weights) {
    constexpr int kEsz = Elem<DT>::kEsz, kPer = Elem<DT>::kPer;
    constexpr int D = NC * kWave * kPer;
    constexpr int XS = TOPK ? (D / 4 + 255) / 256 : 0;  // x units per thread (D <= 4096: at most 4)
    __shared__ __align__(16) f32x4 xs_lds[TOPK ? D / 4 : 1];
    const int lane = threadIdx.x & (kWave - 1);
    const long long item = (long long)blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave);
    int e;
    if constexpr (TOPK) {
        __shared__ __align__(16) float s_v[EMAX_T];
        __shared__ int s_idx[KMAX_T];
        __shared__ __align__(16) float s_pw[KMAX_T];
        __shared__ float s_w[KMAX_T];
        // the block's items lie in slots 0 .. that of its last item, so it needs that many selection
        // rounds; the last block holds slot K - 1 and publishes routing and weights for the down kernel
        const long long last = min(items, (long long)(blockIdx.x + 1) * (blockDim.x / kWave)) - 1;
        const int nr = (int)((last * JW) / H) + 1;
        const bool pub = blockIdx.x == gridDim.x - 1;
        block_topk<XS>(logits, E, K, nr, pub, norm_topk, s_v, s_idx, s_pw, s_w, xb, xs_lds, D / 4);
        if (pub && (int)threadIdx.x < K) {
            routing[threadIdx.x] = s_idx[threadIdx.x];
            weights[threadIdx.x] = s_w[threadIdx.x];
        }
        if (item >= items) return;
        e = s_idx[(int)((item * JW) / H)];
    } else {
        if (item >= items) return;
        e = routing[(item * JW) / H];
    }
    const long long row0 = item * JW;
    const long long p = row0 / H;
    const int j0 = (int)(row0 - p * H);
    const int t = (int)(p / K);
    const uint8_t *w1 = experts + (size_t)e * stride + (size_t)j0 * D * kEsz;
    const uint8_t *w3 = w1 + (size_t)H * D * kEsz;
    const float *x = xb + (size_t)t * D;

    u32x4 a[JW][NC], b[JW][NC];
    f32x4 x0[NC], x1[NC];
#pragma unroll
    for (int jj = 0; jj < JW; ++jj)
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const size_t off = ((size_t)jj * D + (size_t)(lane + kWave * i) * kPer) * kEsz;
            a[jj][i] = ld_stream_u4(w1 + off);
            b[jj][i] = ld_stream_u4(w3 + off);
        }
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const float *xp = (XS > 0 ? reinterpret_cast<const float *>(xs_lds) : x) + (lane + kWave * i) * kPer;
        x0[i] = *reinterpret_cast<const f32x4 *>(xp);
        if constexpr (DT == RBT_DT_BF16) x1[i] = *reinterpret_cast<const f32x4 *>(xp + 4);
    }
    // keep the scheduler from sinking the loads next to their uses: all of them go out first
    __builtin_amdgcn_sched_barrier(0);
    float g[JW], u[JW];
#pragma unroll
    for (int jj = 0; jj < JW; ++jj) {
        g[jj] = 0.0f;
        u[jj] = 0.0f;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            g[jj] += dot16r<DT>(a[jj][i], x0[i], x1[i]);
            u[jj] += dot16r<DT>(b[jj][i], x0[i], x1[i]);
        }
    }
#pragma unroll
    for (int jj = 0; jj < JW; ++jj) {
        const float gs = wave_sum(g[jj]), us = wave_sum(u[jj]);
        if (lane == jj) hbuf[(size_t)p * H + j0 + jj] = (gs / (1.0f + expf(-gs))) * us;
    }
}

// grid (ceil(D / (BT/64*RW)), T), block BT, dynamic LDS K*H*4 bytes; requires H == NH * 64 * kPer.
// HS: 16-byte units of h staged per thread (K*H/4 <= BT*HS). PD: slots of weight rows in flight when
// the block waits for h (0: every slot of the first chunk).
template <int DT, int NH, int RW, int HS, int BT, int PD>
__global__ __launch_bounds__(BT) void down_fast_kernel(const uint8_t *__restrict__ experts, uint64_t stride,
                                                        const int32_t *__restrict__ routing,
                                                        const float *__restrict__ weights,
                                                        const float *__restrict__ hbuf, int K, int D,
                                                        float *__restrict__ x_inout, float *__restrict__ moe_out) {
    constexpr int kEsz = Elem<DT>::kEsz, kPer = Elem<DT>::kPer;
    constexpr int H = NH * kWave * kPer;
    constexpr int KC = NH <= 2 ? 8 : 4;  // slots whose loads are in flight together (<= 32 per lane)
    extern __shared__ __align__(16) float hs[];  // [K][H]
    __shared__ float s_w[64];
    const int t = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;

    const int d0 = (blockIdx.x * (blockDim.x / kWave) + wv) * RW;
    const bool active = d0 < D;
    const int dbase = active ? d0 : 0;  // inactive waves still help stage h; their loads stay in range
    const int nr = D - dbase < RW ? D - dbase : RW;
    const int32_t *rt = routing + (size_t)t * K;

    // Load order: this thread's share of h first (small, from L2), then the weight loads of the first
    // PD slots, then the h stores to LDS. Loads complete in issue order, so the stores wait only for
    // the h loads while those weight loads are in flight. After the barrier each slot's dot products
    // run with the next PD slots in flight: a CU holds only so many outstanding misses, so a wave that
    // issued its whole stream first would stall at its loads and compute only after the last one.
    const f32x4 *hsrc = reinterpret_cast<const f32x4 *>(hbuf + (size_t)t * K * H);
    f32x4 *hdst = reinterpret_cast<f32x4 *>(hs);
    const int units = K * H / 4;  // 16-byte units of h, at most HS per thread
    f32x4 hv[HS];
#pragma unroll
    for (int i = 0; i < HS; ++i) hv[i] = hsrc[min(tid + i * (int)blockDim.x, units - 1)];
    const float wsel = weights[(size_t)t * K + min(tid & 63, K - 1)];

    u32x4 w[KC][RW][NH];
    auto load_slot = [&](int k0, int nk, int kk) {
        const int slot = k0 + (kk < nk ? kk : 0);  // clamped: always a valid expert row
        const uint8_t *base = experts + (size_t)rt[slot] * stride + 2 * (size_t)H * D * kEsz;
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const int d = dbase + (r < nr ? r : 0);
#pragma unroll
            for (int i = 0; i < NH; ++i)
                w[kk][r][i] = ld_stream_u4(base + ((size_t)d * H + (size_t)(lane + kWave * i) * kPer) * kEsz);
        }
    };
    auto load_chunk = [&](int k0, int nk) {
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) load_slot(k0, nk, kk);
    };
    constexpr int P0 = PD > 0 && PD < KC ? PD : KC;
    const int nk0 = K < KC ? K : KC;
#pragma unroll
    for (int kk = 0; kk < P0; ++kk) load_slot(0, nk0, kk);
    __builtin_amdgcn_sched_barrier(0);  // these weight loads issued before the h stores wait on h
    // unconditional stores (clamped lanes rewrite the last unit with the same data): a store behind a
    // branch would let the compiler sink its load into the branch, after the weight stream
#pragma unroll
    for (int i = 0; i < HS; ++i) hdst[min(tid + i * (int)blockDim.x, units - 1)] = hv[i];
    s_w[tid & 63] = wsel;  // entries past K hold weight K-1 and are never read
    __syncthreads();

    // The first chunk is consumed in straight-line code right after the barrier, and waves past D work
    // on clamped rows and only skip the final store: the weights are read-only to this kernel, so the
    // compiler may move their loads anywhere before the first use, and a use behind a branch (an
    // early exit, a loop) would let it sink them below the barrier, serialising the stream.
    float moe[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) moe[r] = 0.0f;
    // slot kk's products: its rows . h_kk over the lane's elements, then the wave sum
    auto slot_dot = [&](int k0, int nk, int kk, float (&acc)[RW]) {
        const float *hk = hs + (size_t)(k0 + (kk < nk ? kk : 0)) * H;
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < NH; ++i) {
            const float *hp = hk + (lane + kWave * i) * kPer;
#pragma unroll
            for (int r = 0; r < RW; ++r) acc[r] += dot16<DT>(w[kk][r][i], hp);
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[r] = wave_sum(acc[r]);
    };
    auto add_slot = [&](int k0, int kk, const float (&acc)[RW]) {
        const float wk = s_w[k0 + kk];
#pragma unroll
        for (int r = 0; r < RW; ++r) {
#pragma clang fp contract(off)
            moe[r] = moe[r] + wk * acc[r];  // rabbit2.c:540, rounded product then add
        }
    };
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) {
        if (kk + P0 < KC) load_slot(0, nk0, kk + P0);  // P0 slots ahead of the one computed now
        __builtin_amdgcn_sched_barrier(0);
        float acc[RW];
        slot_dot(0, nk0, kk, acc);
        if (kk < nk0) add_slot(0, kk, acc);
    }
    auto process = [&](int k0, int nk) {
        float acc[KC][RW];
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) slot_dot(k0, nk, kk, acc[kk]);
        for (int kk = 0; kk < nk; ++kk) add_slot(k0, kk, acc[kk]);
    };
    for (int k0 = KC; k0 < K; k0 += KC) {
        const int nk = K - k0 < KC ? K - k0 : KC;
        load_chunk(k0, nk);
        __builtin_amdgcn_sched_barrier(0);  // every weight load of the chunk is issued before any use
        process(k0, nk);
    }
    if (lane == 0 && active) {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            if (r < nr) {
                const size_t o = (size_t)t * D + d0 + r;
                if (moe_out) moe_out[o] = moe[r];
                if (x_inout) x_inout[o] = x_inout[o] + moe[r];
            }
        }
    }
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int DT, int NC>
hipError_t gateup_nc(const Launch &L, const uint8_t *E, uint64_t stride, int32_t *routing, const float *xb, int T,
                     int K, int H, float *hbuf, const float *logits, int nE, int norm_topk, float *weights) {
    constexpr int JW = 2;
    const long long items = (long long)T * K * H / JW;
    const dim3 g((unsigned)((items + 3) / 4)), b(256);
    if (logits)
        return launch(L, gateup_fast_kernel<DT, NC, JW, true>, g, b, 0, E, stride, routing, xb, K, H, items, hbuf,
                      logits, nE, norm_topk, weights);
    return launch(L, gateup_fast_kernel<DT, NC, JW, false>, g, b, 0, E, stride, routing, xb, K, H, items, hbuf,
                  logits, nE, norm_topk, weights);
}

template <int DT, int NH>
hipError_t down_nh(const Launch &L, const uint8_t *E, uint64_t stride, const int32_t *routing, const float *weights,
                   const float *hbuf, int T, int K, int D, float *x_inout, float *moe_out) {
    constexpr int RW = kDownRows, BT = kDownThreads, WPB = BT / kWave;
    constexpr int H = NH * kWave * Elem<DT>::kPer;
    const dim3 g((unsigned)((D + WPB * RW - 1) / (WPB * RW)), (unsigned)T), b(BT);
    const uint32_t lds = (uint32_t)((size_t)K * H * 4);
    const int per = (K * H / 4 + BT - 1) / BT;  // h units per thread
    if (per <= 2)
        return launch(L, down_fast_kernel<DT, NH, RW, 2, BT, kDownPrefetch>, g, b, lds, E, stride, routing, weights, hbuf, K, D,
                      x_inout, moe_out);
    if (per <= 4)
        return launch(L, down_fast_kernel<DT, NH, RW, 4, BT, kDownPrefetch>, g, b, lds, E, stride, routing, weights, hbuf, K, D,
                      x_inout, moe_out);
    return launch(L, down_fast_kernel<DT, NH, RW, kHStageMax, BT, kDownPrefetch>, g, b, lds, E, stride, routing, weights, hbuf, K,
                  D, x_inout, moe_out);
}

template <int DT>
hipError_t decode_dt(const Launch &Lg, const Launch &Ld, const uint8_t *E, uint64_t stride, int32_t *routing,
                     float *weights, const float *xb, float *hbuf, int T, int K, int D, int H, float *x_inout,
                     float *moe_out, const float *logits, int nE, int norm_topk) {
    constexpr int step = kWave * Elem<DT>::kPer;
    const int nc = D / step, nh = H / step;
    hipError_t e;
    switch (nc) {
        case 1: e = gateup_nc<DT, 1>(Lg, E, stride, routing, xb, T, K, H, hbuf, logits, nE, norm_topk, weights); break;
        case 2: e = gateup_nc<DT, 2>(Lg, E, stride, routing, xb, T, K, H, hbuf, logits, nE, norm_topk, weights); break;
        case 3: e = gateup_nc<DT, 3>(Lg, E, stride, routing, xb, T, K, H, hbuf, logits, nE, norm_topk, weights); break;
        case 4: e = gateup_nc<DT, 4>(Lg, E, stride, routing, xb, T, K, H, hbuf, logits, nE, norm_topk, weights); break;
        case 6: e = gateup_nc<DT, 6>(Lg, E, stride, routing, xb, T, K, H, hbuf, logits, nE, norm_topk, weights); break;
        case 8: e = gateup_nc<DT, 8>(Lg, E, stride, routing, xb, T, K, H, hbuf, logits, nE, norm_topk, weights); break;
        default: return hipErrorNotSupported;
    }
    if (e != hipSuccess) return e;
    switch (nh) {
        case 1: return down_nh<DT, 1>(Ld, E, stride, routing, weights, hbuf, T, K, D, x_inout, moe_out);
        case 2: return down_nh<DT, 2>(Ld, E, stride, routing, weights, hbuf, T, K, D, x_inout, moe_out);
        case 3: return down_nh<DT, 3>(Ld, E, stride, routing, weights, hbuf, T, K, D, x_inout, moe_out);
        case 4: return down_nh<DT, 4>(Ld, E, stride, routing, weights, hbuf, T, K, D, x_inout, moe_out);
        default: return hipErrorNotSupported;
    }
}

}  // namespace

bool experts_decode_supported(int dtype, int T, int K, int D, int H, const void *experts, uint64_t stride,
                              const float *xb, const float *hbuf) {
    const int step = dtype == RBT_DT_BF16 ? 512 : 256;
    const int nc = D / step, nh = H / step;
    const bool nc_ok = D % step == 0 && (nc == 1 || nc == 2 || nc == 3 || nc == 4 || nc == 6 || nc == 8);
    const bool nh_ok = H % step == 0 && nh >= 1 && nh <= 4;
    return nc_ok && nh_ok && H % 2 == 0 && T >= 1 && T <= 65535 && (size_t)K * H <= 4 * (size_t)kDownThreads * kHStageMax &&
           aligned16(experts) && stride % 16 == 0 && aligned16(xb) && aligned16(hbuf);
}

hipError_t launch_experts_decode(const Launch &Lg, const Launch &Ld, int dtype, const void *experts, uint64_t stride,
                                 int32_t *routing, float *weights, const float *xb, float *hbuf, int T, int K, int D,
                                 int H, float *x_inout, float *moe_out, const float *logits, int E, int norm_topk) {
    if (logits && (T != 1 || E > EMAX_T)) return hipErrorInvalidValue;
    const uint8_t *Eb = static_cast<const uint8_t *>(experts);
    return dtype == RBT_DT_BF16 ? decode_dt<RBT_DT_BF16>(Lg, Ld, Eb, stride, routing, weights, xb, hbuf, T, K, D, H,
                                                         x_inout, moe_out, logits, E, norm_topk)
                                : decode_dt<RBT_DT_F32>(Lg, Ld, Eb, stride, routing, weights, xb, hbuf, T, K, D, H,
                                                        x_inout, moe_out, logits, E, norm_topk);
}

}  // namespace rbt
