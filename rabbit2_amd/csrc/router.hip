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
// Each chain is one thread: the work is D/16 (or D/4) dependent adds per thread, and a token's
// E rows are spread over ceil(E/rows_per_block) blocks so the router bytes stream through many CUs.
// No multiply-add contraction anywhere in this file: every product is rounded before its add,
// exactly as the engine's `-std=c99` build does.
#pragma clang fp contract(off)

#include <math.h>

#include "rbt2_internal.h"

namespace rbt {
namespace {

constexpr int kLdsProbsMax = 4096;  // tokens with E <= this keep probabilities in LDS

__device__ float block_max_f(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
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

// grid (ceil(E/rpb), T), block rpb*NCH threads (a multiple of 64, at most 256).
template <int NCH, int DT>
__global__ __launch_bounds__(256) void router_kernel(const float *__restrict__ xb, const void *__restrict__ W,
                                                     const float *__restrict__ bias, int E, int D, int K,
                                                     int norm_topk, int rpb, float *__restrict__ probs,
                                                     unsigned *__restrict__ counters, int32_t *__restrict__ routing,
                                                     float *__restrict__ weights) {
    extern __shared__ float smem[];  // max(blockDim, E<=kLdsProbsMax ? E : 0) floats
    __shared__ float red_f[4];
    __shared__ unsigned long long red_u[4];
    __shared__ int s_last;
    __shared__ int32_t s_idx[64];
    __shared__ float s_wt[64];
    __shared__ float s_sum;

    const int t = blockIdx.y;
    const int tid = threadIdx.x;
    const int rr = tid / NCH, c = tid - rr * NCH;
    const int r = blockIdx.x * rpb + rr;
    const float *x = xb + (size_t)t * D;
    float *prow = probs + (size_t)t * E;
    const int nfull = D / NCH;

    // ---- one chain per thread
    float acc = 0.0f;
    if (r < E) {
        const size_t rb = (size_t)r * D;
#pragma unroll 8
        for (int m = 0; m < nfull; ++m) {
            const int col = m * NCH + c;
            acc = acc + load_w<DT>(W, rb + col) * x[col];
        }
    }
    smem[tid] = acc;
    __syncthreads();
    if (c == 0 && r < E) {
        const size_t rb = (size_t)r * D;
        float res;
        if constexpr (NCH == 16) {
            float sum = 0.0f;
            for (int j = 0; j < 8; ++j) sum = sum + (smem[tid + j] + smem[tid + 8 + j]);
            for (int i = nfull * 16; i < D; ++i) sum = sum + load_w<DT>(W, rb + i) * x[i];
            res = sum;
        } else {
            float s0 = smem[tid], s1 = smem[tid + 1], s2 = smem[tid + 2], s3 = smem[tid + 3];
            for (int i = nfull * 4; i < D; ++i) s0 = s0 + load_w<DT>(W, rb + i) * x[i];
            res = (s0 + s1) + (s2 + s3);
        }
        if (bias) res = res + bias[r];
        prow[r] = res;
    }

    // ---- the last block of this token to finish does softmax + top-k (no spinning: the others exit)
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&counters[t], 1u) == gridDim.x - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    const int nt = blockDim.x;
    const bool lds = E <= kLdsProbsMax;
    float *pb = lds ? smem : prow;
    __syncthreads();  // smem held the chain partials until here
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
        // expf rounded correctly from a double evaluation (glibc's expf is within 0.502 ulp)
        pb[i] = (float)exp((double)(pb[i] - mx));
    }
    if (!lds) __threadfence();
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int i = 0; i < E; ++i) sum = sum + pb[i];  // the engine's sequential order
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
        counters[t] = 0u;  // ready for the next launch
    }
}

template <int NCH, int DT>
hipError_t launch_t(hipStream_t s, const float *xb, const void *W, const float *bias, int T, int E, int D, int K,
                    int norm_topk, float *probs, unsigned *counters, int32_t *routing, float *weights) {
    // Small batches: 64-thread blocks (4 or 16 rows) so even one token spreads over E/rpb CUs.
    const int threads = T <= 8 ? 64 : 256;
    const int rpb = threads / NCH;
    const dim3 grid((E + rpb - 1) / rpb, T);
    const int lds_floats = E <= kLdsProbsMax ? (E > threads ? E : threads) : threads;
    hipLaunchKernelGGL((router_kernel<NCH, DT>), grid, dim3(threads), lds_floats * sizeof(float), s, xb, W, bias, E,
                       D, K, norm_topk, rpb, probs, counters, routing, weights);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_router(hipStream_t s, int order, int dtype, const float *xb, const void *W, const float *bias, int T,
                         int E, int D, int K, int norm_topk, float *probs, unsigned *counters, int32_t *routing,
                         float *weights) {
    if (T <= 0) return hipSuccess;
    if (order == RBT_ORDER_AVX2) {
        return dtype == RBT_DT_BF16
                   ? launch_t<16, RBT_DT_BF16>(s, xb, W, bias, T, E, D, K, norm_topk, probs, counters, routing, weights)
                   : launch_t<16, RBT_DT_F32>(s, xb, W, bias, T, E, D, K, norm_topk, probs, counters, routing, weights);
    }
    return dtype == RBT_DT_BF16
               ? launch_t<4, RBT_DT_BF16>(s, xb, W, bias, T, E, D, K, norm_topk, probs, counters, routing, weights)
               : launch_t<4, RBT_DT_F32>(s, xb, W, bias, T, E, D, K, norm_topk, probs, counters, routing, weights);
}

}  // namespace rbt
