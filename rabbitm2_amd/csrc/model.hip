// The rest of the engine's per-token forward pass on the GPU, around the MoE block: token embedding,
// RMSNorm, the q/k/v, wo and lm_head matvecs, QK-norm, RoPE, the KV cache in HBM, attention, and the
// greedy argmax. Reference: rabbit2/src/rabbit2.c:453-548 (forward), :392-397 (rmsnorm), :399-405
// (softmax), :410-423 (rope), :552-556 (argmax), :703-740 (the prompt and --gen loops).
//
// Every kernel reads the token and position of the step from a small device record (StepState), so
// one captured step replays unchanged for every position: the prompt's tokens sit in seq[] before the
// first step, and the argmax kernel appends each generated token to seq[] and advances pos. A step can
// carry B independent sequences (batched decode): the per-token kernels take the sequence from a grid
// dimension, each sequence with its own record, token row seq[b][ctx] and KV cache.
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
                                                    int ctx, float *__restrict__ x) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, b = blockIdx.y;
    if (i >= D) return;
    x += (size_t)b * D;
    int tok = seq[(size_t)b * ctx + st[b].pos];
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

// ---------------------------------------------------------------- dense matvec, many rows per wave
// Rows of D = NC * 64 * kPer elements (D a multiple of 512 bf16 / 256 f32): each wave takes RPW
// consecutive rows and issues all RPW * NC of its 16-byte loads before the input vector is staged,
// so the weight stream is in flight while the block computes the RMSNorm (MODE 0/2) or stages the
// attention output (MODE 1).
//   MODE 0: out_s[r] = W_s[r] . (x * inv * nw)          (q/k/v: up to three row segments)
//   MODE 1: x[r] += W[r] . a (wo + residual, rabbit2.c:500-501)
//   MODE 2: out[r] = W[r] . (x * inv * nw), and the block's argmax candidate (largest value, first
//           index) to cand[block] for argmax_cand_kernel (lm_head, rabbit2.c:545-546)
template <int DT, int NC, int RPW, int MODE, int WPB>
__global__ __launch_bounds__(64 * WPB) void dense_kernel(const float *__restrict__ x, const float *__restrict__ nw,
                                                         float eps, Segs sg, int total_rows, float *__restrict__ resid,
                                                         float2 *__restrict__ cand) {
    constexpr int kPer = DT == RBT_DT_BF16 ? 8 : 4, kEsz = DT == RBT_DT_BF16 ? 2 : 4;
    constexpr int D = NC * kWave * kPer;
    __shared__ __align__(16) float xs[D];
    __shared__ float red[16];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r0 = (blockIdx.x * WPB + wv) * RPW;
    // the input vector (and norm weights) first: D / (64 WPB) elements per thread in i = tid, tid + 64 WPB,
    // ... order; loads return in issue order, so the norm below waits for these and not for the
    // weight rows, which stream in while the block reduces and stages x
    constexpr int XU = (D + 64 * WPB - 1) / (64 * WPB);
    float xr[XU], nr[XU];
#pragma unroll
    for (int u = 0; u < XU; ++u) {
        const int i = threadIdx.x + 64 * WPB * u;
        xr[u] = i < D ? x[i] : 0.0f;
        nr[u] = MODE == 1 || i >= D ? 0.0f : nw[i];
    }
    __builtin_amdgcn_sched_barrier(0);
    // then the weights: row r0 + j (clamped into range; clamped rows are computed and dropped)
    u32x4 w[RPW][NC];
    int seg[RPW], row[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        int r = min(r0 + j, total_rows - 1), s = 0;
        while (s < 2 && r >= sg.rows[s]) {
            r -= sg.rows[s];
            ++s;
        }
        seg[j] = s;
        row[j] = r;
        const uint8_t *src = sg.W[s] + (size_t)r * D * kEsz;
#pragma unroll
        for (int i = 0; i < NC; ++i) w[j][i] = ld_stream_u4(src + (size_t)(lane + kWave * i) * 16);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (MODE == 1) {
#pragma unroll
        for (int u = 0; u < XU; ++u)
            if (threadIdx.x + 64 * WPB * u < D) xs[threadIdx.x + 64 * WPB * u] = xr[u];
    } else {
        float ss = 0.0f;  // rms_inv's per-thread order
#pragma unroll
        for (int u = 0; u < XU; ++u) ss += xr[u] * xr[u];
        ss = block_sum(ss, red);
        const float inv = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
        for (int u = 0; u < XU; ++u)
            if (threadIdx.x + 64 * WPB * u < D) xs[threadIdx.x + 64 * WPB * u] = xr[u] * inv * nr[u];
    }
    __syncthreads();
    float acc[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        acc[j] = 0.0f;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const float *xp = xs + (lane + kWave * i) * kPer;
            if constexpr (DT == RBT_DT_BF16) {
                const f32x4 x0 = *reinterpret_cast<const f32x4 *>(xp), x1 = *reinterpret_cast<const f32x4 *>(xp + 4);
                const u32x4 v = w[j][i];
                acc[j] += bf16_lo(v.x) * x0.x + bf16_hi(v.x) * x0.y + bf16_lo(v.y) * x0.z + bf16_hi(v.y) * x0.w +
                          bf16_lo(v.z) * x1.x + bf16_hi(v.z) * x1.y + bf16_lo(v.w) * x1.z + bf16_hi(v.w) * x1.w;
            } else {
                const f32x4 x0 = *reinterpret_cast<const f32x4 *>(xp);
                const u32x4 v = w[j][i];
                acc[j] += __uint_as_float(v.x) * x0.x + __uint_as_float(v.y) * x0.y + __uint_as_float(v.z) * x0.z +
                          __uint_as_float(v.w) * x0.w;
            }
        }
    }
    float best = -INFINITY;
    int bi = -1;
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        const float v = wave_sum(acc[j]);
        const bool valid = r0 + j < total_rows;
        if (lane == 0 && valid) {
            if constexpr (MODE == 1)
                resid[row[j]] = resid[row[j]] + v;
            else
                sg.out[seg[j]][row[j]] = v;
        }
        if constexpr (MODE == 2) {
            if (valid && v == v && (bi < 0 || v > best)) {  // rows ascend: equal values keep the first
                best = v;
                bi = r0 + j;
            }
        }
    }
    if constexpr (MODE == 2) {
        __shared__ float s_b[WPB];
        __shared__ int s_i[WPB];
        if (lane == 0) {
            s_b[wv] = best;
            s_i[wv] = bi;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float b = -INFINITY;
            int k = -1;
            for (int q = 0; q < WPB; ++q)
                if (s_i[q] >= 0 && (k < 0 || s_b[q] > b || (s_b[q] == b && s_i[q] < k))) {
                    b = s_b[q];
                    k = s_i[q];
                }
            cand[blockIdx.x] = make_float2(b, __int_as_float(k));
        }
    }
}

// ---------------------------------------------------------------- dense matvec over B tokens
// The rows of dense_kernel for B token vectors (batched decode): each wave keeps its RPW rows' weights
// in registers, and the B input rows pass through LDS TB at a time, so every weight is read from HBM
// once per step whatever B is.
//   MODE 0: out_s[b * rows_s + r] = W_s[r] . xin[b]     (q/k/v, lm_head)
//   MODE 1: resid[b * total_rows + r] += W[r] . xin[b]   (wo + residual)
template <int DT, int NC, int RPW, int MODE>
__global__ __launch_bounds__(256) void dense_batch_kernel(const float *__restrict__ xin, int B, Segs sg, int total_rows,
                                                          float *__restrict__ resid) {
    constexpr int kPer = DT == RBT_DT_BF16 ? 8 : 4, kEsz = DT == RBT_DT_BF16 ? 2 : 4;
    constexpr int D = NC * kWave * kPer;
    constexpr int TB = 16384 / D < 16 ? 16384 / D : 16;  // 64 KiB of LDS
    __shared__ __align__(16) float xs[TB * D];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r0 = (blockIdx.x * 4 + wv) * RPW;
    u32x4 w[RPW][NC];
    int seg[RPW], row[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        int r = min(r0 + j, total_rows - 1), s = 0;
        while (s < 2 && r >= sg.rows[s]) {
            r -= sg.rows[s];
            ++s;
        }
        seg[j] = s;
        row[j] = r;
        const uint8_t *src = sg.W[s] + (size_t)r * D * kEsz;
#pragma unroll
        for (int i = 0; i < NC; ++i) w[j][i] = ld_stream_u4(src + (size_t)(lane + kWave * i) * 16);
    }
    constexpr int UPT = (TB * D / 4 + 255) / 256;  // 16-byte staging units per thread for a full chunk
    for (int b0 = 0; b0 < B; b0 += TB) {  // block-uniform
        const int nb = B - b0 < TB ? B - b0 : TB;
        const int nu = nb * D / 4;
        // the chunk's token rows: every load issued before the first store (indices clamped, so the
        // loads carry no branches)
        f32x4 sv[UPT];
        const f32x4 *src4 = reinterpret_cast<const f32x4 *>(xin + (size_t)b0 * D);
#pragma unroll
        for (int k = 0; k < UPT; ++k) sv[k] = src4[min((int)threadIdx.x + 256 * k, nu - 1)];
        __syncthreads();  // the previous chunk's reads are done
#pragma unroll
        for (int k = 0; k < UPT; ++k) {
            const int u = threadIdx.x + 256 * k;
            if (u < nu) reinterpret_cast<f32x4 *>(xs)[u] = sv[k];
        }
        __syncthreads();
        float res[RPW];  // lane tt keeps token b0 + tt's sums
#pragma unroll
        for (int j = 0; j < RPW; ++j) res[j] = 0.0f;
        for (int tt = 0; tt < nb; ++tt) {
            const float *xt = xs + tt * D;
#pragma unroll
            for (int j = 0; j < RPW; ++j) {
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < NC; ++i) {
                    const float *xp = xt + (lane + kWave * i) * kPer;
                    const u32x4 v = w[j][i];
                    if constexpr (DT == RBT_DT_BF16) {
                        const f32x4 x0 = *reinterpret_cast<const f32x4 *>(xp), x1 = *reinterpret_cast<const f32x4 *>(xp + 4);
                        acc += bf16_lo(v.x) * x0.x + bf16_hi(v.x) * x0.y + bf16_lo(v.y) * x0.z + bf16_hi(v.y) * x0.w +
                               bf16_lo(v.z) * x1.x + bf16_hi(v.z) * x1.y + bf16_lo(v.w) * x1.z + bf16_hi(v.w) * x1.w;
                    } else {
                        const f32x4 x0 = *reinterpret_cast<const f32x4 *>(xp);
                        acc += __uint_as_float(v.x) * x0.x + __uint_as_float(v.y) * x0.y +
                               __uint_as_float(v.z) * x0.z + __uint_as_float(v.w) * x0.w;
                    }
                }
                const float sum = wave_sum(acc);  // wave-uniform
                if (lane == tt) res[j] = sum;
            }
        }
        // the chunk's outputs: lane tt writes token b0 + tt's rows (residual reads first, all in flight)
        if (lane < nb) {
            const size_t b = (size_t)(b0 + lane);
            if constexpr (MODE == 1) {
                float old[RPW];
#pragma unroll
                for (int j = 0; j < RPW; ++j) old[j] = resid[b * total_rows + row[j]];
#pragma unroll
                for (int j = 0; j < RPW; ++j)
                    if (r0 + j < total_rows) resid[b * total_rows + row[j]] = old[j] + res[j];
            } else {
#pragma unroll
                for (int j = 0; j < RPW; ++j)
                    if (r0 + j < total_rows) sg.out[seg[j]][b * sg.rows[seg[j]] + row[j]] = res[j];
            }
        }
    }
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// out[b][r] = W[r] . x[b] for B <= 16 * TB token rows on the matrix cores (batched decode: q/k/v, wo,
// lm_head): one block per 16 weight rows (one segment); its NW waves split the row into NW slices of
// WS k-steps of 32. A operand: 16 weight rows x 32 of K, bf16 straight from the weights (exact); B
// operand: the tokens' bf16 hi and lo planes (hi + lo = x to ~16 bits, each product with a bf16 weight
// exact in the f32 accumulator), as matrix-core planes (mfma_plane_index): each operand load of a wave
// is one contiguous 1 KiB tile (at the lm_head shape 78 us, against 134 us for [B][K] rows, whose loads
// touch 16 rows per instruction). A wave issues all of its weight loads and then, per pair of 16-token
// blocks, all of their activation loads before the first MFMA, so a block costs about one memory round
// trip. v_mfma_f32_16x16x32_bf16 per (k-step, 16 tokens, part); the NW slices are added in order
// through LDS. Lane l of a 16 x 16 result holds rows 4 (l / 16) + v, token l % 16.
// MODE 0: segment outputs; 1: resid[b][r] += (one segment). SPLIT: the block takes the one token block
// blockIdx.y (TB = 1) -- for products with few row tiles, so that twice the blocks share the chip and
// each reads half the planes. RT: row tiles of 16 per block (segments whole multiples of 16 RT rows),
// each wave's activation operands serving all of them, so the planes are read once per 16 RT weight
// rows; every row tile runs the same MFMA sequence and slice order as with RT = 1 (bit-identical).
template <int KS>
struct MfmaShape {
    static constexpr int NW = KS >= 4 ? 16 : 4 * KS;  // waves per block
    static constexpr int WS = 4 * KS / NW;             // k-steps per wave (1..4)
};
template <int KS, int TB, int MODE, bool SPLIT = false, int RT = 1>
__global__ __launch_bounds__(1024) void dense_mfma_kernel(const uint16_t *__restrict__ x_hi,
                                                          const uint16_t *__restrict__ x_lo, int B, Segs sg,
                                                          int total_rows, float *__restrict__ resid) {
    constexpr int K = 128 * KS, NW = MfmaShape<KS>::NW, WS = MfmaShape<KS>::WS;
    static_assert(WS >= 1 && WS <= 4 && NW * WS * 32 == K, "k split");
    static_assert(!SPLIT || TB == 1, "one token block per block");
    static_assert(RT == 1 || (MODE == 0 && !SPLIT), "several row tiles: segment outputs only");
    __shared__ f32x4 part[NW][RT][TB][kWave];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int row0 = blockIdx.x * 16 * RT;
    const int tbase = SPLIT ? (int)blockIdx.y : 0;  // this block's first token block
    const int tbt = (B + 15) / 16;                   // token blocks of the planes
    int s = 0, r = row0;  // the tile's segment and first row in it (segments are whole tiles)
    while (s < 2 && r >= sg.rows[s]) {
        r -= sg.rows[s];
        ++s;
    }
    u32x4 a[RT][WS];
    if constexpr (WS % 2 == 0) {
        // pairs of k-steps as whole 128-byte lines per load, shuffled into operands (blob_operands)
        const uint8_t *wp = sg.W[s] + ((size_t)(r + (lane & 7)) * K + (size_t)w * WS * 32) * 2 + 16 * blob_chunk(lane);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int i = 0; i < WS; ++i)
                a[rt][i] = ld_stream_u4(wp + (size_t)rt * 16 * K * 2 + (size_t)(i & 1) * 8 * K * 2 + 128 * (i >> 1));
    } else {
        const size_t koff = (size_t)w * WS * 32 + 8 * (lane >> 4);
        const uint8_t *wp = sg.W[s] + ((size_t)(r + (lane & 15)) * K + koff) * 2;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int i = 0; i < WS; ++i) a[rt][i] = ld_stream_u4(wp + (size_t)rt * 16 * K * 2 + 64 * i);
    }
    f32x4 acc[RT][TB];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc[rt][tb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int tb0 = 0; tb0 < TB; tb0 += 2) {
        constexpr int NBMAX = TB < 2 ? TB : 2;
        u32x4 bh[WS][NBMAX], bl[WS][NBMAX];
#pragma unroll
        for (int j = 0; j < NBMAX; ++j) {
            if (tb0 + j < TB) {
#pragma unroll
                for (int i = 0; i < WS; ++i) {
                    const size_t o = (((size_t)(w * WS + i) * tbt + (tbase + tb0 + j)) * kWave + lane) * 8;
                    bh[i][j] = *reinterpret_cast<const u32x4 *>(x_hi + o);
                    bl[i][j] = *reinterpret_cast<const u32x4 *>(x_lo + o);
                }
            }
        }
        // every load out before the first MFMA (the scheduler would otherwise reuse registers and
        // serialise round trips)
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (WS % 2 == 0) {
            if (tb0 == 0) {
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                    for (int i = 0; i < WS; i += 2) blob_operands(a[rt][i], a[rt][i + 1]);
            }
        }
#pragma unroll
        for (int i = 0; i < WS; ++i) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const bf16x8_t av = __builtin_bit_cast(bf16x8_t, a[rt][i]);
#pragma unroll
                for (int j = 0; j < NBMAX; ++j) {
                    if (tb0 + j < TB) {
                        acc[rt][tb0 + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            av, __builtin_bit_cast(bf16x8_t, bh[i][j]), acc[rt][tb0 + j], 0, 0, 0);
                        acc[rt][tb0 + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            av, __builtin_bit_cast(bf16x8_t, bl[i][j]), acc[rt][tb0 + j], 0, 0, 0);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) part[w][rt][tb][lane] = acc[rt][tb];
    __syncthreads();
    // one output element per thread: (row tile rt, block tb, lane l, element j) summed over the NW
    // slices in order
    const float *pf = reinterpret_cast<const float *>(part);
    for (int e = threadIdx.x; e < RT * TB * kWave * 4; e += blockDim.x) {
        float v[NW];
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) v[ww] = pf[(size_t)ww * RT * TB * kWave * 4 + e];
        float sum = v[0];
#pragma unroll
        for (int ww = 1; ww < NW; ++ww) sum = sum + v[ww];
        const int rt = e / (TB * kWave * 4), tb = (e / (kWave * 4)) % TB, l = (e / 4) % kWave, j = e % 4;
        const int t = 16 * (tbase + tb) + (l & 15), rr = 16 * rt + 4 * (l >> 4) + j;
        if (t >= B) continue;
        if constexpr (MODE == 1) {
            float *dst = resid + (size_t)t * total_rows + row0 + rr;
            *dst = *dst + sum;
        } else {
            sg.out[s][(size_t)t * sg.rows[s] + r + rr] = sum;
        }
    }
}

// Greedy argmax over the lm_head blocks' candidates (value, first index; index -1 = none), then the step
// advances like argmax_kernel: the engine's scan keeps index 0 when logits[0] is NaN or nothing beats it.
__global__ __launch_bounds__(1024) void argmax_cand_kernel(const float2 *__restrict__ cand, int nc,
                                                           const float *__restrict__ logits, StepState *st,
                                                           int32_t *__restrict__ seq, int ctx) {
    __shared__ float s_b[16];
    __shared__ int s_i[16];
    // thread 0's step-state and first-logit loads go out with the candidates, not after the reduction
    const float v0 = threadIdx.x == 0 ? logits[0] : 0.0f;
    const int p = threadIdx.x == 0 ? st->pos : 0, n_prompt = threadIdx.x == 0 ? st->n_prompt : 0;
    float b = -INFINITY;
    int k = -1;
    // eight candidates per thread in flight at a time (indices clamped; a repeated candidate changes
    // nothing: the comparison keeps the first of equal values and an equal index is not lower)
    constexpr int kU = 8;
    for (int q0 = threadIdx.x; q0 < nc; q0 += kU * blockDim.x) {
        float2 c[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) c[u] = cand[min(q0 + u * (int)blockDim.x, nc - 1)];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int ci = __float_as_int(c[u].y);
            if (ci >= 0 && (k < 0 || c[u].x > b || (c[u].x == b && ci < k))) {
                b = c[u].x;
                k = ci;
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ob = __shfl_down(b, off, 64);
        const int ok = __shfl_down(k, off, 64);
        if (ok >= 0 && (k < 0 || ob > b || (ob == b && ok < k))) {
            b = ob;
            k = ok;
        }
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (lane == 0) {
        s_b[wv] = b;
        s_i[wv] = k;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        b = -INFINITY;
        k = -1;
        for (int q = 0; q < (int)(blockDim.x >> 6); ++q)
            if (s_i[q] >= 0 && (k < 0 || s_b[q] > b || (s_b[q] == b && s_i[q] < k))) {
                b = s_b[q];
                k = s_i[q];
            }
        if (k < 0 || v0 != v0) k = 0;
        st->last = k;
        if (p + 1 < ctx && p + 1 >= n_prompt) seq[p + 1] = k;
        st->pos = p + 1;
    }
}

// ---------------------------------------------------------------- attention, split over positions
// grid (n_heads, S, B). Block (h, s, b): QK-norm over the whole q and k projections (rabbit2.c:475-478),
// RoPE of head h's q and of its kv head's k at pos (:479-480) from the [ctx][hd/2] (cos, sin) table, then
// the positions t of its share of [0, pos]: scores q.k_t / sqrt(hd) (:486-492), and per wave an online
// softmax (running max m, l = sum exp(score - m), o = sum exp(score - m) v_t) over its positions, the
// K and V rows of KG positions in flight at once. The four waves merge into the block's partial
// (m, l, o), which attn_merge_kernel merges across the S splits (:493-498). The current position's k
// and v come from LDS; block (h, 0) of the first query head of each kv head appends them to the cache
// (:482-484).
// Latency: after pos, every global load the block needs before its first scores (the norm inputs,
// the head's q/k/v and norm weights, its RoPE entries, the first round of cached K/V rows) is issued
// before any of them is used, and each later round's K/V rows are loaded during the previous round's
// arithmetic.
// AE = elements of a head row per lane (head_dim <= 64 AE).
constexpr int kAttnMaxE = 4;  // head_dim <= 256
constexpr int kAttnKG = 8;    // positions per wave per round
constexpr int kAttnNU = 8;    // norm inputs per thread held in registers (q/k dims up to 2048 in one pass)

template <int AE>
__device__ __forceinline__ void attn_load_round(float (&kr)[kAttnKG][AE], float (&vr)[kAttnKG][AE],
                                                const float *__restrict__ kc, const float *__restrict__ vc, int tb,
                                                int t1, int kv_dim, int kvh, int hd, int lane) {
#pragma unroll
    for (int g = 0; g < kAttnKG; ++g) {
        const int t = min(tb + g, t1 - 1);  // past the share: a repeat of the last row, weight 0 below
        const float *kt = kc + (size_t)t * kv_dim + (size_t)kvh * hd, *vt = vc + (size_t)t * kv_dim + (size_t)kvh * hd;
#pragma unroll
        for (int e = 0; e < AE; ++e) {
            const int i = lane + kWave * e;
            kr[g][e] = i < hd ? __builtin_nontemporal_load(kt + i) : 0.0f;
            vr[g][e] = i < hd ? __builtin_nontemporal_load(vt + i) : 0.0f;
        }
    }
}

// hd = 128 (AE = 0): a wave takes 8 positions per round, 8 lanes per position. Lane (g, j) = (l / 8,
// l % 8) holds the 16 elements 32 i + 4 j + c (i, c < 4) of row g, so each of a row's four 16-byte
// loads covers whole 128-byte lines, a score is 16 products and a 3-step sum over the lane's group, and
// each group runs its own online softmax over the positions tb + g of the wave's rounds: two exps per
// round instead of nine (the layout with a row spread over the wave spent ~590 VALU instructions per
// 8-position round and stalled at 5.5 TB/s on its arithmetic). The 32 (wave, group) partials of a
// block merge at its end through LDS.
constexpr int kAttnG8Hd = 128;
constexpr int kAttnG8Pos = 8;  // positions per wave-round
static_assert(kAttnG8Pos == kAttnKG, "the first round's prefetch is shared by both layouts");
__device__ __forceinline__ float group8_sum(float v) {  // sum over the lane's aligned group of 8
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    return v + dpp_f<kDppHalfMirror>(v);
}
__device__ __forceinline__ void attn_g8_load(f32x4 (&kr)[4], f32x4 (&vr)[4], const float *kc, const float *vc, int t,
                                             int kv_dim, int kvh, int j) {
    const size_t o = (size_t)t * kv_dim + (size_t)kvh * kAttnG8Hd + 4 * j;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        kr[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(kc + o + 32 * i));
        vr[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(vc + o + 32 * i));
    }
}

// With one split (S = 1) the block writes the attention output itself: what attn_merge_kernel computes
// for a single partial (weight exp(0) = 1, sum L), into ao [B][q_dim] and, if given, the matrix-core planes.
__device__ __forceinline__ void attn_out_direct(float *ao, uint16_t *ao_hi, uint16_t *ao_lo, int b, int B, int h,
                                                int hd, int q_dim, int i, float acc, float L) {
    const float v = (0.0f + acc) * (1.0f / L);
    ao[(size_t)b * q_dim + (size_t)h * hd + i] = v;
    if (ao_hi) {
        const size_t oi = mfma_plane_index(b, h * hd + i, (B + 15) / 16);
        const uint32_t hb = f32_to_bf16_rne(v);
        ao_hi[oi] = (uint16_t)hb;
        ao_lo[oi] = (uint16_t)f32_to_bf16_rne(v - __uint_as_float(hb << 16));
    }
}

template <int AE>
__global__ __launch_bounds__(256) void attn_kernel(const float *__restrict__ q_raw, const float *__restrict__ k_raw,
                                                   const float *__restrict__ v_raw, const float *__restrict__ qw,
                                                   const float *__restrict__ kw, int qk_norm, float eps, int n_heads,
                                                   int n_kv, int hd, int S, const StepState *__restrict__ st,
                                                   float *__restrict__ kc, float *__restrict__ vc, size_t seq_stride,
                                                   const float2 *__restrict__ rope_cs, float *__restrict__ part,
                                                   float *__restrict__ ao, uint16_t *__restrict__ ao_hi,
                                                   uint16_t *__restrict__ ao_lo) {
    __shared__ __align__(16) float qh[256], kh[256], vh[256];
    __shared__ float red[16], w_m[4], w_l[4];
    __shared__ __align__(16) float w_o[4][256];
    const int h = blockIdx.x, s = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int group = n_heads / n_kv, kvh = h / group;
    const int q_dim = n_heads * hd, kv_dim = n_kv * hd, half = hd / 2;
    // sequence b: its q/k/v rows, KV cache and partials
    q_raw += (size_t)b * q_dim;
    k_raw += (size_t)b * kv_dim;
    v_raw += (size_t)b * kv_dim;
    kc += (size_t)b * seq_stride;
    vc += (size_t)b * seq_stride;
    part += (size_t)b * n_heads * S * (hd + 2);
    const int pos = st[b].pos;

    // ---- loads: norm inputs and this thread's element of the head (independent of pos) ...
    float qa[kAttnNU], ka[kAttnNU];
#pragma unroll
    for (int u = 0; u < kAttnNU; ++u) {
        const int i = tid + 256 * u;
        qa[u] = qk_norm && i < q_dim ? q_raw[i] : 0.0f;
        ka[u] = qk_norm && i < kv_dim ? k_raw[i] : 0.0f;
    }
    float qv = 0.0f, qwv = 0.0f, kv = 0.0f, kwv = 0.0f, vv = 0.0f;
    if (tid < hd) {
        const int qi = h * hd + tid, ki = kvh * hd + tid;
        qv = q_raw[qi];
        kv = k_raw[ki];
        vv = v_raw[ki];
        if (qk_norm) {
            qwv = qw[qi];
            kwv = kw[ki];
        }
    }
    // ... then its RoPE entry and the first round of cached rows (pos is known by now)
    const float2 cs = tid < half ? rope_cs[(size_t)pos * half + tid] : make_float2(0.0f, 0.0f);
    const int n = pos + 1;
    const int chunk = (n + S - 1) / S;
    const int t0 = min(n, s * chunk), t1 = min(n, t0 + chunk);
    constexpr int AEr = AE > 0 ? AE : 1;
    float kr[kAttnKG][AEr], vr[kAttnKG][AEr];
    f32x4 kg[4], vg[4];  // AE = 0: the first round's rows
    const int tb0 = t0 + wv * kAttnKG;  // kAttnKG == kAttnG8Pos
    if constexpr (AE == 0) {
        if (tb0 < t1) attn_g8_load(kg, vg, kc, vc, min(tb0 + (lane >> 3), t1 - 1), kv_dim, kvh, lane & 7);
    } else {
        if (tb0 < t1) attn_load_round(kr, vr, kc, vc, tb0, t1, kv_dim, kvh, hd, lane);
    }

    // ---- QK-norm: both sums of squares in one reduction (per thread in i = tid, tid + 256, ... order)
    float inv_q = 1.0f, inv_k = 1.0f;
    if (qk_norm) {
        float sq = 0.0f, sk = 0.0f;
#pragma unroll
        for (int u = 0; u < kAttnNU; ++u) {
            sq += qa[u] * qa[u];
            sk += ka[u] * ka[u];
        }
        for (int i = tid + 256 * kAttnNU; i < q_dim; i += blockDim.x) sq += q_raw[i] * q_raw[i];
        for (int i = tid + 256 * kAttnNU; i < kv_dim; i += blockDim.x) sk += k_raw[i] * k_raw[i];
        sq = wave_sum(sq);
        sk = wave_sum(sk);
        if (lane == 0) {
            red[wv] = sq;
            red[8 + wv] = sk;
        }
        __syncthreads();
        sq = (red[0] + red[1]) + (red[2] + red[3]);
        sk = (red[8] + red[9]) + (red[10] + red[11]);
        inv_q = 1.0f / sqrtf(sq / (float)q_dim + eps);
        inv_k = 1.0f / sqrtf(sk / (float)kv_dim + eps);
    }
    if (tid < hd) {
        qh[tid] = qk_norm ? qv * inv_q * qwv : qv;
        kh[tid] = qk_norm ? kv * inv_k * kwv : kv;
        vh[tid] = vv;
    }
    __syncthreads();
    if (tid < half) {
#pragma clang fp contract(off)
        float a = qh[tid], c = qh[tid + half];
        qh[tid] = a * cs.x - c * cs.y;
        qh[tid + half] = c * cs.x + a * cs.y;
        a = kh[tid];
        c = kh[tid + half];
        kh[tid] = a * cs.x - c * cs.y;
        kh[tid + half] = c * cs.x + a * cs.y;
    }
    __syncthreads();
    if (s == 0 && h % group == 0) {
        float *kd = kc + (size_t)pos * kv_dim + (size_t)kvh * hd, *vd = vc + (size_t)pos * kv_dim + (size_t)kvh * hd;
        for (int i = tid; i < hd; i += blockDim.x) {
            kd[i] = kh[i];
            vd[i] = vh[i];
        }
    }
    const float scale = 1.0f / sqrtf((float)hd);
    if constexpr (AE == 0) {
        const int g = lane >> 3, j = lane & 7;
        f32x4 q4[4], o4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q4[i] = *reinterpret_cast<const f32x4 *>(qh + 32 * i + 4 * j);
            o4[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        float m = -INFINITY, l = 0.0f;
        auto step = [&](f32x4 (&kr4)[4], f32x4 (&vr4)[4], int tb) {
            const int t = tb + g;
            if (min(t, t1 - 1) == pos) {  // the current position: from LDS, not the cache
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    kr4[i] = *reinterpret_cast<const f32x4 *>(kh + 32 * i + 4 * j);
                    vr4[i] = *reinterpret_cast<const f32x4 *>(vh + 32 * i + 4 * j);
                }
            }
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                d += (q4[i].x * kr4[i].x + q4[i].y * kr4[i].y) + (q4[i].z * kr4[i].z + q4[i].w * kr4[i].w);
            d = group8_sum(d);
            const float sc = t < t1 ? d * scale : -INFINITY;  // rows past the share: a repeat, weight 0
            const float mn = fmaxf(m, sc);
            const float mref = mn == -INFINITY ? 0.0f : mn;  // no position yet: alpha = p = 0
            const float alpha = expf(m - mref), p = expf(sc - mref);
            l = l * alpha + p;
#pragma unroll
            for (int i = 0; i < 4; ++i) o4[i] = o4[i] * alpha + p * vr4[i];
            m = mn;
        };
        // wave-uniform rounds 4 * kAttnG8Pos positions apart, two per iteration (ping-pong buffers), the
        // next round's rows in flight during each round's arithmetic
        f32x4 kb[4], vb[4];
        for (int tb = tb0; tb < t1; tb += 8 * kAttnG8Pos) {
            const int tn = tb + 4 * kAttnG8Pos;
            if (tn < t1) attn_g8_load(kb, vb, kc, vc, min(tn + g, t1 - 1), kv_dim, kvh, j);
            step(kg, vg, tb);
            if (tn >= t1) break;
            const int tn2 = tn + 4 * kAttnG8Pos;
            if (tn2 < t1) attn_g8_load(kg, vg, kc, vc, min(tn2 + g, t1 - 1), kv_dim, kvh, j);
            step(kb, vb, tn);
        }
        // merge the 32 (wave, group) partials: scales by wave 0, then one element per thread
        __shared__ float g_m[32], g_l[32], g_a[32], g_L;
        __shared__ __align__(16) float g_o[32][kAttnG8Hd];
        const int src = wv * 8 + g;
        if (j == 0) {
            g_m[src] = m;
            g_l[src] = l;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<f32x4 *>(&g_o[src][32 * i + 4 * j]) = o4[i];
        __syncthreads();
        float *po = part + ((size_t)h * S + s) * (hd + 2);
        if (wv == 0) {
            const float ms = lane < 32 ? g_m[lane] : -INFINITY, ls = lane < 32 ? g_l[lane] : 0.0f;
            const float M = wave_max(ms);
            const float a = ls > 0.0f ? expf(ms - M) : 0.0f;
            if (lane < 32) g_a[lane] = a;
            const float L = wave_sum(a * ls);
            if (lane == 0) {
                g_L = L;
                if (!ao) {
                    po[0] = M;
                    po[1] = L;
                }
            }
        }
        __syncthreads();
        if (tid < kAttnG8Hd) {
            float acc = 0.0f;
#pragma unroll 8
            for (int q2 = 0; q2 < 32; ++q2) acc += g_a[q2] * g_o[q2][tid];
            if (ao)
                attn_out_direct(ao, ao_hi, ao_lo, b, gridDim.z, h, hd, n_heads * hd, tid, acc, g_L);
            else
                po[2 + tid] = acc;
        }
        return;
    }
    float q[AEr], o[AEr];
#pragma unroll
    for (int e = 0; e < AE; ++e) {
        const int i = lane + kWave * e;
        q[e] = i < hd ? qh[i] : 0.0f;
        o[e] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    for (int tb = tb0; tb < t1; tb += 4 * kAttnKG) {  // wave-uniform rounds
#pragma unroll
        for (int g = 0; g < kAttnKG; ++g) {
            if (min(tb + g, t1 - 1) == pos) {  // the current position: from LDS, not the cache
#pragma unroll
                for (int e = 0; e < AE; ++e) {
                    const int i = lane + kWave * e;
                    kr[g][e] = i < hd ? kh[i] : 0.0f;
                    vr[g][e] = i < hd ? vh[i] : 0.0f;
                }
            }
        }
        float kn[kAttnKG][AEr], vn[kAttnKG][AEr];
        const int tn = tb + 4 * kAttnKG;
        if (tn < t1) attn_load_round(kn, vn, kc, vc, tn, t1, kv_dim, kvh, hd, lane);  // the next round, in flight
        float sc[kAttnKG];
#pragma unroll
        for (int g = 0; g < kAttnKG; ++g) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < AE; ++e) d += q[e] * kr[g][e];
            sc[g] = tb + g < t1 ? wave_sum(d) * scale : -INFINITY;
        }
        float mn = m;
#pragma unroll
        for (int g = 0; g < kAttnKG; ++g) mn = fmaxf(mn, sc[g]);
        const float alpha = expf(m - mn);  // m = -inf on the first round: alpha 0
        l *= alpha;
#pragma unroll
        for (int e = 0; e < AE; ++e) o[e] *= alpha;
#pragma unroll
        for (int g = 0; g < kAttnKG; ++g) {
            const float p = expf(sc[g] - mn);  // positions past the share: exp(-inf) = 0
            l += p;
#pragma unroll
            for (int e = 0; e < AE; ++e) o[e] += p * vr[g][e];
        }
        m = mn;
        if (tn < t1) {
#pragma unroll
            for (int g = 0; g < kAttnKG; ++g)
#pragma unroll
                for (int e = 0; e < AE; ++e) {
                    kr[g][e] = kn[g][e];
                    vr[g][e] = vn[g][e];
                }
        }
    }
    // merge the four waves
    if (lane == 0) {
        w_m[wv] = m;
        w_l[wv] = l;
    }
#pragma unroll
    for (int e = 0; e < AE; ++e) {
        const int i = lane + kWave * e;
        if (i < hd) w_o[wv][i] = o[e];
    }
    __syncthreads();
    float *po = part + ((size_t)h * S + s) * (hd + 2);
    const float M = fmaxf(fmaxf(w_m[0], w_m[1]), fmaxf(w_m[2], w_m[3]));
    float sw[4];
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        sw[w] = w_l[w] > 0.0f ? expf(w_m[w] - M) : 0.0f;
        L += sw[w] * w_l[w];
    }
    for (int i = tid; i < hd; i += blockDim.x) {
        const float acc = ((sw[0] * w_o[0][i] + sw[1] * w_o[1][i]) + (sw[2] * w_o[2][i] + sw[3] * w_o[3][i]));
        if (ao)
            attn_out_direct(ao, ao_hi, ao_lo, b, gridDim.z, h, hd, n_heads * hd, i, acc, L);
        else
            po[2 + i] = acc;
    }
    if (tid == 0 && !ao) {
        po[0] = M;
        po[1] = L;
    }
}

// attn_out[h*hd + i] = sum_s a_s o_s[i] / sum_s a_s l_s with a_s = exp(m_s - max m): block h merges the
// S split partials of head h (the engine's softmax-weighted sum over all positions, rabbit2.c:493-498).
__global__ __launch_bounds__(256) void attn_merge_kernel(const float *__restrict__ part, int hd, int S,
                                                         float *__restrict__ ao, uint16_t *__restrict__ ao_hi,
                                                         uint16_t *__restrict__ ao_lo) {
    __shared__ float wa[64], s_inv;
    const int h = blockIdx.x, b = blockIdx.y, n_heads = gridDim.x;
    const float *ph = part + ((size_t)b * n_heads + h) * S * (hd + 2);
    ao += (size_t)b * n_heads * hd;
    // loads first: this thread's element of splits 0..15 (clamped indices, no branches) and wave 0's
    // (m, l) of split q = lane
    const int ie = min((int)threadIdx.x, hd - 1);
    float ov[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) ov[q] = ph[(size_t)min(q, S - 1) * (hd + 2) + 2 + ie];
    const int qc = min((int)threadIdx.x & 63, S - 1);
    const float pm = ph[(size_t)qc * (hd + 2)], pl = ph[(size_t)qc * (hd + 2) + 1];
    if (threadIdx.x < 64) {  // S <= 64 split weights, by wave 0
        const int q = threadIdx.x;
        const float m = q < S ? pm : -INFINITY;
        const float l = q < S ? pl : 0.0f;
        const float M = wave_max(m);
        const float a = l > 0.0f ? expf(m - M) : 0.0f;
        wa[q] = a;
        const float L = wave_sum(a * l);
        if (q == 0) s_inv = 1.0f / L;
    }
    __syncthreads();
    const int i = threadIdx.x;  // hd <= blockDim.x
    if (i < hd) {
        float o = 0.0f;
#pragma unroll
        for (int q = 0; q < 16; ++q)
            if (q < S) o += wa[q] * ov[q];
        for (int q = 16; q < S; ++q) o += wa[q] * ph[(size_t)q * (hd + 2) + 2 + i];
        const float v = o * s_inv;
        const size_t oi = mfma_plane_index(b, h * hd + i, (gridDim.y + 15) / 16);
        ao[(size_t)h * hd + i] = v;
        if (ao_hi) {
            const uint32_t hb = f32_to_bf16_rne(v);
            ao_hi[oi] = (uint16_t)hb;
            ao_lo[oi] = (uint16_t)f32_to_bf16_rne(v - __uint_as_float(hb << 16));
        }
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
                                                       float eps, float *__restrict__ out, uint16_t *__restrict__ hi,
                                                       uint16_t *__restrict__ lo) {
    __shared__ float red[16];
    x += (size_t)blockIdx.x * n;  // one row per block
    out += (size_t)blockIdx.x * n;
    const int tbs = (gridDim.x + 15) / 16;  // token blocks of the planes
    auto put = [&](int i, float v) {
        out[i] = v;
        if (hi) {
            const size_t pi = mfma_plane_index(blockIdx.x, i, tbs);
            const uint32_t h = f32_to_bf16_rne(v);
            hi[pi] = (uint16_t)h;
            lo[pi] = (uint16_t)f32_to_bf16_rne(v - __uint_as_float(h << 16));
        }
    };
    // rows of up to 4 * 1024 elements from registers (x and w loaded together), longer ones by the loop
    constexpr int U = 4;
    float xr[U], wr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = min((int)threadIdx.x + 1024 * u, n - 1);
        xr[u] = x[i];
        wr[u] = w[i];
    }
    float ss = 0.0f;  // rms_inv's per-thread order
#pragma unroll
    for (int u = 0; u < U; ++u)
        if ((int)threadIdx.x + 1024 * u < n) ss += xr[u] * xr[u];
    for (int i = threadIdx.x + 1024 * U; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = threadIdx.x + 1024 * u;
        if (i < n) put(i, xr[u] * inv * wr[u]);
    }
    for (int i = threadIdx.x + 1024 * U; i < n; i += blockDim.x) put(i, x[i] * inv * w[i]);
}

// The grouped path's combine for token t (combine_rows_kernel's arithmetic: moe = sum_k w_k y[pos(t,k)]
// in selection order with rounded products, x += moe, rabbit2.c:540-542) followed by rmsnorm_kernel on
// the new row (same per-thread order and block sum, same planes): one block per token, n <= 4096, K <= 8.
__global__ __launch_bounds__(1024) void combine_rmsnorm_kernel(const float *__restrict__ y,
                                                               const int32_t *__restrict__ pos_of,
                                                               const float *__restrict__ weights, int K, int n,
                                                               float *__restrict__ x, const float *__restrict__ w,
                                                               float eps, float *__restrict__ out,
                                                               uint16_t *__restrict__ hi, uint16_t *__restrict__ lo) {
    __shared__ float red[16];
    const int t = blockIdx.x;
    x += (size_t)t * n;
    out += (size_t)t * n;
    const int tbs = (gridDim.x + 15) / 16;
    int p[8];
    float wk[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int kc = min(k, K - 1);
        p[k] = pos_of[t * K + kc];
        wk[k] = weights[t * K + kc];
    }
    constexpr int U = 4;
    float xr[U], wr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = min((int)threadIdx.x + 1024 * u, n - 1);
        float tmp[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) tmp[k] = y[(size_t)p[k] * n + i];
        float moe = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
#pragma clang fp contract(off)
            if (k < K) moe = moe + wk[k] * tmp[k];
        }
        xr[u] = x[i] + moe;
        wr[u] = w[i];
    }
    float ss = 0.0f;  // rmsnorm_kernel's per-thread order
#pragma unroll
    for (int u = 0; u < U; ++u)
        if ((int)threadIdx.x + 1024 * u < n) ss += xr[u] * xr[u];
    ss = block_sum(ss, red);  // its first barrier also orders every read of x before the stores below
#pragma unroll
    for (int u = 0; u < U; ++u)
        if ((int)threadIdx.x + 1024 * u < n) x[threadIdx.x + 1024 * u] = xr[u];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = threadIdx.x + 1024 * u;
        if (i >= n) continue;
        const float v = xr[u] * inv * wr[u];
        out[i] = v;
        if (hi) {
            const size_t pi = mfma_plane_index(t, i, tbs);
            const uint32_t h = f32_to_bf16_rne(v);
            hi[pi] = (uint16_t)h;
            lo[pi] = (uint16_t)f32_to_bf16_rne(v - __uint_as_float(h << 16));
        }
    }
}

// ---------------------------------------------------------------- greedy argmax (rabbit2.c:552-556)
// best = 0; for i: if v[i] > v[best] best = i -- the first index of the largest value; a NaN never
// wins, and a NaN at index 0 is never beaten. Then the step advances: seq[pos + 1] = best when that
// slot is past the prompt (generation), pos += 1.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ v, int n, StepState *st,
                                                      int32_t *__restrict__ seq, int ctx) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    v += (size_t)blockIdx.x * n;  // one sequence per block
    st += blockIdx.x;
    seq += (size_t)blockIdx.x * ctx;
    float best = -INFINITY;
    int idx = n;  // n: nothing found yet
    auto visit = [&](float a, int i) {
        if (a == a && (idx == n || a > best)) {  // first non-NaN, then strictly larger
            best = a;
            idx = i;
        }
    };
    // each thread visits its indices in ascending order: 16-byte chunks c = tid, tid + 1024, ... (four
    // in flight per round, indices clamped), then the tail past the last whole chunk
    const int n4 = (n % 4 == 0) ? n / 4 : 0;
    const f32x4 *v4 = reinterpret_cast<const f32x4 *>(v);
    for (int c0 = threadIdx.x; c0 < n4; c0 += 4 * 1024) {
        f32x4 a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = v4[min(c0 + 1024 * j, n4 - 1)];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = c0 + 1024 * j;
            if (c < n4) {
                visit(a[j].x, 4 * c);
                visit(a[j].y, 4 * c + 1);
                visit(a[j].z, 4 * c + 2);
                visit(a[j].w, 4 * c + 3);
            }
        }
    }
    for (int i = 4 * n4 + threadIdx.x; i < n; i += blockDim.x) visit(v[i], i);
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

// ---------------------------------------------------------------- sampler (rabbit2.c:558-610)
// sample_logits for one sequence per block, in the engine's operations and orders: prob = logits / T
// (idx = i); with 0 < top_k < n, K rounds that each swap the largest remaining value (first position on
// ties, in the current order) to the front; max, expf(v - max) over the finite values summed in index
// order, divide; top-p over the first m (K, or n) entries in that order; then the first position whose
// running double sum passes the xorshift64* draw. The K rounds and elementwise steps run across the
// block; every sum, whose order fixes its rounding, runs in one thread like the engine's loops.
__device__ __forceinline__ uint64_t rng_next_dev(uint64_t *s) {
    uint64_t x = *s ? *s : 0x9E3779B97F4A7C15ull;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *s = x;
    return x * 2685821657736338717ull;
}

// first position of the largest value among prob[from..n) (a NaN never wins; -1 if all NaN)
__device__ __forceinline__ int block_first_max(const float *prob, int from, int n, float *s_b, int *s_i) {
    float b = 0.0f;
    int k = -1;
    for (int i = from + threadIdx.x; i < n; i += blockDim.x) {
        const float v = prob[i];
        if (v == v && (k < 0 || v > b)) {
            b = v;
            k = i;
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ob = __shfl_down(b, off, 64);
        const int ok = __shfl_down(k, off, 64);
        if (ok >= 0 && (k < 0 || ob > b || (ob == b && ok < k))) {
            b = ob;
            k = ok;
        }
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    __syncthreads();  // s_b / s_i are free
    if (lane == 0) {
        s_b[wv] = b;
        s_i[wv] = k;
    }
    __syncthreads();
    b = 0.0f;
    k = -1;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w)
        if (s_i[w] >= 0 && (k < 0 || s_b[w] > b || (s_b[w] == b && s_i[w] < k))) {
            b = s_b[w];
            k = s_i[w];
        }
    return k;
}

__global__ __launch_bounds__(1024) void sample_kernel(const float *__restrict__ logits, int n, Sampling sp,
                                                      float *__restrict__ prob, int32_t *__restrict__ idx,
                                                      StepState *st, int32_t *__restrict__ seq, int ctx) {
    __shared__ float s_b[16];
    __shared__ int s_i[16];
    __shared__ int s_res;
    const int b = blockIdx.x;
    logits += (size_t)b * n;
    prob += (size_t)b * n;
    idx += (size_t)b * n;
    st += b;
    seq += (size_t)b * ctx;
    const int tid = threadIdx.x;
    for (int i = tid; i < n; i += blockDim.x) {
        idx[i] = i;
        prob[i] = logits[i] / sp.temperature;
    }
    const bool use_k = sp.top_k > 0 && sp.top_k < n;
    if (use_k) {
        for (int r = 0; r < sp.top_k; ++r) {
            __syncthreads();  // the previous swap (and the fill) are visible
            int best = block_first_max(prob, r, n, s_b, s_i);
            const float pr = prob[r];
            // the engine's scan starts from position r: a NaN there is never beaten, and nothing beats it
            // when every value is NaN
            if (best < 0 || pr != pr) best = r;
            if (tid == 0 && best != r) {
                const float tp = prob[r];
                prob[r] = prob[best];
                prob[best] = tp;
                const int32_t ti = idx[r];
                idx[r] = idx[best];
                idx[best] = ti;
            }
        }
    }
    __syncthreads();
    const int m = use_k ? sp.top_k : n;  // positions past m are -inf under top-k
    if (tid == 0) {
        int res = -1;
        float mx = -INFINITY;
        for (int i = 0; i < m; ++i)
            if (prob[i] > mx) mx = prob[i];
        float sum = 0.0f;
        for (int i = 0; i < m; ++i) {
            const float v = prob[i];
            const float e = isfinite(v) ? expf(v - mx) : 0.0f;
            prob[i] = e;
            sum += e;
        }
        if (!(sum > 0.0f)) {
            res = -2;  // the engine falls back to argmax(logits)
        } else {
            for (int i = 0; i < m; ++i) prob[i] /= sum;
            int keep = m;
            if (sp.top_p > 0.0f && sp.top_p < 1.0f) {
                float cum = 0.0f;
                for (int i = 0; i < m; ++i) {
                    cum += prob[i];
                    if (cum >= sp.top_p) {
                        keep = i + 1;
                        break;
                    }
                }
                float s2 = 0.0f;
                for (int i = 0; i < keep; ++i) s2 += prob[i];  // zeros past keep add nothing
                if (!(s2 > 0.0f)) {
                    res = idx[0];
                } else {
                    for (int i = 0; i < keep; ++i) prob[i] /= s2;
                }
            }
            if (res == -1) {
                uint64_t rng = st->rng;
                const double r = (double)(rng_next_dev(&rng) >> 11) * (1.0 / 9007199254740992.0);
                st->rng = rng;
                double cum = 0.0;
                for (int i = 0; i < keep && res < 0; ++i) {
                    cum += prob[i];
                    if (r < cum) res = idx[i];
                }
                for (int i = keep - 1; i >= 0 && res < 0; --i)
                    if (prob[i] > 0.0f) res = idx[i];
                if (res < 0) res = -2;
            }
        }
        s_res = res;
    }
    __syncthreads();
    int tok = s_res;
    if (tok == -2) {  // argmax(logits): first index of the largest, a NaN at 0 kept (rabbit2.c:552-556)
        tok = block_first_max(logits, 0, n, s_b, s_i);
        const float v0 = logits[0];
        if (tok < 0 || v0 != v0) tok = 0;
    }
    if (tid == 0) {
        const int p = st->pos;
        st->last = tok;
        if (p + 1 < ctx && p + 1 >= st->n_prompt) seq[p + 1] = tok;
        st->pos = p + 1;
    }
}

// advances the step records without an argmax (prompt positions whose logits nobody reads)
__global__ void advance_kernel(StepState *st, int B) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) st[b].pos = st[b].pos + 1;
}

// The step's routing [n_layers][B][K] copied into each sequence's history [B][ctx][n_layers][K] at the
// step's position (before the step advances it). Grid: B blocks of 256 threads.
__global__ __launch_bounds__(256) void record_routing_kernel(const StepState *__restrict__ st,
                                                             const int32_t *__restrict__ routing, int n_layers, int K,
                                                             int B, int ctx, int32_t *__restrict__ hist) {
    const int b = blockIdx.x;
    const int pos = st[b].pos;
    if (pos < 0 || pos >= ctx) return;
    const int per = n_layers * K;
    int32_t *dst = hist + ((size_t)b * ctx + pos) * per;
    for (int i = threadIdx.x; i < per; i += blockDim.x) {
        const int l = i / K, k = i - l * K;
        dst[i] = routing[((size_t)l * B + b) * K + k];
    }
}

inline bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The specialised dense kernel when rows are whole 1 KiB wave-steps (D = 512 * NC bf16 / 256 * NC f32,
// NC in 1..8), else nullopt-like false. mode: 0 norm + matvec, 1 matvec + residual, 2 lm_head + argmax.
bool dense_ok(int dtype, int D, const void *const W[3], const int rows[3]) {
    const int step = dtype == RBT_DT_BF16 ? 512 : 256;
    if (D % step != 0 || D / step < 1 || D / step > 8) return false;
    for (int i = 0; i < 3; ++i)
        if (rows[i] > 0 && !al16(W[i])) return false;
    return true;
}

// Launch shapes (rows per wave RPW, waves per block WPB), measured on the OLMoE shapes: the lm_head
// (50304 rows) streams fastest with 2 rows per wave in 4-wave blocks; q/k/v (6144 rows) and wo (2048
// rows) with one block of 8 waves per CU, 3 and 1 rows per wave.
template <int MODE>
struct DenseShape {
    static constexpr int RPW = MODE == 2 ? 2 : MODE == 0 ? 3 : 1, WPB = MODE == 2 ? 4 : 8;
};

template <int DT, int MODE>
hipError_t dense_dt(const Launch &L, int D, const float *x, const float *nw, float eps, const Segs &sg, int total,
                    float *resid, float2 *cand) {
    constexpr int step = DT == RBT_DT_BF16 ? 512 : 256;
    constexpr int RPW = DenseShape<MODE>::RPW, WPB = DenseShape<MODE>::WPB;
    const dim3 g((unsigned)((total + RPW * WPB - 1) / (RPW * WPB))), b(64 * WPB);
    switch (D / step) {
#define DENSE_CASE(nc) \
    case nc:           \
        return launch(L, dense_kernel<DT, nc, RPW, MODE, WPB>, g, b, 0, x, nw, eps, sg, total, resid, cand);
        DENSE_CASE(1)
        DENSE_CASE(2)
        DENSE_CASE(3)
        DENSE_CASE(4)
        DENSE_CASE(5)
        DENSE_CASE(6)
        DENSE_CASE(7)
        DENSE_CASE(8)
#undef DENSE_CASE
        default:
            return hipErrorNotSupported;
    }
}

template <int MODE>
hipError_t launch_dense_mode(const Launch &L, int dtype, int D, const float *x, const float *nw, float eps,
                             const Segs &sg, int total, float *resid, float2 *cand) {
    return dtype == RBT_DT_BF16 ? dense_dt<RBT_DT_BF16, MODE>(L, D, x, nw, eps, sg, total, resid, cand)
                                : dense_dt<RBT_DT_F32, MODE>(L, D, x, nw, eps, sg, total, resid, cand);
}
}  // namespace

hipError_t launch_embed(const Launch &L, int dtype, const void *emb, int D, int vocab, const StepState *st,
                        const int32_t *seq, int ctx, float *x, int B) {
    const dim3 g((unsigned)((D + 255) / 256), (unsigned)B), b(256);
    const uint8_t *e = static_cast<const uint8_t *>(emb);
    return dtype == RBT_DT_BF16 ? launch(L, embed_kernel<RBT_DT_BF16>, g, b, 0, e, D, vocab, st, seq, ctx, x)
                                : launch(L, embed_kernel<RBT_DT_F32>, g, b, 0, e, D, vocab, st, seq, ctx, x);
}

template <int DT, int MODE>
hipError_t dense_batch_dt(const Launch &L, int D, const float *xin, int B, const Segs &sg, int total, float *resid) {
    constexpr int step = DT == RBT_DT_BF16 ? 512 : 256;
    constexpr int RPW = 4;
    const dim3 g((unsigned)((total + 4 * RPW - 1) / (4 * RPW))), b(256);
    switch (D / step) {
#define DB_CASE(nc) \
    case nc:        \
        return launch(L, dense_batch_kernel<DT, nc, RPW, MODE>, g, b, 0, xin, B, sg, total, resid);
        DB_CASE(1)
        DB_CASE(2)
        DB_CASE(3)
        DB_CASE(4)
        DB_CASE(5)
        DB_CASE(6)
        DB_CASE(7)
        DB_CASE(8)
#undef DB_CASE
        default:
            return hipErrorNotSupported;
    }
}

bool dense_mfma_supported(int dtype, int B, int K, const void *const W[3], const int rows[3]) {
    if (dtype != RBT_DT_BF16 || B < 1 || B > 64 || K % 128 != 0) return false;
    const int ks = K / 128;
    if (ks != 1 && ks != 2 && ks != 4 && ks != 8 && ks != 16) return false;
    for (int i = 0; i < 3; ++i)
        if (rows[i] % 16 != 0 || (rows[i] && (reinterpret_cast<uintptr_t>(W[i]) & 15u))) return false;
    return true;
}

namespace {
// Row tiles below which a product over two or more token blocks is split by token block: fewer tiles
// than CUs leave CUs idle (wo at 2048 rows, 128 tiles: 7.7 -> 6.6 us at 32 tokens), while more have
// each weight row read twice (q/k/v at 6144 rows, 384 tiles: 14.2 -> 16.6 us when split, 15.5 us even
// with a tile's token blocks placed 8 blocks apart, on one XCD back to back, to share its L2).
constexpr int kMfmaSplitTiles = 256;
template <int KS, int MODE>
hipError_t dense_mfma_ks(const Launch &L, const uint16_t *xh, const uint16_t *xl, int B, const Segs &sg,
                         int total, float *resid) {
    const dim3 g((unsigned)(total / 16)), b(64 * MfmaShape<KS>::NW);
    const int tbt = (B + 15) / 16;
    if (tbt >= 2 && total / 16 < kMfmaSplitTiles)  // few row tiles: a block per (row tile, token block)
        return launch(L, dense_mfma_kernel<KS, 1, MODE, true>, dim3((unsigned)(total / 16), (unsigned)tbt), b, 0, xh, xl,
                      B, sg, total, resid);
    // two row tiles per block where every segment is whole 32-row pairs (the planes read once per 32
    // weight rows)
    if constexpr (MODE == 0) {
        if (tbt <= 2 && sg.rows[0] % 32 == 0 && sg.rows[1] % 32 == 0 && sg.rows[2] % 32 == 0) {
            const dim3 g2((unsigned)(total / 32));
            return tbt == 1 ? launch(L, dense_mfma_kernel<KS, 1, 0, false, 2>, g2, b, 0, xh, xl, B, sg, total, resid)
                            : launch(L, dense_mfma_kernel<KS, 2, 0, false, 2>, g2, b, 0, xh, xl, B, sg, total, resid);
        }
    }
    switch (tbt) {
        case 1: return launch(L, dense_mfma_kernel<KS, 1, MODE>, g, b, 0, xh, xl, B, sg, total, resid);
        case 2: return launch(L, dense_mfma_kernel<KS, 2, MODE>, g, b, 0, xh, xl, B, sg, total, resid);
        case 3: return launch(L, dense_mfma_kernel<KS, 3, MODE>, g, b, 0, xh, xl, B, sg, total, resid);
        case 4: return launch(L, dense_mfma_kernel<KS, 4, MODE>, g, b, 0, xh, xl, B, sg, total, resid);
        default: return hipErrorNotSupported;
    }
}
template <int MODE>
hipError_t dense_mfma_mode(const Launch &L, const uint16_t *xh, const uint16_t *xl, int B, int K,
                           const Segs &sg, int total, float *resid) {
    switch (K / 128) {
        case 1: return dense_mfma_ks<1, MODE>(L, xh, xl, B, sg, total, resid);
        case 2: return dense_mfma_ks<2, MODE>(L, xh, xl, B, sg, total, resid);
        case 4: return dense_mfma_ks<4, MODE>(L, xh, xl, B, sg, total, resid);
        case 8: return dense_mfma_ks<8, MODE>(L, xh, xl, B, sg, total, resid);
        case 16: return dense_mfma_ks<16, MODE>(L, xh, xl, B, sg, total, resid);
        default: return hipErrorNotSupported;
    }
}
}  // namespace

hipError_t launch_dense_mfma(const Launch &L, const uint16_t *x_hi, const uint16_t *x_lo, int B, int K,
                             const void *const W[3], float *const out[3], const int rows[3], float *resid) {
    Segs sg;
    int total = 0;
    for (int i = 0; i < 3; ++i) {
        sg.W[i] = static_cast<const uint8_t *>(W[i]);
        sg.out[i] = out[i];
        sg.rows[i] = rows[i];
        total += rows[i];
    }
    if (total == 0 || B == 0) return hipSuccess;
    if (!dense_mfma_supported(RBT_DT_BF16, B, K, W, rows) || (resid && rows[1] + rows[2] != 0))
        return hipErrorNotSupported;
    return resid ? dense_mfma_mode<1>(L, x_hi, x_lo, B, K, sg, total, resid)
                 : dense_mfma_mode<0>(L, x_hi, x_lo, B, K, sg, total, nullptr);
}

hipError_t launch_dense_batch(const Launch &L, int dtype, const float *xin, int B, int D, const void *const W[3],
                              float *const out[3], const int rows[3], float *resid) {
    Segs sg;
    int total = 0;
    for (int i = 0; i < 3; ++i) {
        sg.W[i] = static_cast<const uint8_t *>(W[i]);
        sg.out[i] = out[i];
        sg.rows[i] = rows[i];
        total += rows[i];
    }
    if (total == 0 || B == 0) return hipSuccess;
    if (resid)
        return dtype == RBT_DT_BF16 ? dense_batch_dt<RBT_DT_BF16, 1>(L, D, xin, B, sg, total, resid)
                                    : dense_batch_dt<RBT_DT_F32, 1>(L, D, xin, B, sg, total, resid);
    return dtype == RBT_DT_BF16 ? dense_batch_dt<RBT_DT_BF16, 0>(L, D, xin, B, sg, total, nullptr)
                                : dense_batch_dt<RBT_DT_F32, 0>(L, D, xin, B, sg, total, nullptr);
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

bool dense_supported(int dtype, int D, const void *const W[3], const int rows[3]) {
    return dense_ok(dtype, D, W, rows);
}

hipError_t launch_dense_norm(const Launch &L, int dtype, const float *x, const float *nw, float eps, int D,
                             const void *const W[3], float *const out[3], const int rows[3]) {
    Segs sg;
    int total = 0;
    for (int i = 0; i < 3; ++i) {
        sg.W[i] = static_cast<const uint8_t *>(W[i]);
        sg.out[i] = out[i];
        sg.rows[i] = rows[i];
        total += rows[i];
    }
    if (total == 0) return hipSuccess;
    return launch_dense_mode<0>(L, dtype, D, x, nw, eps, sg, total, nullptr, nullptr);
}

hipError_t launch_dense_resid(const Launch &L, int dtype, const float *a, int cols, const void *W, int rows,
                              float *x) {
    Segs sg{};
    sg.W[0] = static_cast<const uint8_t *>(W);
    sg.rows[0] = rows;
    return launch_dense_mode<1>(L, dtype, cols, a, nullptr, 0.0f, sg, rows, x, nullptr);
}

int dense_argmax_blocks(int rows) {
    constexpr int per = DenseShape<2>::RPW * DenseShape<2>::WPB;
    return (rows + per - 1) / per;
}

hipError_t launch_dense_argmax(const Launch &L, int dtype, const float *x, const float *nw, float eps, int D,
                               const void *W, int rows, float *logits, float2 *cand, StepState *st, int32_t *seq,
                               int ctx) {
    Segs sg{};
    sg.W[0] = static_cast<const uint8_t *>(W);
    sg.out[0] = logits;
    sg.rows[0] = rows;
    hipError_t e = launch_dense_mode<2>(L, dtype, D, x, nw, eps, sg, rows, nullptr, cand);
    if (e != hipSuccess) return e;
    Launch L2 = L;  // the event pair (if any) brackets the first launch only
    L2.start = L2.stop = nullptr;
    return launch(L2, argmax_cand_kernel, dim3(1), dim3(1024), 0, (const float2 *)cand, dense_argmax_blocks(rows),
                  (const float *)logits, st, seq, ctx);
}

hipError_t launch_attention(const Launch &L, const float *q, const float *k, const float *v, const float *qw,
                            const float *kw, int qk_norm, float eps, int n_heads, int n_kv, int hd, int S,
                            const StepState *st, float *kc, float *vc, size_t seq_stride, const float2 *rope_cs,
                            float *part, int B, float *ao, uint16_t *ao_hi, uint16_t *ao_lo) {
    if (hd > kWave * kAttnMaxE || S > 64) return hipErrorInvalidValue;
    if (ao && (S != 1 || (ao_hi == nullptr) != (ao_lo == nullptr) || (ao_hi && (B > 64 || (n_heads * hd) % 32 != 0))))
        return hipErrorInvalidValue;
    const dim3 g((unsigned)n_heads, (unsigned)S, (unsigned)B), b(256);
    const int kvd = n_kv * hd;
    if (hd == kAttnG8Hd && kvd % 4 == 0 && seq_stride % 4 == 0 && al16(kc) && al16(vc))
        return launch(L, attn_kernel<0>, g, b, 0, q, k, v, qw, kw, qk_norm, eps, n_heads, n_kv, hd, S, st, kc, vc,
                      seq_stride, rope_cs, part, ao, ao_hi, ao_lo);
    if (hd <= kWave)
        return launch(L, attn_kernel<1>, g, b, 0, q, k, v, qw, kw, qk_norm, eps, n_heads, n_kv, hd, S, st, kc, vc,
                      seq_stride, rope_cs, part, ao, ao_hi, ao_lo);
    if (hd <= 2 * kWave)
        return launch(L, attn_kernel<2>, g, b, 0, q, k, v, qw, kw, qk_norm, eps, n_heads, n_kv, hd, S, st, kc, vc,
                      seq_stride, rope_cs, part, ao, ao_hi, ao_lo);
    return launch(L, attn_kernel<kAttnMaxE>, g, b, 0, q, k, v, qw, kw, qk_norm, eps, n_heads, n_kv, hd, S, st, kc, vc,
                  seq_stride, rope_cs, part, ao, ao_hi, ao_lo);
}

hipError_t launch_attn_merge(const Launch &L, const float *part, int n_heads, int hd, int S, float *ao, int B,
                             uint16_t *ao_hi, uint16_t *ao_lo) {
    if ((ao_hi == nullptr) != (ao_lo == nullptr) || (ao_hi && (B > 64 || (n_heads * hd) % 32 != 0)))
        return hipErrorInvalidValue;
    return launch(L, attn_merge_kernel, dim3((unsigned)n_heads, (unsigned)B), dim3(256), 0, part, hd, S, ao, ao_hi,
                  ao_lo);
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

hipError_t launch_combine_rmsnorm(const Launch &L, const float *y, const int32_t *pos_of, const float *weights, int K,
                                  int T, int n, float *x, const float *w, float eps, float *out, uint16_t *hi,
                                  uint16_t *lo) {
    if (T <= 0) return hipSuccess;
    if (K < 1 || K > 8 || n < 1 || n > 4096 || T > 65535 || (hi == nullptr) != (lo == nullptr) ||
        (hi && (T > 64 || n % 32 != 0)))
        return hipErrorInvalidValue;
    return launch(L, combine_rmsnorm_kernel, dim3((unsigned)T), dim3(1024), 0, y, pos_of, weights, K, n, x, w, eps, out,
                  hi, lo);
}

hipError_t launch_rmsnorm(const Launch &L, const float *x, const float *w, int n, float eps, float *out, int B,
                          uint16_t *out_hi, uint16_t *out_lo) {
    if ((out_hi == nullptr) != (out_lo == nullptr) || (out_hi && (B > 64 || n % 32 != 0))) return hipErrorInvalidValue;
    return launch(L, rmsnorm_kernel, dim3((unsigned)B), dim3(1024), 0, x, w, n, eps, out, out_hi, out_lo);
}

hipError_t launch_argmax(const Launch &L, const float *v, int n, StepState *st, int32_t *seq, int ctx, int B) {
    return launch(L, argmax_kernel, dim3((unsigned)B), dim3(1024), 0, v, n, st, seq, ctx);
}

hipError_t launch_sample(const Launch &L, const float *logits, int n, const Sampling &sp, float *prob, int32_t *idx,
                         StepState *st, int32_t *seq, int ctx, int B) {
    return launch(L, sample_kernel, dim3((unsigned)B), dim3(1024), 0, logits, n, sp, prob, idx, st, seq, ctx);
}

hipError_t launch_advance(const Launch &L, StepState *st, int B) {
    return launch(L, advance_kernel, dim3((unsigned)((B + 63) / 64)), dim3(64), 0, st, B);
}

hipError_t launch_record_routing(const Launch &L, const StepState *st, const int32_t *routing, int n_layers, int K,
                                 int B, int ctx, int32_t *hist) {
    return launch(L, record_routing_kernel, dim3((unsigned)B), dim3(256), 0, st, routing, n_layers, K, B, ctx, hist);
}

}  // namespace rbt
