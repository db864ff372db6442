// Internal declarations shared by the gfx950 kernels and the C-ABI layer (not installed).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rbt2_hip.h"

namespace rbt {

constexpr int kWave = 64;  // CDNA wavefront width

// bf16 storage -> f32 is exact: the 16 stored bits are the high half of the f32 (rabbit2.c:304-309).
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xFFFF0000u); }

// f32 -> bf16 bits, round to nearest even (the converter's rule, rabbit2/ref/rbt2.py:106-113, finite
// values). Activations multiplied on the matrix cores are split into hi = bf16(x) and
// lo = bf16(x - hi), which carry ~16 significant bits; products with exact bf16 weights are exact.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

template <int DT>
__device__ __forceinline__ float load_w(const void *W, size_t i) {
    if constexpr (DT == RBT_DT_F32) {
        return static_cast<const float *>(W)[i];
    } else {
        return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t *>(W)[i]) << 16);
    }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (weights are read once per layer; the non-temporal hint keeps them from
// displacing reused data in the caches).
__device__ __forceinline__ u32x4 ld_stream_u4(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ f32x4 ld_stream_f4(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
}
__device__ __forceinline__ f32x4 ld_f4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }

// Matrix-core weight operands straight from row-major bf16 rows. The operand order of
// v_mfma_f32_16x16x32_bf16 (lane -> row lane & 15, 16 bytes at 16 * (lane >> 4) of a 64-byte half-line)
// makes every load instruction touch 16 rows x 64 B, which HBM serves at ~5.3-5.6 TB/s in the grouped
// GEMMs' access pattern, against ~6.6-6.9 TB/s when each instruction reads whole 128-byte lines
// (8 rows x 128 B; measured with read-only probes of the same pattern). So a 16-row group's 128-byte
// k-window (two 32-wide k-steps) is loaded as two such instructions -- a: rows 0-7, b: rows 8-15 of the
// group, lane -> row (lane & 7), 16-byte chunk blob_chunk(lane) of the window -- and turned into the
// operands by one row shift of 8 lanes each way: afterwards a holds chunks 0-3 (k 0..31) and b chunks
// 4-7 (k 32..63) of row (lane & 15), the operands of the two k-steps in the usual order.
__device__ __forceinline__ int blob_chunk(int lane) { return 4 * ((lane >> 3) & 1) + (lane >> 4); }

__device__ __forceinline__ void blob_operands(u32x4 &a, u32x4 &b) {
    u32x4 lo, hi;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // lanes 8..15 of each 16-lane row take b from 8 lanes below; lanes 0..7 of hi take a from 8 above
        lo[i] = (uint32_t)__builtin_amdgcn_update_dpp((int)a[i], (int)b[i], 0x118, 0xF, 0xC, false);  // row_shr:8
        hi[i] = (uint32_t)__builtin_amdgcn_update_dpp((int)b[i], (int)a[i], 0x108, 0xF, 0x3, false);  // row_shl:8
    }
    a = lo;
    b = hi;
}


// Cross-lane moves through DPP (a VALU operand modifier, no LDS round trip). Within each row of 16
// lanes: swap neighbours, swap pairs, mirror each half-row, mirror the row -- after four steps every
// lane of a row holds the same row total (each step adds commutative partners, so all lanes of a
// row see identical operands). ds_bpermute-based shuffles cost an LDS round trip per step instead.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror

__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    v += dpp_f<kDppHalfMirror>(v);
    v += dpp_f<kDppMirror>(v);
    return v;
}

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the 64 lanes, returned to every lane (row totals combined in a fixed order).
__device__ __forceinline__ float wave_sum(float v) {
    v = row_sum16(v);
    return ((lane_value(v, 0) + lane_value(v, 16)) + lane_value(v, 32)) + lane_value(v, 48);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// Where and how a kernel is launched: the stream, and optionally a pair of events that the runtime
// stamps with the kernel's own start and end (hipExtLaunchKernel), used by the profiling mode.
struct Launch {
    hipStream_t s = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
};

template <typename F, typename... Args>
inline hipError_t launch(const Launch &L, F kernel, dim3 grid, dim3 block, uint32_t shmem, Args... args) {
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, L.s, L.start, L.stop, 0, args...);
    return hipGetLastError();
}

// ---- launchers (each returns hipSuccess or the launch error) ----

// Router logits in the engine's exact order (logits kernel, launch context L), then softmax + top-k +
// combine weights (one block per token, context Lk). probs: [T][E] workspace (logits, then
// probabilities).
hipError_t launch_router(const Launch &L, const Launch &Lk, int order, int dtype, const float *xb, const void *W,
                         const float *bias, int T, int E, int D, int K, int norm_topk, float *probs,
                         int32_t *routing, float *weights);

// Tokens up to which the AVX2-order router logits run on the decode kernel (E / 4 x T blocks of 64
// threads; at 32 tokens 5.0 us against 19.9 us for the batch kernel, and with the top-k + split launch
// 9.7 us against 18.1 us for the fused prefill front end; at 512 tokens 28.2 + 4.7 against 19.5 us).
constexpr int kRouterDecodeMaxT = 64;
// (sequence, head) attention blocks from which a step takes one position split (no merge launch).
constexpr int kAttnDirectBlocks = 512;
// Softmax + top-k of T tokens' logits [T][E] (E <= 64) and the bf16 hi/lo split of their rows xb [T][D]
// (D % 8 == 0, 16-byte aligned) into x_hi / x_lo [T][D]: one block per token.
hipError_t launch_topk_split(const Launch &L, const float *logits, int T, int E, int K, int norm_topk, const float *xb,
                             int D, int32_t *routing, float *weights, uint16_t *x_hi, uint16_t *x_lo);
// Router logits (AVX2 order, few tokens, bf16) with the RMSNorm in front folded in: x [T][D] is the
// residual stream and nw the norm weights; token t's xb = x * inv * nw also goes to xb_out [T][D].
bool router_norm_supported(int order, int dtype, int T, int D, const void *W, const float *x, const float *nw);
hipError_t launch_router_norm(const Launch &L, const float *x, const float *nw, float eps, const void *W,
                              const float *bias, int T, int E, int D, float *logits, float *xb_out);

// Only the logits kernel of launch_router.
hipError_t launch_router_logits(const Launch &L, int order, int dtype, const float *xb, const void *W,
                                const float *bias, int T, int E, int D, float *logits);

// Per-(token, slot) GEMV form of the expert FFN (decode and small batches).
hipError_t launch_gateup_gemv(const Launch &L, int dtype, const void *experts, uint64_t stride, const int32_t *routing,
                              const float *xb, int T, int K, int D, int H, float *hbuf);
hipError_t launch_down_combine(const Launch &L, int dtype, const void *experts, uint64_t stride, const int32_t *routing,
                               const float *weights, const float *hbuf, int T, int K, int D, int H, float *x_inout,
                               float *moe_out);

// The same expert FFN specialised for whole-wave-step row lengths (the OLMoE shape among them):
// every load of a wave is issued before the first wait. Lg/Ld: launch contexts of the gate/up and
// down kernels.
bool experts_decode_supported(int dtype, int T, int K, int D, int H, const void *experts, uint64_t stride,
                              const float *xb, const float *hbuf);
hipError_t launch_experts_decode(const Launch &Lg, const Launch &Ld, int dtype, const void *experts, uint64_t stride,
                                 int32_t *routing, float *weights, const float *xb, float *hbuf, int T, int K, int D,
                                 int H, float *x_inout, float *moe_out, const float *logits, int E, int norm_topk);
// With logits != NULL (batch 1, E <= 64) the gate/up kernel runs the softmax + top-k itself and
// fills routing/weights; otherwise it reads routing written by the top-k kernel.
constexpr int kTopkInGateupMaxE = 64;

// Grouped form for many tokens (bf16 weights): dispatch of the (token, slot) pairs into per-expert
// lists, gate/up and down as grouped GEMMs on MFMA (every expert's weights read once per call), and
// the combine in selection order. hbuf [T*K][H]; ws holds prefill_workspace_bytes(). *counts_out
// receives the device address of the tokens-per-expert histogram. Launch contexts: dispatch,
// gate/up, down, combine.
constexpr int kPrefillMinTokensDefault = 12;  // measured crossover with the per-pair GEMVs (OLMoE layer)
bool prefill_supported(int dtype, int T, int min_tokens, int E, int K, int D, int H, const void *experts,
                       uint64_t stride, const float *xb);
size_t prefill_workspace_bytes(int T, int E, int K, int D);
// x_split_done: the bf16 hi/lo planes of xb are already in the workspace (prefill_x_planes), written
// by launch_router_prefill. tile_rows: list rows per GEMM tile (32, 64 or 128; 0 = chosen from the
// mean rows per expert).
hipError_t launch_prefill(const Launch &Ld, const Launch &Lg, const Launch &Lw, const Launch &Lc, const void *experts,
                          uint64_t stride, const float *xb, int T, int E, int K, int D, int H, const int32_t *routing,
                          const float *weights, float *hbuf, void *ws, float *x_inout, float *moe_out,
                          int32_t **counts_out, bool x_split_done,
                          bool combine = true, int tile_rows = 0, const void *tiled = nullptr, bool wide_ok = true);
// The tiled copy of a layer's bf16 experts that the 128-row grouped GEMMs stream contiguously (same
// bytes as the blobs, in tile order): whether the shape has one, its size, and the re-layout launch
// (experts in the blob layout with stride, into dst). tiled = that copy, or nullptr for the blobs.
bool prefill_layout_supported(int dtype, int D, int H);
size_t prefill_layout_bytes(int E, int D, int H);
hipError_t launch_prefill_layout(const Launch &L, const void *experts, uint64_t stride, int E, int D, int H, void *dst);
void prefill_x_planes(void *ws, int T, int E, int K, int D, uint16_t **x_hi, uint16_t **x_lo);
// combine = false: launch_prefill stops after the down GEMM; the combine's inputs (y [P][D] in list
// order, pos_of [P]) are then these, for launch_combine_rmsnorm.
void prefill_combine_inputs(void *ws, int T, int E, int K, int D, const float **y, const int32_t **pos_of);
// The grouped path's combine (x += sum_k w[t][k] y[pos_of[t*K+k]] in selection order, K <= 8) fused
// with the RMSNorm of the new rows that the next step starts with (out = x * inv * w, and the
// matrix-core planes if hi/lo are given): one block per token, bit for bit the two launches.
hipError_t launch_combine_rmsnorm(const Launch &L, const float *y, const int32_t *pos_of, const float *weights, int K,
                                  int T, int n, float *x, const float *w, float eps, float *out, uint16_t *hi,
                                  uint16_t *lo);

// Router logits + softmax + top-k + the activation hi/lo split in one launch, for the grouped path
// (AVX2 order, E <= 64). x_hi/x_lo may be NULL (no split).
bool router_prefill_supported(int order, int dtype, int T, int E, int D, int K, const void *W, const float *xb);
hipError_t launch_router_prefill(const Launch &L, int dtype, const float *xb, const void *W, const float *bias, int T,
                                 int E, int D, int K, int norm_topk, int32_t *routing, float *weights,
                                 uint16_t *x_hi, uint16_t *x_lo);

// ---- full forward pass around the MoE block (model.hip)
// The step record every forward kernel reads: the position being processed; seq[pos] is its token.
struct StepState {
    int32_t pos;       // position of the step being processed
    int32_t n_prompt;  // prompt length: the argmax / sampler appends tokens to seq[] only past it
    int32_t last;      // the last argmax / sampler result
    int32_t pad;
    uint64_t rng;      // the sampler's xorshift64* state (rabbit2.c:558-567, :723)
    uint64_t pad2;
};
// The engine's sampling settings (--temperature, --top-k, --top-p; rabbit2.c:634-638).
struct Sampling {
    float temperature = 0.0f;  // <= 0: greedy
    int top_k = 0;
    float top_p = 1.0f;
};
// sample_logits (rabbit2.c:569-610) for B sequences, one block each: logits [B][n], scratch prob/idx
// [B][n]; then the step advances like the argmax.
hipError_t launch_sample(const Launch &L, const float *logits, int n, const Sampling &sp, float *prob, int32_t *idx,
                         StepState *st, int32_t *seq, int ctx, int B);
// Per-token kernels take B sequences: sequence b has the record st[b], the token row seq[b * ctx ..),
// and rows b of x / q / k / v / attn_out / logits.
hipError_t launch_embed(const Launch &L, int dtype, const void *emb, int D, int vocab, const StepState *st,
                        const int32_t *seq, int ctx, float *x, int B);
// out_s = W_s (x * inv * nw) for up to three row segments (rows[s] may be 0); W_s rows have D elements.
hipError_t launch_norm_matvec(const Launch &L, int dtype, const float *x, const float *nw, float eps, int D,
                              const void *const W[3], float *const out[3], const int rows[3]);
// The same with many rows per wave and every weight load issued first, for rows of whole 1 KiB
// wave-steps (D a multiple of 512 bf16 / 256 f32, at most 8 steps) -- dense_supported(). _resid: x[r] +=
// W[r] . a (wo). _argmax: the
// final norm + lm_head rows with one (value, index) candidate per block (dense_argmax_blocks(rows) of
// them), then a one-block launch that reduces them, advances the step and appends the token.
bool dense_supported(int dtype, int D, const void *const W[3], const int rows[3]);
hipError_t launch_dense_norm(const Launch &L, int dtype, const float *x, const float *nw, float eps, int D,
                             const void *const W[3], float *const out[3], const int rows[3]);
hipError_t launch_dense_resid(const Launch &L, int dtype, const float *a, int cols, const void *W, int rows, float *x);
int dense_argmax_blocks(int rows);
hipError_t launch_dense_argmax(const Launch &L, int dtype, const float *x, const float *nw, float eps, int D,
                               const void *W, int rows, float *logits, float2 *cand, StepState *st, int32_t *seq,
                               int ctx);
// Attention of one step: grid (n_heads, S splits of the positions), each block writes its partial
// (m, l, o[hd]) to part [n_heads][S][hd + 2]; launch_attn_merge merges them into ao (S <= 64). With
// S == 1 and ao given, the attention writes ao [B][n_heads * hd] (and the matrix-core planes ao_hi /
// ao_lo, if given) itself, bit for bit what the merge would, and no merge is launched.
// rope_cs: [ctx][hd/2] (cos, sin) of the engine's RoPE angles. hd <= 256.
// kc/vc: this layer's cache of sequence 0; sequence b's starts seq_stride floats further.
hipError_t launch_attention(const Launch &L, const float *q, const float *k, const float *v, const float *qw,
                            const float *kw, int qk_norm, float eps, int n_heads, int n_kv, int hd, int S,
                            const StepState *st, float *kc, float *vc, size_t seq_stride, const float2 *rope_cs,
                            float *part, int B,
                            float *ao = nullptr, uint16_t *ao_hi = nullptr, uint16_t *ao_lo = nullptr);
hipError_t launch_attn_merge(const Launch &L, const float *part, int n_heads, int hd, int S, float *ao, int B,
                             uint16_t *ao_hi = nullptr, uint16_t *ao_lo = nullptr);
// Dense rows over B token vectors xin [B][D] (batched decode): out_s [B][rows_s], or with resid != NULL
// resid [B][rows] += (one segment). Same row shapes as dense_supported.
hipError_t launch_dense_batch(const Launch &L, int dtype, const float *xin, int B, int D, const void *const W[3],
                              float *const out[3], const int rows[3], float *resid);
hipError_t launch_wo(const Launch &L, int dtype, const float *ao, int q_dim, const void *Wo, int D, float *x);
// out_hi / out_lo (may be null): the rows' bf16 hi and lo parts as well, as matrix-core planes
// (mfma_plane_index; n a multiple of 32).
hipError_t launch_rmsnorm(const Launch &L, const float *x, const float *w, int n, float eps, float *out, int B,
                          uint16_t *out_hi = nullptr, uint16_t *out_lo = nullptr);
// launch_dense_batch on the matrix cores: B <= 64 token rows given as bf16 hi/lo planes (mfma_plane_index); bf16
// weights only, K = 128 * {1, 2, 4, 8, 16}, every segment a multiple of 16 rows
// (dense_mfma_supported). The products are exact; the sums run in the MFMA order, then the slices of
// K in a fixed order.
bool dense_mfma_supported(int dtype, int B, int K, const void *const W[3], const int rows[3]);
hipError_t launch_dense_mfma(const Launch &L, const uint16_t *x_hi, const uint16_t *x_lo, int B, int K,
                             const void *const W[3], float *const out[3], const int rows[3], float *resid);
// The bf16 hi/lo planes of B <= 64 token rows of K elements (K a multiple of 32) in the order the matrix
// cores take their B operand: one 1 KiB tile per (k-step of 32, block of 16 tokens), k-step-major;
// inside a tile, lane (t % 16) + 16 * ((k % 32) / 8) holds token t's 8 elements from k - k % 8 on.
// A wave's load of one operand tile is then one contiguous 1 KiB. Tiles of a partial token block are
// whole (their unused lanes are never written and only feed outputs that are dropped).
inline size_t mfma_plane_elems(int B, int K) { return (size_t)K * (size_t)((B + 15) / 16) * 16; }
__device__ __forceinline__ size_t mfma_plane_index(int t, int k, int TB) {
    return ((size_t)(k >> 5) * (size_t)TB + (size_t)(t >> 4)) * 512 + (size_t)(((t & 15) + 16 * ((k >> 3) & 3)) * 8 + (k & 7));
}
hipError_t launch_argmax(const Launch &L, const float *v, int n, StepState *st, int32_t *seq, int ctx, int B);
hipError_t launch_advance(const Launch &L, StepState *st, int B);
// Copies the step's routing [n_layers][B][K] into hist [B][ctx][n_layers][K] at each sequence's
// current position (run before the step advances).
hipError_t launch_record_routing(const Launch &L, const StepState *st, const int32_t *routing, int n_layers, int K,
                                 int B, int ctx, int32_t *hist);

// Dense matvec (one row per wave).
hipError_t launch_matvec(const Launch &L, int dtype, const void *W, const float *x, float *out, int rows, int cols);

// Synthetic normal fill (SplitMix64 + Box-Muller), see rbt_hip_fill_normal.
hipError_t launch_fill_normal(const Launch &L, void *dst, int dtype, uint64_t n, uint64_t seed, uint64_t stream,
                              uint64_t first, float scale, float offset);

}  // namespace rbt
