// Prefill (many tokens per call): expert dispatch, grouped SwiGLU GEMMs on bf16 MFMA, combine.
//
// Reference semantics: rabbit2/src/rabbit2.c:531-542, applied to every token of the batch (the
// engine evaluates a prompt one token at a time, :703-714; the tokens are independent inside the
// MoE block): for each selected expert k of a token, h = silu(W1 xb) * (W3 xb), tmp = W2 h,
// moe += w_k * tmp in selection order, x += moe. Expert blob layout w1[H][D] | w3[H][D] | w2[D][H]
// (rabbit2.c:173, rabbit2/tools/rbt2.py:152-156), bf16 elements.
//
// 1. dispatch_kernel: per-expert lists of the (token, slot) pairs, stable in pair order (counts,
//    row offsets, perm, inverse perm) and the per-expert count of row tiles (64 rows, or 32 when the
//    experts average at most 16 rows).
// 2. grouped_gemm_kernel<2>: for each expert's rows, h = silu(W1 a) * (W3 a), written as bf16 hi/lo
//    planes; grouped_gemm_kernel<1>: y = W2 h (f32 rows). Both on v_mfma_f32_16x16x32_bf16.
//    The f32 activations are split into bf16 hi + lo parts and both parts are multiplied (two MFMAs
//    per product). The bf16 weights are exact, so each product keeps ~16 bits of the activation
//    instead of 8. A full 64-row tile then does 64 rows x 2 parts x 2 flop = 256 flop per weight
//    element, 128 flop per weight byte: below the bf16 MFMA/HBM ridge (2.5 PFLOP/s / 8 TB/s =
//    312), so the kernels stay bound by HBM.
//    Tiles: 64 rows x 256 weight rows per block of 16 waves (or 32 x 128 per 8 waves for decode-sized
//    batches);
//    the reduction runs in chunks of 64 (128) through a three-stage LDS ring filled by direct
//    HBM -> LDS copies (weights and activations).
//    Tile order (expert, column tile, row tile), split into 8 contiguous ranges, one per XCD (the
//    hardware hands block b to XCD b % 8): the row tiles of a hot expert then share each weight
//    tile in that XCD's L2, and an expert's activation rows are reused across its column tiles.
// 3. combine_rows_kernel: moe[t] = sum_k w[t][k] * y[pos(t,k)] in selection order, x += moe.
#include <math.h>

#include <algorithm>

#include "rbt2_internal.h"

namespace rbt {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kDispatchMaxE = 256;


// ---------------------------------------------------------------- dispatch (one block, 1024 threads)
// routing [P] with pair p = t*K + k. Outputs: counts[E]; offsets[E+1] (exclusive prefix of counts);
// perm[P]: pair ids grouped by expert, increasing within an expert; pos_of[P]: inverse of perm;
// m_off[E+1]: exclusive prefix of ceil(counts / mt_rows) (the grouped GEMMs' row tiles per expert).
// Wave w owns the pair slice [w*S, (w+1)*S). A: each wave ranks its pairs, 64 at a time, against
// equal experts (ballots over the expert-id bits) and keeps per-expert running counts in its own LDS
// row; a pair's rank inside its wave's slice goes to pos_of as a temporary. B: wave 0 (4 experts per
// lane) sums the waves' counts, scans them into the offsets, and turns each wave's counts into that
// wave's first position per expert. C: every pair adds its wave's base. Three barriers in all.
__global__ __launch_bounds__(1024) void dispatch_kernel(const int32_t *__restrict__ routing, int P, int E,
                                                        int32_t *__restrict__ counts, int32_t *__restrict__ offsets,
                                                        int32_t *__restrict__ perm, int32_t *__restrict__ pos_of,
                                                        int32_t *__restrict__ m_off, int mt_rows) {
    constexpr int NW = 16;
    __shared__ int s_w[NW][kDispatchMaxE];  // A: running counts per wave; B: each wave's base positions
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int i = tid; i < NW * kDispatchMaxE; i += 1024) (&s_w[0][0])[i] = 0;
    __syncthreads();
    const int S = ((P + NW - 1) / NW + 63) / 64 * 64;  // slice per wave, whole 64-pair steps
    const int base = wv * S, end = min(P, base + S);
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int p0 = base; p0 < end; p0 += 64) {  // wave-uniform loop
        const int p = p0 + lane;
        const bool valid = p < end;
        const int e = valid ? min(max(routing[p], 0), E - 1) : 0;
        uint64_t same = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (e >> b) & 1;
            const uint64_t ones = __ballot(bit);
            same &= bit ? ones : ~ones;
        }
        const int before = __popcll(same & below);
        const int cur = valid ? s_w[wv][e] : 0;  // read by every lane before any update (in-order LDS)
        if (valid) pos_of[p] = cur + before;
        if (valid && (same >> lane) == 1ull) s_w[wv][e] = cur + before + 1;  // last lane of its expert
    }
    __syncthreads();
    if (wv == 0) {
        int c[4], mt[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            int tot = 0;
            if (e < E)
                for (int w = 0; w < NW; ++w) tot += s_w[w][e];
            c[i] = tot;
            mt[i] = (tot + mt_rows - 1) / mt_rows;
        }
        // exclusive scans across the wave of the lanes' sums (4 experts per lane, ascending)
        int sc = ((c[0] + c[1]) + c[2]) + c[3], sm = ((mt[0] + mt[1]) + mt[2]) + mt[3];
        int ic = sc, im = sm;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int uc = __shfl_up(ic, d, 64), um = __shfl_up(im, d, 64);
            if (lane >= d) {
                ic += uc;
                im += um;
            }
        }
        int oc = ic - sc, om = im - sm;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            if (e < E) {
                counts[e] = c[i];
                offsets[e] = oc;
                m_off[e] = om;
                int run = oc;  // each wave's first position for expert e
                for (int w = 0; w < NW; ++w) {
                    const int n = s_w[w][e];
                    s_w[w][e] = run;
                    run += n;
                }
            }
            if (e == E - 1) {
                offsets[E] = oc + c[i];
                m_off[E] = om + mt[i];
            }
            oc += c[i];
            om += mt[i];
        }
    }
    __syncthreads();
    for (int p0 = base; p0 < end; p0 += 64) {
        const int p = p0 + lane;
        if (p < end) {
            const int e = min(max(routing[p], 0), E - 1);
            const int pos = s_w[wv][e] + pos_of[p];
            perm[pos] = p;
            pos_of[p] = pos;
        }
    }
}

// ---------------------------------------------------------------- activation split
// x (f32) -> hi = bf16_rne(x), lo = bf16_rne(x - hi): hi + lo carries ~16 significant bits, and every
// MFMA product with an exact bf16 weight is exact in the f32 accumulator.
__global__ __launch_bounds__(256) void split_hilo_kernel(const float *__restrict__ x, size_t n8,
                                                        uint16_t *__restrict__ hi, uint16_t *__restrict__ lo) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n8; i += (size_t)gridDim.x * blockDim.x) {
        const f32x4 a = ld_f4(x + 8 * i), b = ld_f4(x + 8 * i + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t h[8], l[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            h[k] = f32_to_bf16_rne(v[k]);
            l[k] = f32_to_bf16_rne(v[k] - __uint_as_float(h[k] << 16));
        }
        *reinterpret_cast<u32x4 *>(hi + 8 * i) = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                                                      h[6] | (h[7] << 16)};
        *reinterpret_cast<u32x4 *>(lo + 8 * i) = u32x4{l[0] | (l[1] << 16), l[2] | (l[3] << 16), l[4] | (l[5] << 16),
                                                      l[6] | (l[7] << 16)};
    }
}

// ---------------------------------------------------------------- grouped GEMM
// Direct HBM -> LDS copies (global_load_lds_dwordx4): each lane's 16 bytes land at LDS m0 + 16*lane, so
// one instruction fills 1 KiB of LDS in lane order and costs no registers. They are issued from inline
// assembly and waited for by hand (s_waitcnt vmcnt): the compiler, which would otherwise wait for every
// pending copy before any LDS read, does not see them. The main loop issues no other vector-memory
// operation, so vmcnt counts exactly these copies.
__device__ __forceinline__ void lds_dma16(const void *g, uint32_t lds_byte) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_byte), "v"(g) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_dma() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Tile: ROWS list rows x WROWS weight rows (gate/up: half W1 rows, the same rows of W3; down: W2
// rows), the reduction in chunks that are one ring stage in LDS each; three stages, the copies of
// stages c+1 and c+2 in flight while the MFMAs run on stage c:
//   ROWS = 64: 256 weight rows x 128 B (k-chunks of 64) + 2 x 64 activation rows x 128 B = 48 KiB
//   ROWS = 32: 128 weight rows x 256 B (k-chunks of 128) + 2 x 32 activation rows x 256 B = 48 KiB
// (the activation rows: bf16 hi and lo planes). The kernel is bound by its copies: it keeps 90% of
// its time with the MFMAs and operand reads taken out, and a stage takes ~1.45 us whether two or
// three stages are in flight and whether a row is read in 128- or 256-byte runs. At 5.8 TB/s of
// weights it runs at ~94% of what one block per CU streams with plain loads of 32 KiB steps (6.2
// TB/s, measured for 512 and 1024 threads and runs of 128 B to 1 KiB); the LDS ring leaves no room
// for a second block. Copies: 1 KiB each (8 rows of 128 B or 4 of 256 B), 4 weight + 2 activation
// per wave.
constexpr int kGWRows = 256, kGKC = 64;  // the 64-row tile; prefill_supported's shape rules
constexpr int kSmallTileRowsPerExpert = 16;  // mean list rows per expert up to which tiles have 32 rows
template <int ROWS>
struct GTile {
    static constexpr int kWRows = ROWS == 64 ? 256 : 128;  // weight rows per tile
    static constexpr int kKC = ROWS == 64 ? 64 : 128;      // k per stage
    static constexpr int kRowB = 2 * kKC;                  // bytes of each row per stage
    static constexpr int kGran = kRowB / 16;               // 16-byte granules per row per stage
    static constexpr int kRowsPerCopy = 1024 / kRowB;      // rows one 1 KiB copy covers
    static constexpr int kStages = 3;
    static constexpr int kWBytes = kWRows * kRowB;         // 32 KiB
    static constexpr int kABytes = ROWS * kRowB;
    static constexpr int kStageBytes = kWBytes + 2 * kABytes;
    static constexpr int kWaves = ROWS == 64 ? 16 : 8;    // waves per block (each needs a W1/W3 pair)
    static constexpr int kRG = ROWS / 16;                  // row groups of 16 (one per wave)
    static constexpr int kCH = kWaves / kRG;               // weight-row splits (waves per row group)
    static constexpr int kNB = kWRows / 16 / kCH;          // weight blocks of 16 per wave
    static constexpr int kWI = kWBytes / 1024 / kWaves;    // weight copies per wave per stage
    static constexpr int kACP = kABytes / 1024;            // copies per activation plane
    static constexpr int kAI = 2 * kACP / kWaves;          // activation copies per wave per stage
    static constexpr int kDmaPerWave = kWI + kAI;
    static_assert((ROWS == 64 || ROWS == 32) && kStages * kStageBytes <= 160 * 1024 &&
                      kAI * kWaves == 2 * kACP && kWI * kWaves * 1024 == kWBytes && kNB >= 2 && kNB % 2 == 0,
                  "tile shape");
    // Inside a stage, row r's granule g sits at slot swz(r, g): the MFMA operand reads (16 consecutive
    // rows at one granule per 16 lanes) then hit 16 distinct bank groups (two rows per 256 bytes of
    // banks for 128-byte rows, one for 256-byte rows).
    __device__ static int swz(int r, int g) { return kRowB == 128 ? g ^ ((r >> 1) & 7) : g ^ (r & 15); }
};

// MATS = 2: h = silu(W1 a) * (W3 a) for a = xb rows gathered through perm (N = H columns, Kd = D),
//           written as bf16 hi/lo planes [P][N] (the next GEMM's activation operand).
// MATS = 1: y = W2 a for a = the h planes in list order (N = D, Kd = H), written as f32 [P][N].
// Waves: w = kRG*ch + rg computes list rows [16 rg, +16) x the ch-th of kCH parts of the tile's weight
// rows (kNB blocks of 16: gate/up W1 blocks (kNB/2) ch .. and the matching W3 blocks; down W2 blocks
// kNB ch ..).
// Requirements (prefill_supported): N % (256 / MATS) == 0, Kd % 64 == 0, 16-byte aligned rows.
template <int MATS, int ROWS>
__global__ __launch_bounds__(64 * GTile<ROWS>::kWaves, 1) void grouped_gemm_kernel(
    const uint8_t *__restrict__ experts, uint64_t stride, uint64_t w_off, uint64_t w3_off, int N, int Kd,
    const uint16_t *__restrict__ a_hi, const uint16_t *__restrict__ a_lo, int gather, const int32_t *__restrict__ perm,
    int topk, const int32_t *__restrict__ counts, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ m_off, int E, float *__restrict__ out_f32, uint16_t *__restrict__ out_hi,
    uint16_t *__restrict__ out_lo) {
    using TS = GTile<ROWS>;
    constexpr int WROWS = TS::kWRows, NTILE = WROWS / MATS;  // output columns per tile
    constexpr int STAGES = TS::kStages, SBYTES = TS::kStageBytes, NB = TS::kNB, AI = TS::kAI, WI = TS::kWI;
    constexpr int ROWB = TS::kRowB, GRAN = TS::kGran, RPC = TS::kRowsPerCopy, WBYTES = TS::kWBytes;
    __shared__ __align__(1024) uint8_t ring[STAGES * SBYTES];

    // w in a scalar register: the branches on it below are then wave-uniform jumps, not exec masks
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), rg = w % TS::kRG,
              ch = w / TS::kRG;
    const int ntiles_n = N / NTILE;
    const int total = m_off[E] * ntiles_n;
    const int range = (total + 7) >> 3;
    const int slot = (int)(blockIdx.x >> 3);
    const int tau = (int)(blockIdx.x & 7) * range + slot;
    if (slot >= range || tau >= total) return;
    int lo = 0, hi = E - 1;  // the expert owning tile tau: the last e with m_off[e] * ntiles_n <= tau
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (m_off[mid] * ntiles_n <= tau)
            lo = mid;
        else
            hi = mid - 1;
    }
    const int e = lo;
    const int me = m_off[e + 1] - m_off[e];
    const int local = tau - m_off[e] * ntiles_n;
    const int jt = local / me, il = local - jt * me;
    const int row0 = offsets[e] + il * ROWS;
    const int rows = min(ROWS, counts[e] - il * ROWS);
    const int n0 = jt * NTILE;
    const size_t rowb = (size_t)Kd * 2;  // bytes per weight / activation-plane row

    // copy sources of this lane (one pointer per instruction; each stage adds 128 bytes)
    const uint8_t *wsrc[WI];
#pragma unroll
    for (int i = 0; i < WI; ++i) {
        const int t = WI * w + i, r = RPC * t + lane / GRAN, g = TS::swz(r, lane % GRAN);
        const uint8_t *base = experts + (size_t)e * stride + w_off;
        int wr = n0 + r;
        if constexpr (MATS == 2) {
            if (r >= WROWS / 2) {
                base = experts + (size_t)e * stride + w3_off;
                wr = n0 + r - WROWS / 2;
            }
        }
        wsrc[i] = base + (size_t)wr * rowb + 16 * g;
    }
    const uint8_t *asrc[AI];
#pragma unroll
    for (int i = 0; i < AI; ++i) {
        // copy u: plane u / kACP, rows RPC * (u % kACP) ..
        const int u = AI * w + i, plane = u / TS::kACP, r = RPC * (u % TS::kACP) + lane / GRAN,
                  g = TS::swz(r, lane % GRAN);
        const int lr = row0 + (r < rows ? r : 0);  // rows past the list re-read its first row
        const size_t arow = gather ? (size_t)(perm[lr] / topk) : (size_t)lr;
        asrc[i] = reinterpret_cast<const uint8_t *>(plane ? a_lo : a_hi) + arow * rowb + 16 * g;
    }
    const uint32_t ring0 = (uint32_t)(uintptr_t)ring;
    const int nch = Kd / TS::kKC;
    // Stage c reads k-chunk (c + rot) mod nch. Without the rotation every resident block streams the
    // same column window of its rows at the same time, so the whole chip's requests fall on the few
    // DRAM channels that window maps to. The rotation is a function of the weight tile (expert,
    // column tile), so the m-tiles that share a tile read it in the same order and stay in step (their
    // second reads hit L2); the per-output summation order is still fixed for a given input.
    const int rot = (e * ntiles_n + jt) % nch;
    auto issue = [&](int c) {
        const uint32_t sb = ring0 + (uint32_t)((c % STAGES) * SBYTES);
        const int cc = c + rot < nch ? c + rot : c + rot - nch;
        const size_t kb = (size_t)cc * ROWB;
#pragma unroll
        for (int i = 0; i < WI; ++i)
            lds_dma16(wsrc[i] + kb, __builtin_amdgcn_readfirstlane(sb + (WI * w + i) * 1024));
#pragma unroll
        for (int i = 0; i < AI; ++i)
            lds_dma16(asrc[i] + kb, __builtin_amdgcn_readfirstlane(sb + WBYTES + (AI * w + i) * 1024));
    };

    // MFMA operand reads: lane -> row (lane % 16) of a 16-row block, logical granule 4*ks + lane / 16
    int brow[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) {
        int blk;
        if constexpr (MATS == 2)
            blk = q < NB / 2 ? (NB / 2) * ch + q : WROWS / 32 + (NB / 2) * ch + (q - NB / 2);
        else
            blk = NB * ch + q;
        brow[q] = blk * 16 + (lane & 15);
    }
    const int arw = 16 * rg + (lane & 15);
    const bool active = 16 * rg < rows;  // wave-uniform: this wave's 16 rows hold list entries

    f32x4 acc[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) acc[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int c = 0; c < STAGES - 1 && c < nch; ++c) issue(c);
    for (int c = 0; c < nch; ++c) {
        // stages c+1 .. c+STAGES-2 (as far as they exist) may still be in flight, stage c must have landed
        const int ahead = min(STAGES - 2, nch - 1 - c);
        if (ahead >= 2)
            wait_dma<2 * TS::kDmaPerWave>();
        else if (ahead == 1)
            wait_dma<TS::kDmaPerWave>();
        else
            wait_dma<0>();
        __syncthreads();  // every wave's copies of stage c have landed
        if (c + STAGES - 1 < nch) issue(c + STAGES - 1);  // into the stage read at c-1: all waves are past it
        if (active) {
            const uint8_t *st = ring + (c % STAGES) * SBYTES;
#pragma unroll
            for (int ks = 0; ks < TS::kKC / 32; ++ks) {
                const int g = 4 * ks + (lane >> 4);
                const bf16x8 ah = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4 *>(st + WBYTES + arw * ROWB + 16 * TS::swz(arw, g)));
                const bf16x8 al = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4 *>(st + WBYTES + TS::kABytes + arw * ROWB + 16 * TS::swz(arw, g)));
#pragma unroll
                for (int q = 0; q < NB; ++q) {
                    const bf16x8 bv =
                        __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(st + brow[q] * ROWB + 16 * TS::swz(brow[q], g)));
                    acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bv, acc[q], 0, 0, 0);
                    acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bv, acc[q], 0, 0, 0);
                }
            }
        }
    }
    if (!active) return;

    // epilogue: acc[q] lane holds weight row (block q, lane % 16) for list rows 16 rg + 4*(lane/16) + i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 16 * rg + 4 * (lane >> 4) + i;
        if (r >= rows) continue;
        const size_t orow = (size_t)(row0 + r) * N;
        if constexpr (MATS == 2) {
#pragma unroll
            for (int q = 0; q < NB / 2; ++q) {
                const float g = acc[q][i], u = acc[q + NB / 2][i];
                const float v = (g / (1.0f + expf(-g))) * u;  // silu(g) * u, rabbit2.c:535-537
                const uint32_t hb = f32_to_bf16_rne(v);
                const uint32_t lb = f32_to_bf16_rne(v - __uint_as_float(hb << 16));
                const size_t o = orow + n0 + ((NB / 2) * ch + q) * 16 + (lane & 15);
                out_hi[o] = (uint16_t)hb;
                out_lo[o] = (uint16_t)lb;
            }
        } else {
#pragma unroll
            for (int q = 0; q < NB; ++q) out_f32[orow + n0 + (NB * ch + q) * 16 + (lane & 15)] = acc[q][i];
        }
    }
}

// moe[t][d] = sum_k w[t][k] * y[pos_of[t*K+k]][d] in selection order (rabbit2.c:540); x += moe.
__global__ __launch_bounds__(256) void combine_rows_kernel(const float *__restrict__ y,
                                                          const int32_t *__restrict__ pos_of,
                                                          const float *__restrict__ weights, int K, int D,
                                                          float *__restrict__ x_inout, float *__restrict__ moe_out) {
    const int t = blockIdx.y;
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= D) return;
    const size_t o = (size_t)t * D + d;
    const float xo = x_inout ? x_inout[o] : 0.0f;
    float moe = 0.0f;
    if (K <= 8) {  // the common case: every load of the row issued before the sum (indices clamped)
        int p[8];
        float wk[8], tmp[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int kc = min(k, K - 1);
            p[k] = pos_of[t * K + kc];
            wk[k] = weights[t * K + kc];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) tmp[k] = y[(size_t)p[k] * D + d];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
#pragma clang fp contract(off)
            if (k < K) moe = moe + wk[k] * tmp[k];
        }
    } else {
        for (int k = 0; k < K; ++k) {
#pragma clang fp contract(off)
            const float tmp = y[(size_t)pos_of[t * K + k] * D + d];
            const float wk = weights[t * K + k];
            moe = moe + wk * tmp;
        }
    }
    if (moe_out) moe_out[o] = moe;
    if (x_inout) x_inout[o] = xo + moe;
}

template <int MATS, int ROWS>
hipError_t launch_gemm(const Launch &L, const uint8_t *experts, uint64_t stride, uint64_t w_off, uint64_t w3_off,
                       int N, int Kd, const uint16_t *a_hi, const uint16_t *a_lo, int gather, const int32_t *perm,
                       int topk, const int32_t *counts, const int32_t *offsets, const int32_t *m_off, int E,
                       int max_mtiles, float *out_f32, uint16_t *out_hi, uint16_t *out_lo) {
    const long long tiles = (long long)max_mtiles * (N / (GTile<ROWS>::kWRows / MATS));
    const long long blocks = (tiles + 7) / 8 * 8;
    if (blocks > 0x7FFFFFFFll) return hipErrorInvalidValue;
    return launch(L, grouped_gemm_kernel<MATS, ROWS>, dim3((unsigned)blocks), dim3(64 * GTile<ROWS>::kWaves), 0, experts,
                  stride, w_off, w3_off,
                  N, Kd, a_hi, a_lo, gather, perm, topk, counts, offsets, m_off, E, out_f32, out_hi, out_lo);
}

}  // namespace

bool prefill_supported(int dtype, int T, int min_tokens, int E, int K, int D, int H, const void *experts, uint64_t stride,
                       const float *xb) {
    return dtype == RBT_DT_BF16 && T >= min_tokens && T <= 65535 && E <= kDispatchMaxE && (long long)T * K <= (1 << 24) &&
           D % kGWRows == 0 && H % (kGWRows / 2) == 0 && D % kGKC == 0 && H % kGKC == 0 &&
           (reinterpret_cast<uintptr_t>(experts) & 15u) == 0 && stride % 16 == 0 &&
           (reinterpret_cast<uintptr_t>(xb) & 15u) == 0;
}

size_t prefill_workspace_bytes(int T, int E, int K, int D) {
    const size_t P = (size_t)T * K;
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    return up(4 * (size_t)E) + 2 * up(4 * (size_t)(E + 1)) + 2 * up(4 * P) + up(4 * P * (size_t)D) +
           2 * up(2 * (size_t)T * D);
}

namespace {
// Workspace carve-up of the grouped path (prefill_workspace_bytes is its total).
struct PrefillWs {
    int32_t *counts, *offsets, *m_off, *perm, *pos_of;
    float *y;
    uint16_t *x_hi, *x_lo;
};
PrefillWs carve_ws(void *ws, int T, int E, int K, int D) {
    const int P = T * K;
    uint8_t *w = static_cast<uint8_t *>(ws);
    auto carve = [&](size_t bytes) {
        uint8_t *p = w;
        w += (bytes + 255) / 256 * 256;
        return p;
    };
    PrefillWs r;
    r.counts = reinterpret_cast<int32_t *>(carve(4 * (size_t)E));
    r.offsets = reinterpret_cast<int32_t *>(carve(4 * (size_t)(E + 1)));
    r.m_off = reinterpret_cast<int32_t *>(carve(4 * (size_t)(E + 1)));
    r.perm = reinterpret_cast<int32_t *>(carve(4 * (size_t)P));
    r.pos_of = reinterpret_cast<int32_t *>(carve(4 * (size_t)P));
    r.y = reinterpret_cast<float *>(carve(4 * (size_t)P * D));
    r.x_hi = reinterpret_cast<uint16_t *>(carve(2 * (size_t)T * D));
    r.x_lo = reinterpret_cast<uint16_t *>(carve(2 * (size_t)T * D));
    return r;
}
}  // namespace

void prefill_combine_inputs(void *ws, int T, int E, int K, int D, const float **y, const int32_t **pos_of) {
    const PrefillWs r = carve_ws(ws, T, E, K, D);
    *y = r.y;
    *pos_of = r.pos_of;
}

void prefill_x_planes(void *ws, int T, int E, int K, int D, uint16_t **x_hi, uint16_t **x_lo) {
    const PrefillWs r = carve_ws(ws, T, E, K, D);
    *x_hi = r.x_hi;
    *x_lo = r.x_lo;
}

hipError_t launch_prefill(const Launch &Ld, const Launch &Lg, const Launch &Lw, const Launch &Lc, const void *experts,
                          uint64_t stride, const float *xb, int T, int E, int K, int D, int H, const int32_t *routing,
                          const float *weights, float *hbuf, void *ws, float *x_inout, float *moe_out,
                          int32_t **counts_out, bool x_split_done, bool combine) {
    const int P = T * K;
    const PrefillWs r = carve_ws(ws, T, E, K, D);
    int32_t *counts = r.counts, *offsets = r.offsets, *m_off = r.m_off, *perm = r.perm, *pos_of = r.pos_of;
    float *y = r.y;
    uint16_t *x_hi = r.x_hi, *x_lo = r.x_lo;
    // the h planes (bf16 hi, lo; [P][H] each) take the f32 [P][H] h buffer
    uint16_t *h_hi = reinterpret_cast<uint16_t *>(hbuf), *h_lo = h_hi + (size_t)P * H;
    if (counts_out) *counts_out = counts;
    // activation split (unless the router kernel wrote the planes), then the dispatch: one timed
    // interval (first start .. dispatch end)
    hipError_t e = hipSuccess;
    Launch Ldd = Ld;
    if (!x_split_done) {
        Launch Ls = Ld;
        Ls.stop = nullptr;
        Ldd.start = nullptr;
        const size_t n8 = (size_t)T * D / 8;
        const unsigned sblocks = (unsigned)std::min<size_t>((n8 + 255) / 256, 2048);
        e = launch(Ls, split_hilo_kernel, dim3(sblocks), dim3(256), 0, xb, n8, x_hi, x_lo);
        if (e != hipSuccess) return e;
    }
    // row tiles of 32 when experts average at most 16 rows (decode-sized batches: a deeper copy ring),
    // of 64 otherwise (fewer tiles, each weight tile read once per 64 rows)
    const bool small = P <= kSmallTileRowsPerExpert * E;
    const int mt_rows = small ? 32 : 64;
    e = launch(Ldd, dispatch_kernel, dim3(1), dim3(1024), 0, routing, P, E, counts, offsets, perm, pos_of, m_off,
               mt_rows);
    if (e != hipSuccess) return e;
    const uint8_t *ex = static_cast<const uint8_t *>(experts);
    const int max_mtiles = (P + mt_rows - 1) / mt_rows + E;  // >= sum over experts of ceil(count / mt_rows)
    // gate/up: N = H, Kd = D, activation rows gathered through perm; h written as hi/lo planes
    e = small ? launch_gemm<2, 32>(Lg, ex, stride, 0, (uint64_t)H * D * 2, H, D, x_hi, x_lo, 1, perm, K, counts, offsets,
                                   m_off, E, max_mtiles, nullptr, h_hi, h_lo)
              : launch_gemm<2, 64>(Lg, ex, stride, 0, (uint64_t)H * D * 2, H, D, x_hi, x_lo, 1, perm, K, counts, offsets,
                                   m_off, E, max_mtiles, nullptr, h_hi, h_lo);
    if (e != hipSuccess) return e;
    // down: N = D, Kd = H, activation rows = the h planes in list order
    e = small ? launch_gemm<1, 32>(Lw, ex, stride, 2 * (uint64_t)H * D * 2, 0, D, H, h_hi, h_lo, 0, perm, K, counts,
                                   offsets, m_off, E, max_mtiles, y, nullptr, nullptr)
              : launch_gemm<1, 64>(Lw, ex, stride, 2 * (uint64_t)H * D * 2, 0, D, H, h_hi, h_lo, 0, perm, K, counts,
                                   offsets, m_off, E, max_mtiles, y, nullptr, nullptr);
    if (e != hipSuccess) return e;
    if (!combine) return hipSuccess;
    return launch(Lc, combine_rows_kernel, dim3((unsigned)((D + 255) / 256), (unsigned)T), dim3(256), 0,
                  (const float *)y, (const int32_t *)pos_of, weights, K, D, x_inout, moe_out);
}

}  // namespace rbt
