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
//    Tiles: 128 rows x 512 weight rows per block of 8 waves (grouped_gemm_wide_kernel, where the
//    shape has them), 128 or 64 rows x 256 weight rows per block of 16 waves, or 32 x 128 per 8 waves
//    for decode-sized batches; the 64- and 32-row tiles run the reduction in chunks of 64 (128)
//    through a three- or four-stage LDS ring filled by direct HBM -> LDS copies, the 128-row tiles
//    keep their weight operands in registers. 128-row tiles cover the whole list of an expert with
//    up to 128 rows, so its weight tile is streamed by one block once.
//    Tile order (expert, column tile, row tile), split into 8 contiguous ranges, one per XCD (the
//    hardware hands block b to XCD b % 8): the row tiles of a hot expert then share each weight
//    tile in that XCD's L2, and an expert's activation rows are reused across its column tiles.
// 3. combine_rows_kernel: moe[t] = sum_k w[t][k] * y[pos(t,k)] in selection order, x += moe.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "rbt2_internal.h"

namespace rbt {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kDispatchMaxE = 256;
constexpr int kDispRegs = 4;  // 64-pair steps per wave kept in registers by dispatch_kernel (4096 pairs)


// ---------------------------------------------------------------- dispatch (one block, 1024 threads)
// routing [P] with pair p = t*K + k. Outputs: counts[E]; offsets[E+1] (exclusive prefix of counts);
// perm[P]: pair ids grouped by expert, increasing within an expert; pos_of[P]: inverse of perm;
// m_off[E+1]: exclusive prefix of ceil(counts / mt_rows) (the grouped GEMMs' row tiles per expert);
// with m_off2 given, also m_off2[E+1] for 128-row tiles and *choice, the grouped GEMMs' plan: bit 0 the
// tile height (1: 128 rows, 0: mt_rows; tall = 1 forces mt_rows, else 128), bit 1 the slot order of
// the 128-row tiles (column-major when some list is longer than 4x the mean, else expert-major; see
// tile_of). Measured
// on the OLMoE layer at 512 tokens: 128-row tiles beat 64-row ones with uniform routing (209 against
// 262 us per call) and, in column-major order, with +2 on 8 experts' logits (247 against 255 us) and
// +4 on 4 (223 against 231 us); expert-major order keeps the uniform case's activation rows in one
// XCD's L2 per expert (209 against 214 us).
// Wave w owns the pair slice [w*S, (w+1)*S). A: each wave ranks its pairs, 64 at a time, against
// equal experts (ballots over the expert-id bits) and keeps per-expert running counts in its own LDS
// row; a pair's rank inside its wave's slice stays in a register (pos_of holds it past the first
// kDispRegs steps). B: every thread (wave w, expert e) sums the counts of the waves before w, wave 0
// (4 experts per lane) scans the totals into the offsets, and every thread turns its sum into wave
// w's first position for e. C: every pair adds its wave's base. Five barriers in all.
__global__ __launch_bounds__(1024) void dispatch_kernel(const int32_t *__restrict__ routing, int P, int E,
                                                        int32_t *__restrict__ counts, int32_t *__restrict__ offsets,
                                                        int32_t *__restrict__ perm, int32_t *__restrict__ pos_of,
                                                        int32_t *__restrict__ m_off, int mt_rows,
                                                        int32_t *__restrict__ m_off2, int32_t *__restrict__ choice,
                                                        int tall) {
    constexpr int NW = 16;
    __shared__ int s_w[NW][kDispatchMaxE];  // A: running counts per wave; B: each wave's base positions
    __shared__ int s_tot[kDispatchMaxE];    // B: each expert's total, then its first list position
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int S = ((P + NW - 1) / NW + 63) / 64 * 64;  // slice per wave, whole 64-pair steps
    const int base = wv * S, end = min(P, base + S);
    int rv[kDispRegs];  // the first kDispRegs steps' routing, in flight while the counts are cleared
#pragma unroll
    for (int i = 0; i < kDispRegs; ++i) rv[i] = routing[min(base + 64 * i + lane, P - 1)];  // unconditional
    for (int i = tid; i < NW * kDispatchMaxE; i += 1024) (&s_w[0][0])[i] = 0;
    __syncthreads();
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    // one 64-pair step: the rank of each pair among the wave's earlier pairs of its expert
    auto rank_step = [&](int p, int e, bool valid) {
        uint64_t same = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (e >> b) & 1;
            const uint64_t ones = __ballot(bit);
            same &= bit ? ones : ~ones;
        }
        const int before = __popcll(same & below);
        const int cur = valid ? s_w[wv][e] : 0;  // read by every lane before any update (in-order LDS)
        if (valid && (same >> lane) == 1ull) s_w[wv][e] = cur + before + 1;  // last lane of its expert
        return cur + before;
    };
    // the first kDispRegs steps keep expert and rank in registers (all their routing loads issued
    // together, nothing re-read in C); later steps, for more than 16 * 64 * kDispRegs pairs, keep the
    // rank in pos_of and read the routing again
    int ereg[kDispRegs], rreg[kDispRegs];
#pragma unroll
    for (int i = 0; i < kDispRegs; ++i) ereg[i] = base + 64 * i + lane < end ? min(max(rv[i], 0), E - 1) : -1;
#pragma unroll
    for (int i = 0; i < kDispRegs; ++i)
        if (base + 64 * i < end) rreg[i] = rank_step(base + 64 * i + lane, max(ereg[i], 0), ereg[i] >= 0);
    for (int p0 = base + 64 * kDispRegs; p0 < end; p0 += 64) {  // wave-uniform loop
        const int p = p0 + lane;
        const bool valid = p < end;
        const int e = valid ? min(max(routing[p], 0), E - 1) : 0;
        const int rk = rank_step(p, e, valid);
        if (valid) pos_of[p] = rk;
    }
    __syncthreads();
    // B1: thread (wave w, lane l) sums the counts of waves before w for experts l + 64 j (all threads,
    // instead of one wave walking the 16 waves per expert); wave 15 also keeps the totals
    int pre[kDispatchMaxE / 64];
#pragma unroll
    for (int j = 0; j < kDispatchMaxE / 64; ++j) {
        const int e = lane + 64 * j;
        int run = 0;
        if (e < E) {
            for (int w = 0; w < wv; ++w) run += s_w[w][e];
            if (wv == NW - 1) s_tot[e] = run + s_w[NW - 1][e];
        }
        pre[j] = run;
    }
    __syncthreads();
    if (wv == 0) {
        int c[4], mt[4], mt2[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            const int tot = e < E ? s_tot[e] : 0;
            c[i] = tot;
            mt[i] = (tot + mt_rows - 1) / mt_rows;
            mt2[i] = (tot + 127) / 128;
        }
        // a list longer than 4x the mean: the slots go column-major (tile_of) so the long lists' tiles
        // spread over the XCDs
        int cmax = max(max(c[0], c[1]), max(c[2], c[3]));
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) cmax = max(cmax, __shfl_xor(cmax, d, 64));
        const bool skewed = (long long)cmax * E > 4ll * P;
        // exclusive scans across the wave of the lanes' sums (4 experts per lane, ascending)
        int sc = ((c[0] + c[1]) + c[2]) + c[3], sm = ((mt[0] + mt[1]) + mt[2]) + mt[3];
        int sm2 = ((mt2[0] + mt2[1]) + mt2[2]) + mt2[3];
        int ic = sc, im = sm, im2 = sm2;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int uc = __shfl_up(ic, d, 64), um = __shfl_up(im, d, 64), um2 = __shfl_up(im2, d, 64);
            if (lane >= d) {
                ic += uc;
                im += um;
                im2 += um2;
            }
        }
        int oc = ic - sc, om = im - sm, om2 = im2 - sm2;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            if (e < E) {
                counts[e] = c[i];
                offsets[e] = oc;
                m_off[e] = om;
                if (m_off2) m_off2[e] = om2;
                s_tot[e] = oc;  // the expert's first list position
            }
            if (e == E - 1) {
                offsets[E] = oc + c[i];
                m_off[E] = om + mt[i];
                if (m_off2) {
                    m_off2[E] = om2 + mt2[i];
                    *choice = tall == 1 ? 0 : (1 | (skewed ? 2 : 0));  // 64-row tiles: expert-major
                }
            }
            oc += c[i];
            om += mt[i];
            om2 += mt2[i];
        }
    }
    __syncthreads();
    // B3: each wave's first position for each expert
#pragma unroll
    for (int j = 0; j < kDispatchMaxE / 64; ++j) {
        const int e = lane + 64 * j;
        if (e < E) s_w[wv][e] = s_tot[e] + pre[j];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kDispRegs; ++i) {
        const int p = base + 64 * i + lane;
        if (ereg[i] >= 0) {
            const int pos = s_w[wv][ereg[i]] + rreg[i];
            perm[pos] = p;
            pos_of[p] = pos;
        }
    }
    for (int p0 = base + 64 * kDispRegs; p0 < end; p0 += 64) {
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
// The same for data read once (expert weights): a streaming (non-temporal) load.
__device__ __forceinline__ void lds_dma16_stream(const void *g, uint32_t lds_byte) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(lds_byte), "v"(g) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_dma() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Until at most `ahead` stages of n copies each (n = WI .. WI + AI, this wave's copies per stage) are
// outstanding; copies complete in issue order. Both arguments are wave-uniform.
template <int WI, int AI>
__device__ __forceinline__ void wait_stages(int ahead, int n) {
    static_assert(AI <= 2, "copies per stage");
    if (ahead <= 0) {
        wait_dma<0>();
    } else if (ahead == 1) {
        if (n == WI) wait_dma<WI>();
        else if (n == WI + 1) wait_dma<WI + 1>();
        else wait_dma<WI + 2>();
    } else {
        if (n == WI) wait_dma<2 * WI>();
        else if (n == WI + 1) wait_dma<2 * (WI + 1)>();
        else wait_dma<2 * (WI + 2)>();
    }
}

// Tile: ROWS list rows x WROWS weight rows (gate/up: half W1 rows, the same rows of W3; down: W2
// rows), the reduction in chunks that are one ring stage in LDS each; three (four) stages, the copies
// of the next two (three) stages in flight while the MFMAs run on the current one:
//   64 x 256:  256 weight rows x 128 B (k-chunks of 64) + 2 x 64 activation rows x 128 B = 48 KiB
//   32 x 128:  128 weight rows x 256 B (k-chunks of 128) + 2 x 32 activation rows x 256 B = 48 KiB
// A block's throughput is set by the copies it keeps in flight (two stages, ~96 KiB, about 33 GB/s per
// CU whatever the source, weights from HBM or activation rows from L2), so activation copies of row
// groups past the end of the list are not issued (their LDS rows hold stale data, which only reaches
// output rows that are never written).
// (the activation rows: bf16 hi and lo planes). The kernel is bound by its copies: it keeps 90% of
// its time with the MFMAs and operand reads taken out, and a stage takes ~1.45 us whether two or
// three stages are in flight and whether a row is read in 128- or 256-byte runs. At 5.8 TB/s of
// weights it runs at ~94% of what one block per CU streams with plain loads of 32 KiB steps (6.2
// TB/s, measured for 512 and 1024 threads and runs of 128 B to 1 KiB); the LDS ring leaves no room
// for a second block. Copies: 1 KiB each (8 rows of 128 B or 4 of 256 B), 4 weight + 2 activation
// per wave.
constexpr int kGWRows = 256, kGKC = 64;  // the 64-row tile; prefill_supported's shape rules
constexpr int kSmallTileRowsPerExpert = 16;  // mean list rows per expert up to which tiles have 32 rows
template <int ROWS, int WROWS>
struct GTile {
    static constexpr int kWRows = WROWS;                   // weight rows per tile
    static constexpr int kKC = ROWS == 64 ? 64 : 128;      // k per stage
    static constexpr int kRowB = 2 * kKC;                  // bytes of each row per stage
    static constexpr int kGran = kRowB / 16;               // 16-byte granules per row per stage
    static constexpr int kRowsPerCopy = 1024 / kRowB;      // rows one 1 KiB copy covers
    static constexpr int kStages = 3;
    static constexpr int kWBytes = kWRows * kRowB;         // 32 KiB
    static constexpr int kABytes = ROWS * kRowB;
    static constexpr int kStageBytes = kWBytes + 2 * kABytes;
    static constexpr int kWaves = ROWS == 32 ? 8 : 16;    // waves per block (each needs a W1/W3 pair)
    static constexpr int kRG = ROWS / 16;                  // row groups of 16 (one per wave)
    static constexpr int kCH = kWaves / kRG;               // weight-row splits (waves per row group)
    static constexpr int kNB = kWRows / 16 / kCH;          // weight blocks of 16 per wave
    static constexpr int kWI = kWBytes / 1024 / kWaves;    // weight copies per wave per stage
    static constexpr int kACP = kABytes / 1024;            // copies per activation plane
    static constexpr int kAI = 2 * kACP / kWaves;          // activation copies per wave per stage
    static constexpr int kDmaPerWave = kWI + kAI;  // at most: activation copies past the list are skipped
    static_assert(((ROWS == 64 && WROWS == 256) || (ROWS == 32 && WROWS == 128)) &&
                      kStages * kStageBytes <= 160 * 1024 &&
                      kAI * kWaves == 2 * kACP && kWI * kWaves * 1024 == kWBytes && kNB >= 2 && kNB % 2 == 0,
                  "tile shape");
    // Inside a stage, row r's granule g sits at slot swz(r, g) (an involution in g, so the copies can
    // place it by choosing their source granule): the MFMA operand reads (16 consecutive rows at one
    // granule per 16 lanes) then hit 16 distinct bank groups (two rows per 256 bytes of banks for
    // 128-byte rows, one for 256-byte rows).
    __device__ static int swz(int r, int g) { return kRowB == 128 ? g ^ ((r >> 1) & 7) : g ^ (r & 15); }
};

// MATS = 2: h = silu(W1 a) * (W3 a) for a = xb rows gathered through perm (N = H columns, Kd = D),
//           written as bf16 hi/lo planes [P][N] (the next GEMM's activation operand).
// MATS = 1: y = W2 a for a = the h planes in list order (N = D, Kd = H), written as f32 [P][N].
// Waves: w = kRG*ch + rg computes list rows [16 rg, +16) x the ch-th of kCH parts of the tile's weight
// rows (kNB blocks of 16: gate/up W1 blocks (kNB/2) ch .. and the matching W3 blocks; down W2 blocks
// kNB ch ..).
// Requirements (prefill_supported): N % (256 / MATS) == 0, Kd % 64 == 0, 16-byte aligned rows.
// The block's work on tile slot `bid` (the kernels below pass blockIdx.x); ring: the LDS ring of
// STAGES * SBYTES bytes at LDS offset ring0.
// Tile slot tau -> (expert e, column tile jt, row tile il of e's list), with m_off the prefix of the
// experts' row tiles and nt column tiles. Expert-major (colmajor 0): e's tiles are consecutive, so an
// expert's column tiles share its activation rows in one XCD's L2. Column-major (1): tau = jc * M + rt
// over the M row tiles of all experts (expert e's column tile (jc + e) mod nt), so each XCD's
// contiguous share of the slots spans every expert's row tiles for a few column tiles and a few long
// lists load all XCDs alike. Either way an expert's row tiles of one column tile (one weight tile) are
// consecutive, on one XCD.
__device__ __forceinline__ void tile_of(int tau, const int32_t *__restrict__ m_off, int E, int nt, int colmajor,
                                        int *e_out, int *jt_out, int *il_out) {
    const int M = m_off[E];
    const int jc = colmajor ? tau / M : 0, key = colmajor ? tau - jc * M : tau, scale = colmajor ? 1 : nt;
    int lo = 0, hi = E - 1;  // the last e with m_off[e] * scale <= key
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (m_off[mid] * scale <= key)
            lo = mid;
        else
            hi = mid - 1;
    }
    const int e = lo;
    if (colmajor) {
        // diagonal: slot column jc holds column tile (jc + e) mod nt of expert e, so the tiles that run
        // together on one XCD are not all the same column tile of many experts (the experts' blobs are
        // a multiple of 4 MiB apart, so those would stream congruent address windows at the same time)
        *jt_out = jc + e % nt < nt ? jc + e % nt : jc + e % nt - nt;
        *il_out = key - m_off[e];
    } else {
        const int me = m_off[e + 1] - m_off[e], local = key - m_off[e] * nt;
        *jt_out = local / me;
        *il_out = local - *jt_out * me;
    }
    *e_out = e;
}

template <int MATS, int ROWS, int WROWS>
__device__ __forceinline__ void gemm_lds_tile(
    uint8_t *ring, uint32_t ring0, unsigned bid, const uint8_t *__restrict__ experts, uint64_t stride, uint64_t w_off,
    uint64_t w3_off, int N, int Kd, const uint16_t *__restrict__ a_hi, const uint16_t *__restrict__ a_lo, int gather,
    const int32_t *__restrict__ perm, int topk, const int32_t *__restrict__ counts, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ m_off, int E, int colmajor, float *__restrict__ out_f32, uint16_t *__restrict__ out_hi,
    uint16_t *__restrict__ out_lo) {
    using TS = GTile<ROWS, WROWS>;
    constexpr int NTILE = WROWS / MATS;  // output columns per tile
    constexpr int STAGES = TS::kStages, SBYTES = TS::kStageBytes, NB = TS::kNB, AI = TS::kAI, WI = TS::kWI;
    constexpr int ROWB = TS::kRowB, GRAN = TS::kGran, RPC = TS::kRowsPerCopy, WBYTES = TS::kWBytes;

    // w in a scalar register: the branches on it below are then wave-uniform jumps, not exec masks
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), rg = w % TS::kRG,
              ch = w / TS::kRG;
    const int ntiles_n = N / NTILE;
    const int total = m_off[E] * ntiles_n;
    const int range = (total + 7) >> 3;
    const int slot = (int)(bid >> 3);
    const int tau = (int)(bid & 7) * range + slot;
    if (slot >= range || tau >= total) return;
    int e, jt, il;
    tile_of(tau, m_off, E, ntiles_n, colmajor, &e, &jt, &il);
    const int row0 = offsets[e] + il * ROWS;
    const int rows = __builtin_amdgcn_readfirstlane(min(ROWS, counts[e] - il * ROWS));  // uniform: scalar branches below
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
    bool aon[AI];  // wave-uniform: the copy covers at least one row of the list
    int ncopy = WI;  // copies this wave issues per stage
#pragma unroll
    for (int i = 0; i < AI; ++i) {
        // copy u: plane u / kACP, rows RPC * (u % kACP) ..
        const int u = AI * w + i, plane = u / TS::kACP, r = RPC * (u % TS::kACP) + lane / GRAN,
                  g = TS::swz(r, lane % GRAN);
        aon[i] = RPC * (u % TS::kACP) < rows;
        ncopy += aon[i] ? 1 : 0;
        const int lr = row0 + (r < rows ? r : 0);  // rows past the list (in a copy that is issued) re-read its first row
        const size_t arow = gather ? (size_t)(perm[lr] / topk) : (size_t)lr;
        asrc[i] = reinterpret_cast<const uint8_t *>(plane ? a_lo : a_hi) + arow * rowb + 16 * g;
    }
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
            lds_dma16_stream(wsrc[i] + kb, __builtin_amdgcn_readfirstlane(sb + (WI * w + i) * 1024));
#pragma unroll
        for (int i = 0; i < AI; ++i)
            if (aon[i]) lds_dma16(asrc[i] + kb, __builtin_amdgcn_readfirstlane(sb + WBYTES + (AI * w + i) * 1024));
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
        wait_stages<WI, AI>(ahead, ncopy);
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

template <int MATS, int ROWS, int WROWS>
__global__ __launch_bounds__((64 * GTile<ROWS, WROWS>::kWaves), 1) void grouped_gemm_kernel(
    const uint8_t *__restrict__ experts, uint64_t stride, uint64_t w_off, uint64_t w3_off, int N, int Kd,
    const uint16_t *__restrict__ a_hi, const uint16_t *__restrict__ a_lo, int gather, const int32_t *__restrict__ perm,
    int topk, const int32_t *__restrict__ counts, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ m_off, int E, float *__restrict__ out_f32, uint16_t *__restrict__ out_hi,
    uint16_t *__restrict__ out_lo) {
    __shared__ __align__(1024) uint8_t ring[GTile<ROWS, WROWS>::kStages * GTile<ROWS, WROWS>::kStageBytes];
    gemm_lds_tile<MATS, ROWS, WROWS>(ring, (uint32_t)(uintptr_t)ring, blockIdx.x, experts, stride, w_off, w3_off, N,
                                     Kd, a_hi, a_lo, gather, perm, topk, counts, offsets, m_off, E, 0, out_f32, out_hi,
                                     out_lo);
}

// ---------------------------------------------------------------- grouped GEMM, 128-row tiles
// Where the dispatch kernel picks them, a tile holds up to 128 list rows and 256 weight rows
// (gate/up: 128 W1 rows and the same 128 W3 rows; down: 256 W2 rows), one block of 16 waves per tile,
// so a weight tile is streamed once for up to 128 rows. Wave W owns the 16 weight rows 16 W .. of the
// tile (gate/up: W1 for W < 8, W3 for W >= 8; the two halves meet through LDS in the epilogue) and
// loads their MFMA operands from HBM straight into registers three 64-wide k-steps ahead of its MFMAs;
// the activation rows, which every wave multiplies, are loaded four k-steps ahead into registers and
// pass through a two-stage LDS ring. The row groups past the end of the list are not multiplied.
// Every wait is the compiler's own. Same operands, accumulation order and epilogue arithmetic as
// grouped_gemm_kernel.
constexpr int kWrRows = 128, kWrKC = 64, kWrAhead = 3, kWrWaves = 16;
// buffer resources of the activation planes: records (bytes) past any valid offset, and the config
// word of a raw 32-bit-format buffer
constexpr int kWrBufRecords = 0x7FFF0000, kBufConfig = 0x00020000;
// whole tiles of output columns, and k-steps a multiple of the kWrAhead + 1 register slots
constexpr bool gemm_wr_supported(int mats, int N, int Kd) {
    return N % (mats == 2 ? 128 : 256) == 0 && Kd % (kWrKC * (kWrAhead + 1)) == 0;
}

// The tiled copy of a layer's experts (prefill_layout_kernel): per expert (3 H D bf16, the size of its
// blob) the gate/up part, then the down part, each [tile][k-chunk of 64][row block W 0..15][half s
// 0..1][lane 0..63][16 bytes]: one tile's k-chunk is 32 KiB in the order gemm_wr_tile's
// waves load it (1 KiB per load instruction), so each step of a tile reads contiguous memory (the
// row-major blob spreads a step over 256 rows 4 KiB apart, which holds HBM to ~5 TB/s; contiguous
// 32 KiB steps stream at ~6.9 TB/s). Lane l of block W holds tile row r = 16 W + (l & 15) at
// k = 64 chunk + 32 s + 8 (l >> 4); gate/up tile jt: r < 128 -> W1 row 128 jt + r, else W3 row
// 128 jt + r - 128; down tile jt: W2 row 256 jt + r.
constexpr int kTiledChunk = 32768;
__global__ __launch_bounds__(256) void prefill_layout_kernel(const uint8_t *__restrict__ experts, uint64_t stride,
                                                            int D, int H, uint8_t *__restrict__ dst,
                                                            uint64_t units_per_expert) {
    const uint64_t u = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int e = (int)blockIdx.y;
    if (u >= units_per_expert) return;
    const uint64_t gu_units = (uint64_t)H * D / 4;  // 16-byte units of the gate/up part (2 H D bf16)
    const bool down = u >= gu_units;
    const uint64_t v = down ? u - gu_units : u;
    const int Kd = down ? H : D;
    const uint64_t ch = v / (kTiledChunk / 16);
    const int t = (int)(v % (kTiledChunk / 16)), W = t / 128, s = (t / 64) % 2, l = t % 64;
    const int r = 16 * W + (l & 15);
    const int nch = Kd / kWrKC;
    const int jt = (int)(ch / nch), c = (int)(ch % nch);
    const int k = kWrKC * c + 32 * s + 8 * (l >> 4);
    const uint8_t *src = experts + (size_t)e * stride;
    size_t off;
    if (!down)
        off = (r >= 128 ? (size_t)H * D * 2 : 0) + ((size_t)(128 * jt + (r & 127)) * D + k) * 2;
    else
        off = 2 * (size_t)H * D * 2 + ((size_t)(256 * jt + r) * H + k) * 2;
    *reinterpret_cast<u32x4 *>(dst + (size_t)e * units_per_expert * 16 + u * 16) =
        *reinterpret_cast<const u32x4 *>(src + off);
}

// The block's work on 128-row tile slot `bid`; smem: 2 * 2 * ABYTES bytes of LDS (the ring).
template <int MATS, bool BLOB>
__device__ __forceinline__ void gemm_wr_tile(
    uint8_t *smem, unsigned bid, const uint8_t *__restrict__ experts, uint64_t stride, uint64_t w_off, uint64_t w3_off,
    int N, int Kd, const uint16_t *__restrict__ a_hi, const uint16_t *__restrict__ a_lo, int gather,
    const int32_t *__restrict__ perm, int topk, const int32_t *__restrict__ counts, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ m_off, int E, int colmajor, float *__restrict__ out_f32, uint16_t *__restrict__ out_hi,
    uint16_t *__restrict__ out_lo, const uint8_t *__restrict__ tiled, uint64_t tiled_stride, uint64_t tiled_off) {
    constexpr int NT = 64 * kWrWaves;             // threads
    constexpr int NTILE = MATS == 2 ? 128 : 256;  // output columns per tile
    constexpr int RG = kWrRows / 16;              // row groups of 16
    constexpr int ROWB = 2 * kWrKC;               // bytes of an activation row per k-step
    constexpr int ABYTES = kWrRows * ROWB;        // one plane of a k-step, 16 KiB
    constexpr int AU = 2 * ABYTES / 16 / NT;      // 16-byte activation units per thread per k-step
    constexpr int SLOTS = kWrAhead + 1;           // register sets of weights and of activations
    static_assert(AU * NT * 16 == 2 * ABYTES && 2 * 2 * ABYTES >= (kWrWaves / 2) * RG * 64 * 16, "ring sizes");
    uint8_t(*ring)[2 * ABYTES] = reinterpret_cast<uint8_t(*)[2 * ABYTES]>(smem);
    const int tid = threadIdx.x, lane = tid & 63, W = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ntiles_n = N / NTILE;
    const int total = m_off[E] * ntiles_n;
    const int range = (total + 7) >> 3;
    const int slot = (int)(bid >> 3);
    const int tau = (int)(bid & 7) * range + slot;
    if (slot >= range || tau >= total) return;
    int e, jt, il;
    tile_of(tau, m_off, E, ntiles_n, colmajor, &e, &jt, &il);
    const int row0 = offsets[e] + il * kWrRows;
    const int rows = __builtin_amdgcn_readfirstlane(min(kWrRows, counts[e] - il * kWrRows));
    const int n0 = jt * NTILE;
    const size_t rowb = (size_t)Kd * 2;  // bytes per weight / activation-plane row
    const int nch = Kd / kWrKC;
    // Step c reads k-chunk (c + rot) mod nch, rot a function of the weight tile (see grouped_gemm_kernel)
    const int rot = (e * ntiles_n + jt) % nch;
    auto cidx = [&](int c) { return c + rot < nch ? c + rot : c + rot - nch; };

    // weight operands of this lane: tile row 16 W + (lane & 15), k offset 8 * (lane >> 4) in each 32-wide
    // half s of a 64-wide k-chunk cc, at wp + cc * wck + s * wsb (blobs: the row itself; tiled copy: the
    // tile's contiguous 32 KiB chunks)
    const uint8_t *wp;
    size_t wck, wsb;
    if constexpr (!BLOB) {
        wp = tiled + (size_t)e * tiled_stride + tiled_off + (size_t)jt * nch * kTiledChunk + (size_t)(2 * W) * 1024 +
             16 * lane;
        wck = kTiledChunk;
        wsb = 1024;
    } else {
        // whole 128-byte lines per load (blob_operands): slot s of the step holds rows 8 s .. 8 s + 7
        const int tr = 16 * W + (lane & 7);
        const uint8_t *base = experts + (size_t)e * stride + (MATS == 2 && W >= 8 ? w3_off : w_off);
        const int wr = MATS == 2 ? n0 + (tr & 127) : n0 + tr;
        wp = base + (size_t)wr * rowb + 16 * blob_chunk(lane);
        wck = ROWB;
        wsb = 8 * rowb;
    }
    // activation units of this thread: u = tid + NT i -> plane i (u / (ABYTES / 16)), row, granule. They
    // are buffer loads: a row past the end of the list gets an offset past the buffer's end, which returns
    // zeros without a memory request (every request counts against the CU's in-flight limit, which the
    // weight stream needs), and no branch (which keeps the compiler's waits exact). The buffers start at
    // the tile's first row (list order) or the plane (gathered rows; the planes are below 2 GiB).
    const size_t base_row = gather ? 0 : (size_t)row0;
    const __amdgpu_buffer_rsrc_t rs[2] = {
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a_hi) + base_row * Kd, 0, kWrBufRecords, kBufConfig),
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a_lo) + base_row * Kd, 0, kWrBufRecords, kBufConfig)};
    uint32_t aoff[AU], adst[AU];
#pragma unroll
    for (int i = 0; i < AU; ++i) {
        const int u = tid + NT * i, r = (u % (ABYTES / 16)) / (ROWB / 16), g = u % (ROWB / 16);
        static_assert(NT == ABYTES / 16, "one plane per unit index i");
        const int lr = row0 + (r < rows ? r : 0);
        const size_t arow = gather ? (size_t)(perm[lr] / topk) : (size_t)lr;
        aoff[i] = r < rows ? (uint32_t)((arow - base_row) * rowb + 16 * g) : (uint32_t)kWrBufRecords;
        adst[i] = (uint32_t)(i * ABYTES + r * ROWB + 16 * (g ^ ((r >> 1) & 7)));
    }
    // register sets: activations of k-step x in aset[x % SLOTS] (loaded four steps ahead, stored to the
    // LDS ring one step ahead), weights of k-step x in wv[x % SLOTS] (loaded three steps ahead)
    u32x4 aset[SLOTS][AU];
    u32x4 wv[SLOTS][2];  // [slot][32-wide half]
    auto load_a = [&](u32x4 (&dst)[AU], int c) {
        const uint32_t kb = (uint32_t)(cidx(c) * ROWB);
#pragma unroll
        for (int i = 0; i < AU; ++i) dst[i] = __builtin_amdgcn_raw_buffer_load_b128(rs[i], (int)(aoff[i] + kb), 0, 0);
    };
    auto store_a = [&](const u32x4 (&src)[AU], int buf) {
#pragma unroll
        for (int i = 0; i < AU; ++i) *reinterpret_cast<u32x4 *>(&ring[buf][adst[i]]) = src[i];
    };
    auto load_w = [&](u32x4 (&dst)[2], int c) {
        const size_t kb = (size_t)cidx(c) * wck;
#pragma unroll
        for (int s = 0; s < 2; ++s) dst[s] = ld_stream_u4(wp + kb + s * wsb);
    };

    f32x4 acc[RG];
#pragma unroll
    for (int q = 0; q < RG; ++q) acc[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // k-step c on slot J = c % SLOTS; LAST: the tile's final SLOTS steps. nch is a multiple of SLOTS
    // (gemm_wr_supported), so slots and the remaining loads are compile-time constants. Loads complete in
    // issue order and a wait covers everything issued before its load, so each step stores the next
    // step's activations, then issues activations before weights: the store at step c then waits for
    // loads up to step c - 3's activations, never for weights still three steps from use.
    auto step = [&](auto jc, auto lastc, int c) {
        constexpr int J = decltype(jc)::value;
        constexpr bool LAST = decltype(lastc)::value;
        if constexpr (!LAST || J + 1 < SLOTS) store_a(aset[(J + 1) % SLOTS], (c + 1) & 1);  // buffer of step c - 1
        if constexpr (!LAST) load_a(aset[J], c + SLOTS);
        if constexpr (!LAST || J + kWrAhead < SLOTS) load_w(wv[(J + kWrAhead) % SLOTS], c + kWrAhead);
        const uint8_t *st = ring[c & 1];
        if constexpr (BLOB) blob_operands(wv[J][0], wv[J][1]);
#pragma unroll
        for (int q = 0; q < RG; ++q) {
            if (16 * q < rows) {  // wave-uniform: the row group holds list entries
                const int r = 16 * q + (lane & 15);
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    const int g = 4 * s2 + (lane >> 4);
                    const int off = r * ROWB + 16 * (g ^ ((r >> 1) & 7));
                    const bf16x8 ah = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(st + off));
                    const bf16x8 al = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(st + ABYTES + off));
                    const bf16x8 bv = __builtin_bit_cast(bf16x8, wv[J][s2]);
                    acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bv, acc[q], 0, 0, 0);
                    acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bv, acc[q], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    static_assert(SLOTS == 4 && kWrAhead == 3, "one step call per slot below");
    // prologue, in the steady state's order: activations and weights of steps 0..2, activations of 3
    load_a(aset[0], 0);
    load_w(wv[0], 0);
    load_a(aset[1], 1);
    load_w(wv[1], 1);
    load_a(aset[2], 2);
    load_w(wv[2], 2);
    load_a(aset[3], 3);
    store_a(aset[0], 0);
    __syncthreads();
    int c0 = 0;
    for (; c0 + SLOTS < nch; c0 += SLOTS) {
        step(I0{}, std::false_type{}, c0);
        step(I1{}, std::false_type{}, c0 + 1);
        step(I2{}, std::false_type{}, c0 + 2);
        step(I3{}, std::false_type{}, c0 + 3);
    }
    step(I0{}, std::true_type{}, c0);
    step(I1{}, std::true_type{}, c0 + 1);
    step(I2{}, std::true_type{}, c0 + 2);
    step(I3{}, std::true_type{}, c0 + 3);

    // epilogue: acc[q] lane holds tile row 16 W + (lane % 16) for list rows 16 q + 4*(lane/16) + i. Gate/up:
    // the W3 waves hand their sums to the W1 wave of the same columns through the (idle) ring.
    if constexpr (MATS == 2) {
        f32x4 *xch = reinterpret_cast<f32x4 *>(&ring[0][0]);  // [W - 8][q][lane]
        if (W >= kWrWaves / 2) {
#pragma unroll
            for (int q = 0; q < RG; ++q)
                if (16 * q < rows) xch[((W - kWrWaves / 2) * RG + q) * 64 + lane] = acc[q];
        }
        __syncthreads();
        if (W >= kWrWaves / 2) return;
#pragma unroll
        for (int q = 0; q < RG; ++q) {
            if (16 * q >= rows) break;
            const f32x4 up = xch[(W * RG + q) * 64 + lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 16 * q + 4 * (lane >> 4) + i;
                if (r >= rows) continue;
                const float g = acc[q][i], u = up[i];
                const float v = (g / (1.0f + expf(-g))) * u;  // silu(g) * u, rabbit2.c:535-537
                const uint32_t hb = f32_to_bf16_rne(v);
                const uint32_t lb = f32_to_bf16_rne(v - __uint_as_float(hb << 16));
                const size_t o = (size_t)(row0 + r) * N + n0 + 16 * W + (lane & 15);
                out_hi[o] = (uint16_t)hb;
                out_lo[o] = (uint16_t)lb;
            }
        }
    } else {
#pragma unroll
        for (int q = 0; q < RG; ++q) {
            if (16 * q >= rows) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 16 * q + 4 * (lane >> 4) + i;
                if (r >= rows) continue;
                out_f32[(size_t)(row0 + r) * N + n0 + 16 * W + (lane & 15)] = acc[q][i];
            }
        }
    }
}

// The grouped GEMM of the 64- and 128-row tiles in one launch: the dispatch kernel chose the tile
// height and slot order from the histogram (*choice bit 0: 128-row tiles over m_off128, else 64-row
// tiles over m_off64; bit 1: column-major slot order, see tile_of), and every block runs that path on
// its tile slot. Both paths take 16 waves; the LDS is the larger
// ring (the 64-row tiles').
constexpr int kSelLds = GTile<64, 256>::kStages * GTile<64, 256>::kStageBytes;
static_assert(kSelLds >= 2 * 2 * kWrRows * 2 * kWrKC && GTile<64, 256>::kWaves == kWrWaves, "shared launch shape");
template <int MATS, bool BLOB>
__global__ __launch_bounds__(64 * kWrWaves, 1) void grouped_gemm_sel_kernel(
    const uint8_t *__restrict__ experts, uint64_t stride, uint64_t w_off, uint64_t w3_off, int N, int Kd,
    const uint16_t *__restrict__ a_hi, const uint16_t *__restrict__ a_lo, int gather, const int32_t *__restrict__ perm,
    int topk, const int32_t *__restrict__ counts, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ m_off64, const int32_t *__restrict__ m_off128, const int32_t *__restrict__ choice,
    int E, float *__restrict__ out_f32, uint16_t *__restrict__ out_hi, uint16_t *__restrict__ out_lo,
    const uint8_t *__restrict__ tiled, uint64_t tiled_stride, uint64_t tiled_off) {
    __shared__ __align__(1024) uint8_t smem[kSelLds];
    const int plan = __builtin_amdgcn_readfirstlane(*choice), colmajor = plan >> 1;
    if (plan & 1)
        gemm_wr_tile<MATS, BLOB>(smem, blockIdx.x, experts, stride, w_off, w3_off, N, Kd, a_hi, a_lo, gather, perm, topk,
                           counts, offsets, m_off128, E, colmajor, out_f32, out_hi, out_lo, tiled, tiled_stride,
                           tiled_off);
    else
        gemm_lds_tile<MATS, 64, 256>(smem, (uint32_t)(uintptr_t)smem, blockIdx.x, experts, stride, w_off, w3_off, N,
                                     Kd, a_hi, a_lo, gather, perm, topk, counts, offsets, m_off64, E, colmajor,
                                     out_f32, out_hi, out_lo);
}

// ---------------------------------------------------------------- grouped GEMM, wide 128-row tiles
// The 128-row tile twice as wide: 512 weight rows (gate/up: 256 W1 rows and the same 256 W3 rows; down:
// 512 W2 rows), so each activation row read from L2 serves twice the weight bytes. A CU moves its
// bytes at a bounded rate whatever their source, and the 256-row tile reads as many activation bytes
// as weight bytes, so this halves the activation share of the traffic. Eight waves of 256 registers:
// wave W owns weight rows 64 W .. 64 W + 63 as four 16-row column groups (gate/up: W1 for W < 4, W3 for
// W >= 4); accumulators [8 row groups][4 column groups]; weights one 64-wide k-step ahead in
// registers, activations two k-steps ahead in registers and one ahead in a two-stage LDS ring. Same
// operands and products per output element as gemm_wr_tile (k-chunks of 64, each as two 32-wide
// halves, hi then lo); the chunks are rotated per wide tile, so sums agree within rounding.
constexpr int kWdWaves = 8, kWdGroups = 4;
constexpr bool gemm_wide_supported(int mats, int N, int Kd) {
    return N % (mats == 2 ? 256 : 512) == 0 && Kd % (2 * kWrKC) == 0;
}

template <int MATS, bool BLOB>
__global__ __launch_bounds__(64 * kWdWaves, 1) void grouped_gemm_wide_kernel(
    const uint8_t *__restrict__ experts, uint64_t stride, uint64_t w_off, uint64_t w3_off, int N, int Kd,
    const uint16_t *__restrict__ a_hi, const uint16_t *__restrict__ a_lo, int gather, const int32_t *__restrict__ perm,
    int topk, const int32_t *__restrict__ counts, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ m_off, const int32_t *__restrict__ choice, int E, float *__restrict__ out_f32,
    uint16_t *__restrict__ out_hi, uint16_t *__restrict__ out_lo, const uint8_t *__restrict__ tiled,
    uint64_t tiled_stride, uint64_t tiled_off) {
    constexpr int NT = 64 * kWdWaves;              // threads
    constexpr int NTILE = MATS == 2 ? 256 : 512;   // output columns per tile
    constexpr int RG = kWrRows / 16;               // row groups of 16
    constexpr int ROWB = 2 * kWrKC;                // bytes of an activation row per k-step
    constexpr int ABYTES = kWrRows * ROWB;         // one plane of a k-step, 16 KiB
    constexpr int AU = 2 * ABYTES / 16 / NT;       // 16-byte activation units per thread per k-step (4)
    constexpr int XBYTES = kWdWaves * (RG / 2) * kWdGroups * 64 * 16;  // gate/up epilogue exchange, 128 KiB
    constexpr int LDSB = MATS == 2 ? XBYTES : 2 * 2 * ABYTES;
    static_assert(AU * NT * 16 == 2 * ABYTES && LDSB >= 2 * 2 * ABYTES, "ring sizes");
    __shared__ __align__(1024) uint8_t smem[LDSB];
    uint8_t(*ring)[2 * ABYTES] = reinterpret_cast<uint8_t(*)[2 * ABYTES]>(smem);
    const int tid = threadIdx.x, lane = tid & 63, W = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int colmajor = (__builtin_amdgcn_readfirstlane(*choice) >> 1) & 1;
    const unsigned bid = blockIdx.x;
    const int ntiles_n = N / NTILE;
    const int total = m_off[E] * ntiles_n;
    const int range = (total + 7) >> 3;
    const int slot = (int)(bid >> 3);
    const int tau = (int)(bid & 7) * range + slot;
    if (slot >= range || tau >= total) return;
    int e, jt, il;
    tile_of(tau, m_off, E, ntiles_n, colmajor, &e, &jt, &il);
    const int row0 = offsets[e] + il * kWrRows;
    const int rows = __builtin_amdgcn_readfirstlane(min(kWrRows, counts[e] - il * kWrRows));
    const int n0 = jt * NTILE;
    const size_t rowb = (size_t)Kd * 2;  // bytes per weight / activation-plane row
    const int nch = Kd / kWrKC;
    // step c reads k-chunk (c + rot) mod nch, rot a function of the weight tile and the same for the
    // whole block (every wave stages the step's activation chunk for all of them). Consecutive experts
    // take consecutive rotations and column tiles nch / ntiles_n apart, so the weight tiles that run
    // together on one XCD (a few experts' column tiles, or one column tile of many experts) start at
    // different k-chunks: their row-major lines then spread over the L2 sets and DRAM channels that a
    // k-window maps to (e * ntiles_n + jt left every expert of a column tile on nch / ntiles_n values).
    const int rot = (e + jt * max(1, nch / ntiles_n)) % nch;
    auto cidx = [&](int c) { return c + rot < nch ? c + rot : c + rot - nch; };
    const int jn = 2 * jt + (MATS == 2 ? ((W & 3) >> 1) : (W >> 2));  // the 256-row tile of this wave's rows

    // weight operands of this lane, column group g: tile row 64 W + 16 g + (lane & 15), k offset
    // 8 * (lane >> 4) in each 32-wide half s of a 64-wide k-chunk cc, at wp + g * wg + cc * wck + s * wsb
    const uint8_t *wp;
    size_t wck, wsb, wg;
    if constexpr (!BLOB) {
        // row block of the 256-row tile jn (tiled copy order, see prefill_layout_kernel)
        const int wn = MATS == 2 ? (W >= 4 ? 8 : 0) + 4 * (W & 1) : 4 * (W & 3);
        wp = tiled + (size_t)e * tiled_stride + tiled_off + (size_t)jn * nch * kTiledChunk + (size_t)(2 * wn) * 1024 +
             16 * lane;
        wck = kTiledChunk;
        wsb = 1024;
        wg = 2048;
    } else {
        // whole 128-byte lines per load (blob_operands): slot s2 of group g holds rows 8 s2 .. 8 s2 + 7
        const uint8_t *base = experts + (size_t)e * stride + (MATS == 2 && W >= 4 ? w3_off : w_off);
        const int wr = n0 + (MATS == 2 ? 64 * (W & 3) : 64 * W) + (lane & 7);
        wp = base + (size_t)wr * rowb + 16 * blob_chunk(lane);
        wck = ROWB;
        wsb = 8 * rowb;
        wg = 16 * rowb;
    }
    const size_t base_row = gather ? 0 : (size_t)row0;
    const __amdgpu_buffer_rsrc_t rs[2] = {
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a_hi) + base_row * Kd, 0, kWrBufRecords, kBufConfig),
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a_lo) + base_row * Kd, 0, kWrBufRecords, kBufConfig)};
    uint32_t aoff[AU], adst[AU];
#pragma unroll
    for (int i = 0; i < AU; ++i) {
        const int u = tid + NT * i, pl = u / (ABYTES / 16), r = (u % (ABYTES / 16)) / (ROWB / 16), g = u % (ROWB / 16);
        const int lr = row0 + (r < rows ? r : 0);
        const size_t arow = gather ? (size_t)(perm[lr] / topk) : (size_t)lr;
        aoff[i] = r < rows ? (uint32_t)((arow - base_row) * rowb + 16 * g) : (uint32_t)kWrBufRecords;
        adst[i] = (uint32_t)(pl * ABYTES + r * ROWB + 16 * (g ^ ((r >> 1) & 7)));
    }
    static_assert(2 * (ABYTES / 16) == AU * NT && (ABYTES / 16) % NT == 0, "unit i's plane is i / (AU / 2)");
    u32x4 aset[2][AU];
    u32x4 wv[2][kWdGroups][2];  // [slot][column group][32-wide half]
    auto load_a = [&](u32x4 (&dst)[AU], int c) {
        const uint32_t kb = (uint32_t)(cidx(c) * ROWB);
#pragma unroll
        for (int i = 0; i < AU; ++i)
            dst[i] = __builtin_amdgcn_raw_buffer_load_b128(rs[i / (AU / 2)], (int)(aoff[i] + kb), 0, 0);
    };
    auto store_a = [&](const u32x4 (&src)[AU], int buf) {
#pragma unroll
        for (int i = 0; i < AU; ++i) *reinterpret_cast<u32x4 *>(&ring[buf][adst[i]]) = src[i];
    };
    auto load_w = [&](u32x4 (&dst)[kWdGroups][2], int c) {
        const size_t kb = (size_t)cidx(c) * wck;
#pragma unroll
        for (int g = 0; g < kWdGroups; ++g)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) dst[g][s2] = ld_stream_u4(wp + g * wg + kb + s2 * wsb);
    };

    f32x4 acc[RG][kWdGroups];
#pragma unroll
    for (int q = 0; q < RG; ++q)
#pragma unroll
        for (int g = 0; g < kWdGroups; ++g) acc[q][g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // k-step c on slot J = c % 2; LAST: the tile's final two steps (nch is even). Each step stores the
    // next step's activations, issues activations (two steps ahead) before weights (one step ahead),
    // so the store waits for activations issued a step earlier, never for the weights in flight.
    auto step = [&](auto jc, auto lastc, int c) {
        constexpr int J = decltype(jc)::value;
        constexpr bool LAST = decltype(lastc)::value;
        if constexpr (!LAST || J == 0) store_a(aset[J ^ 1], (c + 1) & 1);
        if constexpr (!LAST) load_a(aset[J], c + 2);
        if constexpr (!LAST || J == 0) load_w(wv[J ^ 1], c + 1);
        const uint8_t *st = ring[c & 1];
        if constexpr (BLOB) {
#pragma unroll
            for (int g = 0; g < kWdGroups; ++g) blob_operands(wv[J][g][0], wv[J][g][1]);
        }
#pragma unroll
        for (int q = 0; q < RG; ++q) {
            if (16 * q < rows) {  // wave-uniform: the row group holds list entries
                const int r = 16 * q + (lane & 15);
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    const int g8 = 4 * s2 + (lane >> 4);
                    const int off = r * ROWB + 16 * (g8 ^ ((r >> 1) & 7));
                    const bf16x8 ah = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(st + off));
                    const bf16x8 al = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(st + ABYTES + off));
#pragma unroll
                    for (int g = 0; g < kWdGroups; ++g) {
                        const bf16x8 bv = __builtin_bit_cast(bf16x8, wv[J][g][s2]);
                        acc[q][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bv, acc[q][g], 0, 0, 0);
                        acc[q][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bv, acc[q][g], 0, 0, 0);
                    }
                }
            }
        }
        __syncthreads();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // prologue, in the steady state's order: activations of steps 0 and 1, weights of step 0
    load_a(aset[0], 0);
    load_w(wv[0], 0);
    load_a(aset[1], 1);
    store_a(aset[0], 0);
    __syncthreads();
    int c0 = 0;
    for (; c0 + 2 < nch; c0 += 2) {
        step(I0{}, std::false_type{}, c0);
        step(I1{}, std::false_type{}, c0 + 1);
    }
    step(I0{}, std::true_type{}, c0);
    step(I1{}, std::true_type{}, c0 + 1);

    // epilogue: acc[q][g] lane holds tile row 64 W + 16 g + (lane % 16) for list rows 16 q + 4 (lane / 16) + i
    if constexpr (MATS == 2) {
        // waves W and W + 4 hold the gate (W1) and up (W3) sums of the same columns; each computes the
        // SwiGLU of half the row groups (W: 0-3, W + 4: 4-7) and hands the partner the other half
        // through LDS, so all eight waves share the exp / divide work
        constexpr int HQ = RG / 2;
        f32x4 *xch = reinterpret_cast<f32x4 *>(smem);  // [wave][HQ][group][lane]
        const bool upw = W >= kWdWaves / 2;  // wave-uniform: each branch below indexes acc by constants
        const int partner = upw ? W - kWdWaves / 2 : W + kWdWaves / 2;
        auto send = [&](auto qc) {
            constexpr int QS = decltype(qc)::value;
#pragma unroll
            for (int qq = 0; qq < HQ; ++qq)
                if (16 * (QS + qq) < rows)
#pragma unroll
                    for (int g = 0; g < kWdGroups; ++g)
                        xch[((W * HQ + qq) * kWdGroups + g) * 64 + lane] = acc[QS + qq][g];
        };
        auto finish = [&](auto qc, auto upc) {
            constexpr int QM = decltype(qc)::value;
            constexpr bool UP = decltype(upc)::value;
#pragma unroll
            for (int qq = 0; qq < HQ; ++qq) {
                const int q = QM + qq;
                if (16 * q >= rows) break;
#pragma unroll
                for (int g = 0; g < kWdGroups; ++g) {
                    const f32x4 other = xch[((partner * HQ + qq) * kWdGroups + g) * 64 + lane];
                    const f32x4 gv = UP ? other : acc[q][g], uv = UP ? acc[q][g] : other;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int r = 16 * q + 4 * (lane >> 4) + i;
                        if (r >= rows) continue;
                        const float gg = gv[i], u = uv[i];
                        const float v = (gg / (1.0f + expf(-gg))) * u;  // silu(g) * u, rabbit2.c:535-537
                        const uint32_t hb = f32_to_bf16_rne(v);
                        const uint32_t lb = f32_to_bf16_rne(v - __uint_as_float(hb << 16));
                        const size_t o = (size_t)(row0 + r) * N + n0 + 64 * (W & 3) + 16 * g + (lane & 15);
                        out_hi[o] = (uint16_t)hb;
                        out_lo[o] = (uint16_t)lb;
                    }
                }
            }
        };
        using IH = std::integral_constant<int, HQ>;
        if (upw)
            send(I0{});
        else
            send(IH{});
        __syncthreads();
        if (upw)
            finish(IH{}, std::true_type{});
        else
            finish(I0{}, std::false_type{});
    } else {
#pragma unroll
        for (int q = 0; q < RG; ++q) {
            if (16 * q >= rows) break;
#pragma unroll
            for (int g = 0; g < kWdGroups; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 16 * q + 4 * (lane >> 4) + i;
                    if (r >= rows) continue;
                    out_f32[(size_t)(row0 + r) * N + n0 + 64 * W + 16 * g + (lane & 15)] = acc[q][g][i];
                }
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

// combine_rows_kernel for K <= 8 with four columns per thread (D % 4 == 0, 16-byte aligned rows): the
// same arithmetic per element, a quarter of the load instructions, every y row load of the thread in
// flight before the sums.
__global__ __launch_bounds__(256) void combine_rows4_kernel(const float *__restrict__ y,
                                                           const int32_t *__restrict__ pos_of,
                                                           const float *__restrict__ weights, int K, int D,
                                                           float *__restrict__ x_inout, float *__restrict__ moe_out) {
    const int t = blockIdx.y;
    const int d = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (d >= D) return;
    const size_t o = (size_t)t * D + d;
    int p[8];
    float wk[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int kc = min(k, K - 1);
        p[k] = pos_of[t * K + kc];
        wk[k] = weights[t * K + kc];
    }
    const f32x4 xo = x_inout ? *reinterpret_cast<const f32x4 *>(x_inout + o) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 tmp[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) tmp[k] = *reinterpret_cast<const f32x4 *>(y + (size_t)p[k] * D + d);
    f32x4 moe = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
#pragma clang fp contract(off)
        if (k < K) {
            moe.x = moe.x + wk[k] * tmp[k].x;
            moe.y = moe.y + wk[k] * tmp[k].y;
            moe.z = moe.z + wk[k] * tmp[k].z;
            moe.w = moe.w + wk[k] * tmp[k].w;
        }
    }
    if (moe_out) *reinterpret_cast<f32x4 *>(moe_out + o) = moe;
    if (x_inout) {
#pragma clang fp contract(off)
        const f32x4 xn = f32x4{xo.x + moe.x, xo.y + moe.y, xo.z + moe.z, xo.w + moe.w};
        *reinterpret_cast<f32x4 *>(x_inout + o) = xn;
    }
}

template <int MATS, int ROWS, int WROWS>
hipError_t launch_gemm(const Launch &L, const uint8_t *experts, uint64_t stride, uint64_t w_off, uint64_t w3_off,
                       int N, int Kd, const uint16_t *a_hi, const uint16_t *a_lo, int gather, const int32_t *perm,
                       int topk, const int32_t *counts, const int32_t *offsets, const int32_t *m_off, int E,
                       int max_mtiles, float *out_f32, uint16_t *out_hi, uint16_t *out_lo) {
    if (N % (WROWS / MATS) != 0) return hipErrorInvalidValue;
    const long long tiles = (long long)max_mtiles * (N / (WROWS / MATS));
    const long long blocks = (tiles + 7) / 8 * 8;
    if (blocks > 0x7FFFFFFFll) return hipErrorInvalidValue;
    return launch(L, grouped_gemm_kernel<MATS, ROWS, WROWS>, dim3((unsigned)blocks), dim3(64 * GTile<ROWS, WROWS>::kWaves),
                  0, experts, stride, w_off, w3_off, N, Kd, a_hi, a_lo, gather, perm, topk, counts, offsets, m_off, E,
                  out_f32, out_hi, out_lo);
}

template <int MATS>
hipError_t launch_gemm_sel(const Launch &L, const uint8_t *experts, uint64_t stride, uint64_t w_off, uint64_t w3_off,
                           int N, int Kd, const uint16_t *a_hi, const uint16_t *a_lo, int gather, const int32_t *perm,
                           int topk, const int32_t *counts, const int32_t *offsets, const int32_t *m_off64,
                           const int32_t *m_off128, const int32_t *choice, int E, int max_mtiles64, float *out_f32,
                           uint16_t *out_hi, uint16_t *out_lo, const uint8_t *tiled, uint64_t tiled_stride,
                           uint64_t tiled_off) {
    constexpr int NTILE = MATS == 2 ? 128 : 256;  // both paths' tile width
    static_assert(NTILE == 256 / MATS, "the 64-row tiles are as wide");
    if (!gemm_wr_supported(MATS, N, Kd)) return hipErrorInvalidValue;
    const long long tiles = (long long)max_mtiles64 * (N / NTILE);  // >= the 128-row tiles
    const long long blocks = (tiles + 7) / 8 * 8;
    if (blocks > 0x7FFFFFFFll) return hipErrorInvalidValue;
    if (tiled)
        return launch(L, grouped_gemm_sel_kernel<MATS, false>, dim3((unsigned)blocks), dim3(64 * kWrWaves), 0, experts,
                      stride, w_off, w3_off, N, Kd, a_hi, a_lo, gather, perm, topk, counts, offsets, m_off64, m_off128,
                      choice, E, out_f32, out_hi, out_lo, tiled, tiled_stride, tiled_off);
    return launch(L, grouped_gemm_sel_kernel<MATS, true>, dim3((unsigned)blocks), dim3(64 * kWrWaves), 0, experts,
                  stride, w_off, w3_off, N, Kd, a_hi, a_lo, gather, perm, topk, counts, offsets, m_off64, m_off128, choice,
                  E, out_f32, out_hi, out_lo, tiled, tiled_stride, tiled_off);
}

template <int MATS>
hipError_t launch_gemm_wide(const Launch &L, const uint8_t *experts, uint64_t stride, uint64_t w_off, uint64_t w3_off,
                            int N, int Kd, const uint16_t *a_hi, const uint16_t *a_lo, int gather, const int32_t *perm,
                            int topk, const int32_t *counts, const int32_t *offsets, const int32_t *m_off128,
                            const int32_t *choice, int E, int max_mtiles, float *out_f32, uint16_t *out_hi,
                            uint16_t *out_lo, const uint8_t *tiled, uint64_t tiled_stride, uint64_t tiled_off) {
    if (!gemm_wide_supported(MATS, N, Kd)) return hipErrorInvalidValue;
    const long long tiles = (long long)max_mtiles * (N / (MATS == 2 ? 256 : 512));  // >= the 128-row tiles
    const long long blocks = (tiles + 7) / 8 * 8;
    if (blocks > 0x7FFFFFFFll) return hipErrorInvalidValue;
    if (tiled)
        return launch(L, grouped_gemm_wide_kernel<MATS, false>, dim3((unsigned)blocks), dim3(64 * kWdWaves), 0, experts,
                      stride, w_off, w3_off, N, Kd, a_hi, a_lo, gather, perm, topk, counts, offsets, m_off128, choice, E,
                      out_f32, out_hi, out_lo, tiled, tiled_stride, tiled_off);
    return launch(L, grouped_gemm_wide_kernel<MATS, true>, dim3((unsigned)blocks), dim3(64 * kWdWaves), 0, experts,
                  stride, w_off, w3_off, N, Kd, a_hi, a_lo, gather, perm, topk, counts, offsets, m_off128, choice, E,
                  out_f32, out_hi, out_lo, tiled, tiled_stride, tiled_off);
}

}  // namespace

bool prefill_layout_supported(int dtype, int D, int H) {
    return dtype == RBT_DT_BF16 && D % kGWRows == 0 && gemm_wr_supported(2, H, D) && gemm_wr_supported(1, D, H);
}

size_t prefill_layout_bytes(int E, int D, int H) { return (size_t)E * 3 * H * D * 2; }

hipError_t launch_prefill_layout(const Launch &L, const void *experts, uint64_t stride, int E, int D, int H, void *dst) {
    if (!prefill_layout_supported(RBT_DT_BF16, D, H) || E < 1 || E > 65535 || stride % 16 != 0 ||
        (reinterpret_cast<uintptr_t>(experts) & 15u) || (reinterpret_cast<uintptr_t>(dst) & 15u))
        return hipErrorInvalidValue;
    const uint64_t units = 3 * (uint64_t)H * D / 8;  // 16-byte units per expert
    return launch(L, prefill_layout_kernel, dim3((unsigned)((units + 255) / 256), (unsigned)E), dim3(256), 0,
                  static_cast<const uint8_t *>(experts), stride, D, H, static_cast<uint8_t *>(dst), units);
}

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
    return up(4 * (size_t)E) + 3 * up(4 * (size_t)(E + 1)) + up(4) + 2 * up(4 * P) + up(4 * P * (size_t)D) +
           2 * up(2 * (size_t)T * D);
}

namespace {
// Workspace carve-up of the grouped path (prefill_workspace_bytes is its total).
struct PrefillWs {
    int32_t *counts, *offsets, *m_off, *m_off128, *choice, *perm, *pos_of;
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
    r.m_off128 = reinterpret_cast<int32_t *>(carve(4 * (size_t)(E + 1)));
    r.choice = reinterpret_cast<int32_t *>(carve(4));
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
                          int32_t **counts_out, bool x_split_done, bool combine, int tile_rows, const void *tiled,
                          bool wide_ok) {
    if (tile_rows != 0 && tile_rows != 32 && tile_rows != 64 && tile_rows != 128) return hipErrorInvalidValue;
    if (T <= 0 || K <= 0) return hipErrorInvalidValue;  // the dispatch reads at least one pair
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
    // Row tiles of 32 when experts average at most 16 rows (decode-sized batches: a deeper copy ring);
    // otherwise 64-row tiles or, where the shape allows, 128-row tiles (a weight tile streamed once for
    // up to 128 rows, by the register kernel), the dispatch kernel choosing between the two from the
    // histogram (tile_rows 64 / 128 forces one).
    // the 128-row kernel addresses the gathered x planes with 32-bit buffer offsets
    const bool tall_ok = gemm_wr_supported(2, H, D) && gemm_wr_supported(1, D, H) &&
                         (size_t)T * D * 2 + 2 * (size_t)D < (size_t)kWrBufRecords;
    const bool small = tile_rows == 32 || (tile_rows == 0 && P <= kSmallTileRowsPerExpert * E);
    const int mt_rows = small ? 32 : 64;
    const int tall = !tall_ok || small || tile_rows == 64 ? 1 : 2;
    const bool sel = !small && tall_ok;
    e = launch(Ldd, dispatch_kernel, dim3(1), dim3(1024), 0, routing, P, E, counts, offsets, perm, pos_of, m_off,
               mt_rows, sel ? r.m_off128 : nullptr, r.choice, tall);
    if (e != hipSuccess) return e;
    // 128-row tiles (the dispatch picks them whenever tall == 2) in the wide kernel where the shape has it
    const bool wide = sel && tall == 2 && wide_ok && gemm_wide_supported(2, H, D) && gemm_wide_supported(1, D, H);
    const uint8_t *ex = static_cast<const uint8_t *>(experts);
    const int max_mtiles = (P + mt_rows - 1) / mt_rows + E;  // >= sum over experts of ceil(count / mt_rows)
    const uint64_t w3 = (uint64_t)H * D * 2, w2 = 2 * (uint64_t)H * D * 2;
    const uint8_t *tl = static_cast<const uint8_t *>(tiled);
    const uint64_t tstride = 3 * (uint64_t)H * D * 2;  // the tiled copy's bytes per expert
    // gate/up: N = H, Kd = D, activation rows gathered through perm; h written as hi/lo planes
    if (small)
        e = launch_gemm<2, 32, 128>(Lg, ex, stride, 0, w3, H, D, x_hi, x_lo, 1, perm, K, counts, offsets, m_off, E,
                                    max_mtiles, nullptr, h_hi, h_lo);
    else if (!sel)
        e = launch_gemm<2, 64, 256>(Lg, ex, stride, 0, w3, H, D, x_hi, x_lo, 1, perm, K, counts, offsets, m_off, E,
                                    max_mtiles, nullptr, h_hi, h_lo);
    else if (wide)
        e = launch_gemm_wide<2>(Lg, ex, stride, 0, w3, H, D, x_hi, x_lo, 1, perm, K, counts, offsets, r.m_off128,
                                r.choice, E, max_mtiles, nullptr, h_hi, h_lo, tl, tstride, 0);
    else
        e = launch_gemm_sel<2>(Lg, ex, stride, 0, w3, H, D, x_hi, x_lo, 1, perm, K, counts, offsets, m_off, r.m_off128,
                               r.choice, E, max_mtiles, nullptr, h_hi, h_lo, tl, tstride, 0);
    if (e != hipSuccess) return e;
    // down: N = D, Kd = H, activation rows = the h planes in list order
    if (small)
        e = launch_gemm<1, 32, 128>(Lw, ex, stride, w2, 0, D, H, h_hi, h_lo, 0, perm, K, counts, offsets, m_off, E,
                                    max_mtiles, y, nullptr, nullptr);
    else if (!sel)
        e = launch_gemm<1, 64, 256>(Lw, ex, stride, w2, 0, D, H, h_hi, h_lo, 0, perm, K, counts, offsets, m_off, E,
                                    max_mtiles, y, nullptr, nullptr);
    else if (wide)
        e = launch_gemm_wide<1>(Lw, ex, stride, w2, 0, D, H, h_hi, h_lo, 0, perm, K, counts, offsets, r.m_off128,
                                r.choice, E, max_mtiles, y, nullptr, nullptr, tl, tstride, w2);
    else
        e = launch_gemm_sel<1>(Lw, ex, stride, w2, 0, D, H, h_hi, h_lo, 0, perm, K, counts, offsets, m_off, r.m_off128,
                               r.choice, E, max_mtiles, y, nullptr, nullptr, tl, tstride, w2);
    if (e != hipSuccess) return e;
    if (!combine) return hipSuccess;
    const auto a16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    if (K <= 8 && D % 4 == 0 && a16(y) && (!x_inout || a16(x_inout)) && (!moe_out || a16(moe_out)))
        return launch(Lc, combine_rows4_kernel, dim3((unsigned)((D / 4 + 255) / 256), (unsigned)T), dim3(256), 0,
                      (const float *)y, (const int32_t *)pos_of, weights, K, D, x_inout, moe_out);
    return launch(Lc, combine_rows_kernel, dim3((unsigned)((D + 255) / 256), (unsigned)T), dim3(256), 0,
                  (const float *)y, (const int32_t *)pos_of, weights, K, D, x_inout, moe_out);
}

}  // namespace rbt
