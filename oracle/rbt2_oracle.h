/*
 * ORACLE -- test infrastructure, not product code.
 *
 * A CPU restatement of the RABBIT2 engine's arithmetic (rabbit2/src/rabbit2.c) and of its .rbt2
 * storage format (rabbit2/ref/rbt2.py). It checks the HIP path's results: only the test suite,
 * the smoke check and the CPU-baseline leg of the benchmark load it. The product library never
 * links, loads or calls anything here.
 *
 * Every function cites the reference lines it restates. The arithmetic is plain fp32 C99 with
 * no FMA contraction (the reference is built with `gcc -O2 -std=c99`, which implies
 * -ffp-contract=off, and baseline x86-64 has no FMA), so the results are bitwise those of the
 * reference engine for both of its matvec orders.
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   orc_layout                 closed-form OLMoE offsets + `--info` of the reference binary
 *   orc_bf16_*                 known answers (RNE ties-to-even, NaN -> 0x7FC0, exact widening)
 *   orc_matvec (both orders)   bitwise vs the reference binary (full forward), float64 brute force
 *   orc_softmax / orc_topk     invariants + brute-force stable sort + reference binary routing
 *   orc_moe_layer              bitwise vs the reference binary (full forward, 1-layer models up to
 *                              the OLMoE layer shape) + float64 brute force + linearity
 *   orc_forward / orc_generate bitwise vs the reference binary --dump / --gen, golden fixtures
 *   orc_normal                 published SplitMix64 outputs + moments of the normal samples
 */
#ifndef RBT2_ORACLE_H
#define RBT2_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_DT_F32 0
#define ORC_DT_BF16 1
#define ORC_ORDER_SCALAR 0 /* rabbit2.c:356-390: 4 interleaved partial sums */
#define ORC_ORDER_AVX2 1   /* rabbit2.c:323-353: two 8-lane accumulators, mul then add */

/* On-disk header fields, bytes 8..67 of a .rbt2 file (rabbit2.c:63-69, rbt2.py:24-44). */
typedef struct {
    int32_t vocab, dim, n_layers, n_heads, n_kv_heads, head_dim;
    int32_t n_experts, top_k, expert_hidden, max_seq;
    int32_t dtype, qk_norm, norm_topk;
    float rope_theta, rms_eps;
} orc_config;

typedef struct {
    uint64_t attn_norm, wq, wk, wv, wo, q_norm, k_norm, ffn_norm, router, experts;
} orc_layer_off;

typedef struct {
    uint64_t tok_emb, final_norm, lm_head, expert_stride, end;
} orc_model_off;

/* Layout rules of rabbit2.c:158-193 / rbt2.py:66-101. `layers` has c->n_layers entries. */
void orc_layout(const orc_config *c, orc_model_off *m, orc_layer_off *layers);

/* bf16 helpers: widening rabbit2.c:304-309; RNE encoder rbt2.py:106-113. */
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
void orc_f32_to_bf16_n(const float *src, uint16_t *dst, size_t n);

/* out[r] = dot(W[r,:], x) in the given reference order (rabbit2.c:323-390). */
void orc_matvec(float *out, const void *W, int dtype, const float *x, int rows, int cols, int order);
/* rabbit2.c:392-407 */
void orc_rmsnorm(float *out, const float *x, const float *w, int n, float eps);
void orc_softmax(float *x, int n);
float orc_silu(float x);
/* Iterative top-k of rabbit2.c:516-528 (strict '>', lowest index wins ties). used[] has n bytes. */
void orc_topk(const float *probs, int n, int k, unsigned char *used, int32_t *idx, float *wt, float *wsum);

/* One MoE feed-forward block, rabbit2.c:513-542, for T tokens (the reference loops tokens one by
 * one; tokens are independent inside the block). The rmsnorm prologue (:512) is the caller's:
 * xb is the normalised input [T][dim].
 *   router       [n_experts][dim] in dtype
 *   experts      expert e blob at experts + e*expert_stride: w1[H,D] | w3[H,D] | w2[D,H]
 *   router_bias  optional [n_experts] f32 added to the logits before softmax (a harness
 *                extension used for skewed-routing workloads; NULL in the reference)
 * Outputs (each may be NULL): x_inout += moe; moe_out [T][dim]; routing [T][top_k];
 * weights [T][top_k] (the combine weights, after norm_topk); probs_out [T][n_experts]. */
typedef struct {
    int32_t dim, n_experts, top_k, expert_hidden, dtype, norm_topk;
    const void *router;
    const unsigned char *experts;
    uint64_t expert_stride;
    const float *router_bias;
} orc_moe_desc;

int orc_moe_layer(const orc_moe_desc *d, const float *xb, int T, int order, float *x_inout, float *moe_out,
                  int32_t *routing, float *weights, float *probs_out);

/* The full per-token engine (rabbit2.c:453-548) over a prompt, exactly as the --dump loop
 * (:703-714): logits [nt][vocab], routing [nt][n_layers][top_k]. Then, if gen > 0, greedy
 * generation as the --gen loop (:718-740): gen_out receives up to `gen` ids; returns the count
 * through *n_gen. ctx <= 0 selects the engine default min(max_seq, 512) (:684-685).
 * Returns 1 on success, 0 on a malformed model / bad arguments (message in orc_last_error()). */
int orc_run(const unsigned char *file, uint64_t file_size, const int32_t *tokens, int nt, int ctx, int order,
            float *logits, int32_t *routing, int gen, int32_t eos, int32_t *gen_out, int *n_gen);
/* The same with the engine's sampling for the generated tokens (--temperature, --top-k, --top-p,
 * --seed; rabbit2.c:558-610, :634-638, :716-740); temperature <= 0 is greedy. */
int orc_run_sampled(const unsigned char *file, uint64_t file_size, const int32_t *tokens, int nt, int ctx, int order,
                    float *logits, int32_t *routing, int gen, int32_t eos, int32_t *gen_out, int *n_gen,
                    float temperature, int top_k, float top_p, uint64_t seed);
/* sample_logits (rabbit2.c:569-610) and its generator (:558-567); idx/prob: [n] scratch. */
uint64_t orc_rng_next(uint64_t *state);
double orc_rng_uniform(uint64_t *state);
int orc_sample(const float *logits, int n, float temperature, int top_k, float top_p, uint64_t *rng, int32_t *idx,
               float *prob);
const char *orc_last_error(void);

/* Parse + validate a header (rabbit2.c:199-228). Returns 1 and fills *c on success. */
int orc_parse_header(const unsigned char *file, uint64_t file_size, orc_config *c);

/* ---- seeded synthetic data (the repository's own generator; not the reference's NumPy stream) ----
 * splitmix64: the published SplitMix64 step (Steele, Lea, Flood 2014; Vigna's splitmix64.c).
 * orc_normal(seed, stream, i): counter-based N(0,1) sample number i of a stream:
 *   key = splitmix64 output of (seed ^ golden*stream); pair p = i/2 uses outputs 2p and 2p+1 of a
 *   SplitMix64 sequence started at key, u1 = (top 53 bits + 0.5) * 2^-53, u2 = top 53 bits * 2^-53,
 *   Box-Muller: r = sqrt(-2 ln u1), z = r*cos(2 pi u2) for even i, r*sin(2 pi u2) for odd i. */
uint64_t orc_splitmix64_next(uint64_t *state);
double orc_normal(uint64_t seed, uint64_t stream, uint64_t i);
/* dst[i] = offset + scale * orc_normal(seed, stream, first + i), rounded to f32 then to dtype. */
void orc_fill_normal(void *dst, int dtype, uint64_t n, uint64_t seed, uint64_t stream, uint64_t first, float scale,
                     float offset);

/* Synthetic .rbt2 models. Stream numbering of each tensor (so any tensor can be regenerated alone):
 *   tok_emb 1, final_norm 2, lm_head 3, layer l: 16 + 16*l + {attn_norm 0, wq 1, wk 2, wv 3, wo 4,
 *   q_norm 5, k_norm 6, ffn_norm 7, router 8}, expert e of layer l: 1<<32 | (l*n_experts + e)*3 + {w1 0, w3 1, w2 2}
 * Matrix scale: w_scale, or w_scale / sqrt(cols) when fan_in_scale is set. Norm vectors:
 * 1 + norm_jitter * N(0,1). Embeddings: emb_scale * N(0,1). */
typedef struct {
    uint64_t seed;
    float w_scale;
    int32_t fan_in_scale;
    float emb_scale;
    float norm_jitter;
} orc_gen_params;

uint64_t orc_expert_stream(const orc_config *c, int layer, int e, int which);
uint64_t orc_layer_stream(int layer, int which);
/* Total file size for a config (layout end rounded up to 4 KiB, as Rbt2Writer truncates). */
uint64_t orc_model_file_size(const orc_config *c);
/* Fill a zeroed buffer of orc_model_file_size(c) bytes with header + tensors. */
int orc_build_model(unsigned char *buf, uint64_t size, const orc_config *c, const orc_gen_params *g);
/* Same, streamed to a file. Returns 1 on success. */
int orc_write_model(const char *path, const orc_config *c, const orc_gen_params *g);

#ifdef __cplusplus
}
#endif
#endif
