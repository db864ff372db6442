/*
 * rbt2_hip.h -- C ABI of the MI355X (gfx950) MoE-layer path for the RABBIT2 engine.
 *
 * The reference engine (rabbit2/src/rabbit2.c) is one C99 file whose MoE feed-forward block
 * (:511-542) runs on three static seams: matvec() (:357), get_expert() (:261) and forward()
 * (:455). This header is the boundary that replaces them: plain C types, plain pointers and sizes,
 * int 1 = ok / 0 = error (the engine's convention, e.g. load_model :199, forward :455), with the
 * message kept per handle (rbt_hip_last_error) and also printed to stderr like the engine does.
 *
 * Failure paths: with the environment variable RBT_HIP_FAULT="<kind>[:<n>]" (kind malloc, launch, copy
 * or sync) the n-th HIP call of that kind in the process is reported as failed without being made,
 * so every entry point's 0 + message path can be exercised from the host.
 *
 * Threading: a handle is used by one host thread at a time (the engine is single-threaded,
 * rabbit2/README.md:255). All device work of a handle runs in order on the handle's own HIP
 * stream. Calls ending in _dev take device pointers and are asynchronous on that stream; every
 * other call takes host pointers and returns when its results are in host memory.
 */
#ifndef RBT2_HIP_H
#define RBT2_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RBT_DT_F32 0  /* rabbit2.c:60 */
#define RBT_DT_BF16 1 /* rabbit2.c:61 */

/* Which CPU summation order the router logits reproduce bit for bit, so that expert selection is
 * identical to the engine's (top-k over softmax probabilities, strict '>', lowest index wins):
 *   RBT_ORDER_SCALAR  rabbit2.c:356-390 (--kernel scalar, and the engine's default)
 *   RBT_ORDER_AVX2    rabbit2.c:323-353 (--kernel auto|avx2 on AVX2 hosts) -- the default here */
#define RBT_ORDER_SCALAR 0
#define RBT_ORDER_AVX2 1

typedef struct rbt_hip rbt_hip; /* opaque: one device, one stream, owns its device memory */

/* Bytes 8..67 of a .rbt2 file header; same field order as Config (rabbit2.c:63-69). */
typedef struct {
    int32_t vocab, dim, n_layers, n_heads, n_kv_heads, head_dim;
    int32_t n_experts, top_k, expert_hidden, max_seq;
    int32_t dtype, qk_norm, norm_topk;
    float rope_theta, rms_eps;
} rbt_config;

/* One MoE layer in device memory, in the .rbt2 storage format (rabbit2.c:173, :186-189):
 * router [n_experts][dim] in dtype; expert e's blob at experts + e*expert_stride holding
 * w1[H][D] | w3[H][D] | w2[D][H] (w1 = gate, w3 = up, w2 = down), row-major, dtype elements.
 * router_bias: optional device [n_experts] f32 added to the router logits before the softmax
 * (no counterpart in the reference; used to build skewed-routing workloads), else NULL. */
typedef struct {
    int32_t dim, n_experts, top_k, expert_hidden, dtype, norm_topk;
    const void *router;
    const void *experts;
    uint64_t expert_stride;
    const float *router_bias;
} rbt_moe_layer;

/* ---- lifetime (replaces the engine's Model/State setup, rabbit2.c:199-228, :427-451) ---- */
int rbt_hip_init(rbt_hip **out, int device);
void rbt_hip_free(rbt_hip *h);
/* Last error message of this handle ("" if none); with h == NULL, the last init failure. */
const char *rbt_hip_last_error(const rbt_hip *h);
int rbt_hip_set_router_order(rbt_hip *h, int order);
/* Tuning switches (no counterpart in the reference):
 *   "fused_decode"        1 (default): a batch-1 block of up to 64 experts runs the softmax + top-k
 *                         inside the expert gate/up kernel (router logits, gate/up, down: three
 *                         launches); 0: a separate top-k launch (four launches). Same results.
 *   "batch_mfma"          1 (default): the batched forward (rbt_hip_batch_init with n_seq > 1) runs
 *                         q/k/v, wo and lm_head for up to 64 sequences on the matrix cores (bf16
 *                         weights; activations as bf16 hi + lo parts, exact products); 0: VALU dot
 *                         products. Both agree with the engine to rounding.
 *   "routing_history"     0 (default) / 1: from the next rbt_hip_state_init / rbt_hip_batch_init on,
 *                         every forward step also records its routing per sequence and position (one
 *                         small launch per step) for rbt_hip_routing_history.
 *   "prefill_min_tokens"  smallest T (1..65536, default 12) that takes the grouped path for bf16
 *                         weights: (token, slot) pairs dispatched into per-expert lists and the
 *                         expert FFN run as grouped GEMMs on the matrix cores, each expert's weights
 *                         read once per call. Smaller T runs one GEMV per pair. Routing is the same
 *                         either way; outputs agree within the parity tolerance.
 *   "prefill_layout"      1 (default): the grouped GEMMs read a layer's tiled expert copy where the
 *                         caller made one with rbt_hip_prefill_layout (none exists otherwise: by
 *                         default every kernel reads the .rbt2 blobs); 0: the blobs only.
 *   "prefill_tile_rows"   0 (default): the grouped GEMMs take tiles of 32 rows of an expert's list
 *                         while the experts average at most 16 rows, else 128 rows where the shape
 *                         has them (64 otherwise), in an order the device picks from the call's
 *                         tokens-per-expert histogram; 32 / 64 / 128: that tile height always (128
 *                         where the shape has it). Outputs agree within the parity tolerance (the
 *                         reduction runs in other chunks).
 *   "prefill_wide"        1 (default): 128-row tiles span 512 weight rows (gate/up: 256 W1 + 256 W3
 *                         rows; H a multiple of 256, D of 512), so each activation row fetched
 *                         serves twice the weight bytes; 0: 256 weight rows. Outputs agree within
 *                         rounding (the k-chunks run in another rotated order).
 *   "generate_timed_from" 1 (default): the generation time rbt_hip_generate* report (ms_out[1]) covers
 *                         generated steps g = 1 .. n_gen - 1 (step g forwards token g - 1); g0 > 1:
 *                         steps g0 .. n_gen - 1 only (0 ms if none), e.g. the last K steps of a run. */
int rbt_hip_set_option(rbt_hip *h, const char *name, int64_t value);

/* Upload a whole .rbt2 image (e.g. the engine's mmap, rabbit2.c:129-156) to HBM once. Validates the
 * header exactly like load_model() (rabbit2.c:199-228) and keeps every expert resident, which
 * replaces the engine's get_expert() streaming and LRU cache (rabbit2.c:233-300): 16 x 64 OLMoE
 * experts are 12 GiB of the 288 GB HBM. Fills *cfg (may be NULL). */
int rbt_hip_upload(rbt_hip *h, const void *file, uint64_t file_size, rbt_config *cfg);
/* The same from a file path: reads the header and validates it like load_model (rabbit2.c:199-228),
 * maps the file read-only and copies the image to HBM once, sequentially (replaces map_file and
 * get_expert's reads, rabbit2.c:129-156, :261-300). Fills *cfg (may be NULL). */
int rbt_hip_upload_file(rbt_hip *h, const char *path, rbt_config *cfg);
/* Host only (no device needed): reads the header of a .rbt2 file and validates it like load_model()
 * (rabbit2.c:199-228), the file included (it must hold its own layout), then reports what --info
 * prints (rabbit2.c:668-679): *cfg (may be NULL) and info (may be NULL) = {tok_emb, layer0_experts,
 * last_layer_experts, expert_stride, lm_head, layout_end, file_size} in bytes, from the layout rules
 * of rabbit2.c:158-193. Errors go to rbt_hip_last_error(NULL). */
int rbt_hip_file_info(const char *path, rbt_config *cfg, uint64_t info[7]);
/* The engine's expert-cache counters (rabbit2.c:745-751) for the HBM-resident image:
 * stats = {hits, misses, evictions, bytes_read, resident_bytes, capacity_bytes}. Every expert is a
 * miss once (read at upload) and stays resident: evictions 0, bytes_read = misses * expert_stride,
 * capacity = resident = all experts; hits counts the experts selected by the host-pointer calls
 * (rbt_hip_moe, rbt_hip_forward), whose routing passes through the host. */
int rbt_hip_expert_stats(rbt_hip *h, uint64_t stats[6]);
/* Device view of layer `layer` of the uploaded model (for the _dev calls). */
int rbt_hip_layer(rbt_hip *h, int layer, rbt_moe_layer *out);
/* An opt-in second HBM layout for the grouped (prefill) path (no counterpart in the reference: an
 * optimisation of the device copy, never made unless asked for here). The 128-row grouped GEMMs
 * stream a layer's experts tile by tile; in the engine's row-major blobs each step of a tile spans
 * 256 rows 4 KiB apart. rbt_hip_prefill_layout keeps a second copy of layer L's experts (the same
 * 3 * H * D bf16 per expert, +12.9 GB for all 16 OLMoE-1B-7B layers) in tile order, each step
 * contiguous; L NULL: every layer of the loaded model. bf16 experts, dim a multiple of 256,
 * expert_hidden of 256. The copy is taken from the blobs now, on the handle stream. Writes made
 * through this library (rbt_hip_h2d, rbt_hip_memset_dev, rbt_hip_fill_normal) into a layer's blobs
 * retake the experts they touch, in place, after the write; after a write made any other way, call
 * rbt_hip_prefill_layout again. Keyed by L->experts; dropped with the model, when rbt_hip_malloc
 * returns memory that held its blobs, by rbt_hip_prefill_layout_drop (L NULL: all) or rbt_hip_free.
 * Outputs are bit for bit the same with or without it. */
int rbt_hip_prefill_layout(rbt_hip *h, const rbt_moe_layer *L);
int rbt_hip_prefill_layout_drop(rbt_hip *h, const rbt_moe_layer *L);

/* ---- the MoE block (replaces rabbit2.c:513-542; the rmsnorm at :512 stays with the caller) ----
 * xb [T][dim] normalised input. x_inout [T][dim] receives x += moe (may be NULL).
 * routing_out [T][top_k] the chosen experts in selection order (the --dump routing record,
 * rabbit2.c:527), may be NULL. T may be 0. Host pointers; synchronous. */
int rbt_hip_moe(rbt_hip *h, int layer, const float *xb, int T, float *x_inout, int32_t *routing_out);

/* Same block on device pointers, asynchronous on the handle stream. Any output may be NULL:
 *   x_dev       [T][dim]    x += moe
 *   moe_dev     [T][dim]    the block output itself
 *   routing_dev [T][top_k]  int32 expert ids, selection order
 *   weights_dev [T][top_k]  combine weights (after norm_topk renormalisation, rabbit2.c:539)
 * Workspace is taken from the handle; it grows (hipMalloc) only when T exceeds every earlier
 * call's T, so call rbt_hip_reserve() first to keep allocation off the per-token path. */
int rbt_hip_moe_dev(rbt_hip *h, const rbt_moe_layer *L, const float *xb_dev, int T, float *x_dev, float *moe_dev,
                    int32_t *routing_dev, float *weights_dev);
int rbt_hip_reserve(rbt_hip *h, const rbt_moe_layer *L, int max_tokens);

/* rbt_hip_moe_dev that allocates nothing (no counterpart in the reference; for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops, hosts that forbid it).
 * Same arguments, kernels and results as rbt_hip_moe_dev, but the workspace is a fixed 64 MiB scratch
 * array the library holds on each GPU until the process ends, instead of the handle's workspace: calls
 * whose workspace would exceed it fail with a message (a 512-token call at the OLMoE layer shape needs
 * 52.2 MiB). No profiling events are taken. Every call on one GPU shares that GPU's array, so calls
 * that overlap on one GPU (other handles, other streams, other threads) race; calls on one stream run
 * in order. rbt_hip_expert_counts_dev then points into the array until the next call. */
int rbt_hip_moe_dev_noalloc(rbt_hip *h, const rbt_moe_layer *L, const float *xb_dev, int T, float *x_dev,
                            float *moe_dev, int32_t *routing_dev, float *weights_dev);

/* Tokens-per-expert histogram of the last rbt_hip_moe_dev call that used the grouped (prefill)
 * path, [n_experts] int32, device pointer owned by the handle; NULL if none. */
const int32_t *rbt_hip_expert_counts_dev(rbt_hip *h);

/* ---- the dense seam (replaces matvec(), rabbit2.c:357, for weights of the uploaded model) ----
 * out[r] = dot(W[r,:], x), W at byte offset w_offset of the uploaded image, [rows][cols] in the
 * model dtype. Host pointers; synchronous. */
int rbt_hip_matvec(rbt_hip *h, float *out, uint64_t w_offset, const float *x, int rows, int cols);
int rbt_hip_matvec_dev(rbt_hip *h, float *out_dev, const void *W_dev, int dtype, const float *x_dev, int rows,
                       int cols);

/* ---- the whole per-token forward pass (replaces forward(), rabbit2.c:453-548, on the State of
 * :427-446): embedding, then per layer RMSNorm, q/k/v, QK-norm, RoPE, the KV cache in HBM,
 * attention, wo + residual and the MoE block, then the final norm and lm_head. The matvecs and
 * attention sum in parallel orders (results agree with the engine to rounding); the router keeps the
 * engine's exact order. ---- */

/* Decode state for contexts of up to ctx positions (0 = the engine's default min(max_seq, 512),
 * larger than max_seq is clamped, rabbit2.c:684-686): the KV cache [n_layers][ctx][kv_dim] f32 (k and
 * v) and the step buffers, in HBM. Needs an uploaded or created model; replaces any earlier state. */
int rbt_hip_state_init(rbt_hip *h, int ctx);

/* One forward(token, pos) as the engine's --dump loop calls it (rabbit2.c:703-714): logits [vocab]
 * and routing_out [n_layers][top_k] (the --dump records, :710-713) in host memory; either may be
 * NULL. Positions are fed in order 0, 1, ... (the cache holds the positions before pos). Synchronous. */
int rbt_hip_forward(rbt_hip *h, int token, int pos, float *logits, int32_t *routing_out);

/* The engine's --gen loop with greedy sampling (temperature 0, rabbit2.c:716-740): the prompt from
 * position 0, then up to n_gen tokens (at most ctx - n_prompt; the eos token is kept and ends the
 * output, -1 = none) into out; *n_out = the count. The loop runs on the device: each step's argmax
 * writes the next step's token, and each step is one HIP graph replay (steps after an eos are run and
 * discarded). ms_out (may be NULL) receives [prompt ms, generation ms] from HIP events: the prompt up to
 * the first generated token, then the steps after it (from option "generate_timed_from" on). */
int rbt_hip_generate(rbt_hip *h, const int32_t *prompt, int n_prompt, int n_gen, int32_t eos, int32_t *out,
                     int *n_out, double *ms_out);

/* The same loop printing as the engine does (rabbit2.c:726-729: printf("%d\n") and fflush per token):
 * on_token(user, id) is called on the calling thread for each generated id in order, as soon as the
 * device has produced it, up to and including the eos token. The device runs at most 32 steps ahead of
 * the last reported id and none are queued after the eos token; if on_token returns 0 no further ids
 * are reported or queued. out [n_gen] and *n_out as rbt_hip_generate (steps already queued when the
 * output stopped are run and discarded). Each step also copies its id into a pinned host buffer (a
 * few us per token over rbt_hip_generate). on_token NULL is rbt_hip_generate. */
typedef int (*rbt_token_fn)(void *user, int32_t token);
int rbt_hip_generate_stream(rbt_hip *h, const int32_t *prompt, int n_prompt, int n_gen, int32_t eos,
                            rbt_token_fn on_token, void *user, int32_t *out, int *n_out, double *ms_out);

/* Routing of the forward steps run since the last rbt_hip_state_init / rbt_hip_batch_init (with option
 * "routing_history" set before it): sequence seq, positions [first_pos, first_pos + n_pos), into out
 * [n_pos][n_layers][top_k] -- what forward() writes to routing_out (rabbit2.c:527) at each position. A
 * position holds the last step run at it. */
int rbt_hip_routing_history(rbt_hip *h, int seq, int first_pos, int n_pos, int32_t *out);

/* Host only (no device needed): the engine's expert cache (rabbit2.c:236-300, --expert-cache-mib) replayed
 * over a routing stream [n_tokens][n_layers][top_k] in the engine's access order (token, layer, slot;
 * one get_expert per selection, :531-532): the same slots (budget / expert_stride of them, at most
 * every expert), the same victim rule (first never-filled slot, else least recently used) and the
 * counters of the engine's stats line (:745-751) into stats = {hits, misses, evictions, bytes_read,
 * resident_bytes, capacity_bytes}. The experts themselves stay resident in HBM; this reports what the
 * engine's cache would have done for the same routing. A budget below one expert fails with the
 * engine's message (:238-242). */
int rbt_hip_expert_cache_replay(uint64_t budget_bytes, uint64_t expert_stride, int n_layers, int n_experts, int top_k,
                                const int32_t *routing, uint64_t n_tokens, uint64_t stats[6]);

/* ---- batched decode (no counterpart in the reference, whose State holds one sequence): n_seq
 * independent sequences stepped together, each with its own KV cache of ctx positions. Every weight is
 * read once per step for all of them: the dense matvecs run over the n_seq token vectors, and the MoE
 * block takes the n_seq tokens as one batch (the grouped path from "prefill_min_tokens" tokens on). */
int rbt_hip_batch_init(rbt_hip *h, int n_seq, int ctx);
/* One forward() per sequence: sequence b takes tokens[b] at position pos[b] (positions advance
 * independently, in order per sequence). logits [n_seq][vocab], routing_out [n_layers][n_seq][top_k]
 * (either may be NULL). Synchronous. */
int rbt_hip_forward_batch(rbt_hip *h, const int32_t *tokens, const int32_t *pos, float *logits, int32_t *routing_out);
/* Greedy --gen for every sequence on the device: prompts [n_seq][n_prompt] from position 0, then
 * n_gen tokens each (at most ctx - n_prompt) into out [n_seq][n_gen]; one graph replay per step for
 * all sequences. ms_out (may be NULL): [prompt ms, generation ms]. */
int rbt_hip_generate_batch(rbt_hip *h, const int32_t *prompts, int n_prompt, int n_gen, int32_t *out, double *ms_out);

/* How rbt_hip_generate / rbt_hip_generate_batch pick tokens: the engine's --temperature, --top-k,
 * --top-p and --seed (rabbit2.c:569-610, :634-638, :723). temperature <= 0 (the default) is greedy;
 * otherwise each generated token is drawn on the device exactly as sample_logits does, with the
 * xorshift64* generator seeded by seed (0 = the engine's default constant), every sequence of a batch
 * from the same seed. The draws equal the engine's wherever its logits do (the device logits agree with
 * the engine's to rounding). */
int rbt_hip_set_sampling(rbt_hip *h, float temperature, int top_k, float top_p, uint64_t seed);

/* A model image built in place on the device instead of uploaded (no counterpart in the reference,
 * whose synthetic models are written to files by rabbit2/ref/rbt2.py): validates cfg like
 * rbt_hip_upload, allocates the image with the file layout (rabbit2.c:158-193) and returns its device
 * base; the contents are left for the caller to fill. */
int rbt_hip_model_create(rbt_hip *h, const rbt_config *cfg, void **model_dev);
/* Byte offset and size of a tensor in the model image (uploaded or created): name is one of
 * "tok_emb", "final_norm", "lm_head" (layer ignored) or "attn_norm", "wq", "wk", "wv", "wo",
 * "q_norm", "k_norm", "ffn_norm", "router", "experts" of layer `layer`. */
int rbt_hip_tensor(rbt_hip *h, const char *name, int layer, uint64_t *offset, uint64_t *bytes);

/* ---- device memory and stream plumbing for hosts without their own HIP code ---- */
int rbt_hip_malloc(rbt_hip *h, void **dev, uint64_t bytes);
int rbt_hip_free_dev(rbt_hip *h, void *dev);
int rbt_hip_h2d(rbt_hip *h, void *dst_dev, const void *src, uint64_t bytes);
int rbt_hip_d2h(rbt_hip *h, void *dst, const void *src_dev, uint64_t bytes);
int rbt_hip_memset_dev(rbt_hip *h, void *dst_dev, int value, uint64_t bytes);
int rbt_hip_synchronize(rbt_hip *h);
void *rbt_hip_stream(rbt_hip *h); /* the hipStream_t all of this handle's work runs on */

/* ---- instrumentation (the reference's only timing is its stderr tok/s line, rabbit2.c:742-744) ----
 * While enabled, every kernel launch of rbt_hip_moe_dev is bracketed by HIP events on the handle
 * stream and its duration is counted under its name ("router", "topk", "gateup",
 * "down_combine"; the grouped path adds "dispatch" -- the activation hi/lo split and the per-expert
 * lists -- and "combine", and its "down_combine" is the down GEMM alone); rbt_hip_forward adds
 * "embed", "attn_norm", "qkv" (RMSNorm + q/k/v), "attention", "attn_merge", "wo", "ffn_norm",
 * "lm_head" (final norm + lm_head, with the argmax inside where the rows allow) and "argmax"
 * (otherwise). Batched steps launch fewer: from 512 (sequence, head) pairs the attention writes its
 * output without "attn_merge", and on the grouped path "combine" also runs the RMSNorm that the
 * next step would time as "attn_norm". rbt_hip_generate is never timed this way. Modes (on):
 *   0  off.
 *   1  each call waits for its own kernels and adds their durations (eager calls only).
 *   2  deferred: each launch takes an event pair stamped by the launch itself and nothing waits for
 *      it, so timed _dev calls run back to back as in a decode loop; the pairs are read (and reused)
 *      when a synchronous call (rbt_hip_moe, rbt_hip_forward, rbt_hip_forward_batch) has waited for its
 *      own work, when 4096 pairs of one name are out, and by rbt_hip_profile_get, which returns the
 *      durations of every launch since the mode was set.
 * Setting a mode clears the counts; neither mode is for stream capture (HIP graphs do not time
 * events). rbt_hip_profile_get fails for an unknown name. */
int rbt_hip_profile_enable(rbt_hip *h, int on);
int rbt_hip_profile_get(rbt_hip *h, const char *kernel, double *total_ms, uint64_t *launches);
/* Host only (no device needed): 1 if a ROCm profiler tool is attached to this process, as its launcher
 * announces in the environment (rocprofv3: ROCPROFILER_LIBRARY_CTOR, ROCPROF_OUTPUT_PATH; older
 * tools: HSA_TOOLS_LIB, ROCP_TOOL_LIB), else 0. While one is, rbt_hip_generate, rbt_hip_generate_stream
 * and rbt_hip_generate_batch fail with a message instead of replaying HIP graphs (traced graph replays
 * have ended in a host SIGSEGV inside the tool); the eager calls trace normally. */
int rbt_hip_profiler_attached(void);

/* Synthetic data (no counterpart in the reference, whose random weights come from NumPy,
 * rabbit2/ref/reference.py:20-50): dst[i] = offset + scale * N(0,1) sample (first + i) of stream
 * `stream` under `seed`, rounded to f32 then to dtype (bf16 round-to-nearest-even). The sample
 * definition is SplitMix64 + Box-Muller, documented with the CPU twin in oracle/rbt2_oracle.h. */
int rbt_hip_fill_normal(rbt_hip *h, void *dst_dev, int dtype, uint64_t n, uint64_t seed, uint64_t stream,
                        uint64_t first, float scale, float offset);

#ifdef __cplusplus
}
#endif
#endif
