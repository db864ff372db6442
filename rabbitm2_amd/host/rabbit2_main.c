/*
 * rabbit2 -- the RABBIT2 engine's command line with forward() on the MI355X.
 *
 * Same flags, output files, stdout/stderr lines and exit codes as the reference engine's main()
 * (rabbit2/src/rabbit2.c:610-755): --dump writes little-endian f32 logits [T][vocab] and int32
 * routing [T][n_layers][top_k] (:703-714), --gen prints one id per line (:716-740), --info prints
 * the header and layout lines (:668-679), the timing line and, with --expert-cache-mib, the
 * expert-cache line go to stderr (:742-751). Exit codes: 0 ok, 1 runtime error, 2 usage.
 *
 * Everything past argument parsing runs through the C ABI of include/rbt2_hip.h: the .rbt2 image is
 * copied to HBM once, the KV cache lives in HBM, and each forward() is the library's per-token pass on
 * hand-written gfx950 kernels. --gen runs the loop on the device (rbt_hip_generate_stream) and prints
 * each id with a flush as soon as the device has produced it, as the engine does (rabbit2.c:726-729).
 *
 * --kernel keeps its meaning as the CPU summation order that expert selection reproduces bit for bit,
 * and prints the engine's line for it (rabbit2.c:652-661): no flag or "scalar" -> the engine's scalar
 * order (its default, rabbit2.c:312), "matvec kernel: scalar"; "avx2" -> the AVX2 order, "matvec
 * kernel: avx2" (reproduced on the device whatever the host CPU); "auto" -> AVX2 when this host has it,
 * as the engine's auto picks; "hip" -> the same order as auto, printed as "matvec kernel: hip-gfx950".
 *
 * --expert-cache-mib: every expert is resident in HBM, so no expert is read from the file after the
 * upload; the budget checks are the engine's (rabbit2.c:238-242, :640-648), and the stats line
 * (:745-751) reports what the engine's LRU cache would have done for the same routing, replayed over
 * the routing of every forward() the engine would have run (rbt_hip_expert_cache_replay).
 */
#define _POSIX_C_SOURCE 200809L /* clock_gettime under -std=c99 */
#include <errno.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "rbt2_hip.h"

static double now_sec(void) { /* the engine's clock (rabbit2.c:114-125) */
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

static int host_has_avx2(void) {
#if defined(__x86_64__) || defined(__i386__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") != 0;
#else
    return 0;
#endif
}

static void usage(const char *p) {
    fprintf(stderr,
            "usage:\n"
            "  %s <model.rbt2> --dump <logits.bin> <routing.bin> [--ctx N] [--expert-cache-mib N] [--kernel auto|scalar|avx2|hip] <token> ...\n"
            "  %s <model.rbt2> --gen <n> [--eos id] [--ctx N] [--temperature T] [--top-k K] [--top-p P] [--seed S] [--expert-cache-mib N] [--kernel auto|scalar|avx2|hip] <token> ...\n"
            "  %s <model.rbt2> --info\n",
            p, p, p);
}

/* "moe: bytes=... GB/s=... %peak=...": the MoE blocks the library timed on the device (its deferred
 * kernel timing, profiling mode 2, in the --dump pass's eager forward() steps; the --gen loop replays
 * HIP graphs, whose kernels HIP does not time): their kernels' summed durations, their bytes as the
 * engine's block reads them (router rows and top_k experts' w1/w3/w2 per token and layer), and that
 * rate against MI355X's published 8 TB/s HBM peak. Nothing is printed when no block was timed. */
static int print_moe_line(rbt_hip *h, const rbt_config *c) {
    static const char *const kern[4] = {"router", "topk", "gateup", "down_combine"};
    double ms = 0.0, t = 0.0;
    uint64_t blocks = 0, n = 0;
    for (int i = 0; i < 4; i++) {
        if (!rbt_hip_profile_get(h, kern[i], &t, &n)) return 0;
        ms += t;
        if (i == 0) blocks = n;
    }
    if (!blocks) return 1;
    const double esz = c->dtype == RBT_DT_BF16 ? 2.0 : 4.0;
    const double bytes =
        (double)blocks * esz * ((double)c->n_experts * c->dim + 3.0 * c->top_k * c->expert_hidden * (double)c->dim);
    const double gbs = ms > 0.0 ? bytes / (ms * 1e-3) / 1e9 : 0.0;
    fprintf(stderr, "moe: bytes=%.0f GB/s=%.1f %%peak=%.1f\n", bytes, gbs, 100.0 * gbs / 8000.0);
    return 1;
}

/* The engine's gen-loop output: one id per line, flushed (rabbit2.c:728-729). */
static int print_token(void *user, int32_t token) {
    (void)user;
    printf("%d\n", token);
    fflush(stdout);
    return 1;
}

/* Runs the engine with the model loaded on device 0; returns the process exit code. cache_budget > 0:
 * print the engine's expert-cache line for that budget. */
static int run(const char *path, const rbt_config *c, uint64_t expert_stride, int order, int ctx,
               const int32_t *tokens, int nt, const char *dump_l, const char *dump_r, int gen, int eos,
               float temperature, int top_k_sample, float top_p, unsigned long long seed,
               unsigned long long cache_budget) {
    rbt_hip *h = NULL;
    if (!rbt_hip_init(&h, 0)) return 1; /* the library printed the reason */
    int rc = 1;
    float *logits = NULL;
    int32_t *routing = NULL, *ids = NULL, *hist = NULL;
    FILE *fl = NULL, *fr = NULL;
    if (!rbt_hip_set_router_order(h, order) || !rbt_hip_upload_file(h, path, NULL)) goto done;
    if (cache_budget && !rbt_hip_set_option(h, "routing_history", 1)) goto done;
    if (!rbt_hip_state_init(h, ctx)) goto done;
    if (!rbt_hip_profile_enable(h, 2)) goto done; /* kernel times of the MoE blocks, for the moe line */

    logits = (float *)malloc(sizeof(float) * (size_t)c->vocab);
    routing = (int32_t *)calloc((size_t)c->n_layers * c->top_k, sizeof(int32_t));
    if (!logits || !routing) {
        fprintf(stderr, "out of memory\n");
        goto done;
    }

    double t0 = now_sec(), t1 = t0, t2 = t0;
    int produced = 0;
    if (dump_l) {
        fl = fopen(dump_l, "wb");
        fr = fopen(dump_r, "wb");
        if (!fl || !fr) {
            fprintf(stderr, "cannot open output files\n");
            goto done;
        }
        for (int i = 0; i < nt; i++) {
            if (!rbt_hip_forward(h, tokens[i], i, logits, routing)) goto done;
            fwrite(logits, sizeof(float), (size_t)c->vocab, fl);
            fwrite(routing, sizeof(int32_t), (size_t)c->n_layers * c->top_k, fr);
        }
        fclose(fl);
        fclose(fr);
        fl = fr = NULL;
        t1 = now_sec();
    }
    t2 = t1;
    if (gen > 0) {
        if (gen > ctx - nt) gen = ctx - nt; /* rabbit2.c:717 */
        ids = (int32_t *)malloc(sizeof(int32_t) * (size_t)(gen > 0 ? gen : 1));
        if (!ids) {
            fprintf(stderr, "out of memory for sampling buffers\n");
            goto done;
        }
        if (temperature > 0.0f && !rbt_hip_set_sampling(h, temperature, top_k_sample, top_p, (uint64_t)seed))
            goto done;
        /* the device loop runs the prompt itself (again, after a --dump pass) and then the tokens,
         * printing each id as it arrives */
        double ms[2] = {0.0, 0.0};
        int n = 0;
        if (gen > 0 && !rbt_hip_generate_stream(h, tokens, nt, gen, eos, print_token, NULL, ids, &n, ms)) goto done;
        produced = n;
        if (!dump_l) { /* the prompt/generation split of the device loop, from its HIP events */
            t1 = t0 + ms[0] * 1e-3;
        }
        t2 = t1 + ms[1] * 1e-3;
    }
    fprintf(stderr, "prompt: %d tokens in %.2fs (%.2f tok/s)", nt, t1 - t0, nt / (t1 - t0 + 1e-9));
    if (gen > 0) fprintf(stderr, " | generated %d in %.2fs (%.2f tok/s)", produced, t2 - t1, produced / (t2 - t1 + 1e-9));
    fprintf(stderr, "\n");
    if (!print_moe_line(h, c)) goto done;
    if (cache_budget) {
        /* the forward() calls the engine makes: the prompt, then one per generated id but the last
         * (rabbit2.c:704, :732-733) */
        const int n_fwd = nt + (produced > 0 ? produced - 1 : 0);
        const size_t per = (size_t)c->n_layers * c->top_k;
        uint64_t s[6];
        hist = (int32_t *)malloc(sizeof(int32_t) * per * (size_t)n_fwd);
        if (!hist) {
            fprintf(stderr, "out of memory\n");
            goto done;
        }
        if (!rbt_hip_routing_history(h, 0, 0, n_fwd, hist) ||
            !rbt_hip_expert_cache_replay(cache_budget, expert_stride, c->n_layers, c->n_experts, c->top_k, hist,
                                         (uint64_t)n_fwd, s))
            goto done;
        fprintf(stderr,
                "expert cache: hits=%llu misses=%llu evictions=%llu bytes_read=%llu resident_bytes=%llu "
                "capacity_bytes=%llu\n",
                (unsigned long long)s[0], (unsigned long long)s[1], (unsigned long long)s[2],
                (unsigned long long)s[3], (unsigned long long)s[4], (unsigned long long)s[5]);
    }
    rc = 0;
done:
    if (fl) fclose(fl);
    if (fr) fclose(fr);
    free(logits);
    free(routing);
    free(ids);
    free(hist);
    rbt_hip_free(h);
    return rc;
}

int main(int argc, char **argv) {
    if (argc < 3) {
        usage(argv[0]);
        return 2;
    }
    const char *dump_l = NULL, *dump_r = NULL, *kernel = NULL;
    int gen = 0, eos = -1, ctx = 0, nt = 0, info = 0, top_k_sample = 0;
    float temperature = 0.0f, top_p = 1.0f;
    unsigned long long seed = 0, cache_mib = 0;
    int32_t *tokens = (int32_t *)malloc(sizeof(int32_t) * (size_t)argc);
    if (!tokens) {
        fprintf(stderr, "out of memory\n");
        return 1;
    }
    for (int i = 2; i < argc; i++) {
        if (!strcmp(argv[i], "--dump") && i + 2 < argc) {
            dump_l = argv[++i];
            dump_r = argv[++i];
        } else if (!strcmp(argv[i], "--info")) {
            info = 1;
        } else if (!strcmp(argv[i], "--gen") && i + 1 < argc) {
            gen = atoi(argv[++i]);
        } else if (!strcmp(argv[i], "--eos") && i + 1 < argc) {
            eos = atoi(argv[++i]);
        } else if (!strcmp(argv[i], "--ctx") && i + 1 < argc) {
            ctx = atoi(argv[++i]);
        } else if (!strcmp(argv[i], "--kernel") && i + 1 < argc) {
            kernel = argv[++i];
        } else if (!strcmp(argv[i], "--temperature") && i + 1 < argc) {
            temperature = (float)strtod(argv[++i], NULL);
        } else if (!strcmp(argv[i], "--top-k") && i + 1 < argc) {
            top_k_sample = atoi(argv[++i]);
        } else if (!strcmp(argv[i], "--top-p") && i + 1 < argc) {
            top_p = (float)strtod(argv[++i], NULL);
        } else if (!strcmp(argv[i], "--seed") && i + 1 < argc) {
            seed = strtoull(argv[++i], NULL, 10);
        } else if (!strcmp(argv[i], "--expert-cache-mib") && i + 1 < argc) {
            /* the engine's validation (rabbit2.c:640-648) */
            const char *arg = argv[++i];
            char *end = NULL;
            errno = 0;
            const unsigned long long mib = strtoull(arg, &end, 10);
            if (arg[0] < '0' || arg[0] > '9' || *end || errno || !mib || mib > SIZE_MAX / (1024u * 1024u)) {
                fprintf(stderr, "--expert-cache-mib must be a positive integer that fits in memory\n");
                return 2;
            }
            cache_mib = mib;
        } else if (argv[i][0] == '-' && argv[i][1] == '-') {
            fprintf(stderr, "bad option %s\n", argv[i]);
            usage(argv[0]);
            return 2;
        } else {
            tokens[nt++] = atoi(argv[i]);
        }
    }
    if (!info && (nt < 1 || (!dump_l && gen <= 0))) {
        usage(argv[0]);
        return 2;
    }
    int order = RBT_ORDER_SCALAR; /* the engine's default matvec (use_avx2 = 0, rabbit2.c:312) */
    if (kernel) {                 /* rabbit2.c:652-661 */
        if (strcmp(kernel, "scalar") && strcmp(kernel, "auto") && strcmp(kernel, "avx2") && strcmp(kernel, "hip")) {
            fprintf(stderr, "--kernel must be scalar, auto, avx2 or hip\n");
            return 2;
        }
        if (!strcmp(kernel, "avx2"))
            order = RBT_ORDER_AVX2;
        else if (strcmp(kernel, "scalar"))
            order = host_has_avx2() ? RBT_ORDER_AVX2 : RBT_ORDER_SCALAR;
        if (!strcmp(kernel, "hip"))
            fprintf(stderr, "matvec kernel: hip-gfx950 (router order %s)\n", order == RBT_ORDER_AVX2 ? "avx2" : "scalar");
        else
            fprintf(stderr, "matvec kernel: %s\n", order == RBT_ORDER_AVX2 ? "avx2" : "scalar");
    }

    rbt_config c;
    uint64_t inf[7];
    if (!rbt_hip_file_info(argv[1], &c, inf)) return 1; /* the header checks of load_model */
    if (info) {
        printf("vocab=%d dim=%d n_layers=%d n_heads=%d n_kv_heads=%d head_dim=%d n_experts=%d top_k=%d\n", c.vocab,
               c.dim, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.n_experts, c.top_k);
        printf("expert_hidden=%d max_seq=%d dtype=%d qk_norm=%d norm_topk=%d\n", c.expert_hidden, c.max_seq, c.dtype,
               c.qk_norm, c.norm_topk);
        printf("tok_emb=%llu layer0_experts=%llu last_layer_experts=%llu expert_stride=%llu lm_head=%llu "
               "layout_end=%llu file_size=%llu\n",
               (unsigned long long)inf[0], (unsigned long long)inf[1], (unsigned long long)inf[2],
               (unsigned long long)inf[3], (unsigned long long)inf[4], (unsigned long long)inf[5],
               (unsigned long long)inf[6]);
        free(tokens);
        return 0;
    }
    /* the budget checks of expert_cache_init (rabbit2.c:236-243); every expert is resident in HBM */
    if (cache_mib && cache_mib * 1024u * 1024u < inf[3]) {
        fprintf(stderr, "expert cache budget too small: need at least %llu bytes for one expert\n",
                (unsigned long long)inf[3]);
        return 1;
    }
    if (ctx <= 0) ctx = c.max_seq < 512 ? c.max_seq : 512; /* rabbit2.c:684-686 */
    if (ctx > c.max_seq) ctx = c.max_seq;
    if (nt > ctx) {
        fprintf(stderr, "prompt has %d tokens but context is %d (use --ctx)\n", nt, ctx);
        return 1;
    }
    for (int i = 0; i < nt; i++)
        if (tokens[i] < 0 || tokens[i] >= c.vocab) {
            fprintf(stderr, "token %d out of range\n", tokens[i]);
            return 1;
        }
    const int rc = run(argv[1], &c, inf[3], order, ctx, tokens, nt, dump_l, dump_r, gen, eos, temperature,
                       top_k_sample, top_p, seed, cache_mib * 1024u * 1024u);
    free(tokens);
    return rc;
}
