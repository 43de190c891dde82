/*
 * intllm_run — command-line driver of the C host (q48_host.h).
 *
 * Model sources (one of):
 *   --tiny                 2 layers, d=256, 8/2 heads, ffn 688, vocab 512
 *   --tinyllama            22 layers, d=2048, 32/4 heads, ffn 5632, vocab 32000
 *   --model-dir DIR        shape from DIR/config.json (load_config_json)
 *   --mgw FILE             native .mgw weights (mgw_load)
 * Synthetic models are seeded random-init (q48_synth.h, --seed).
 *
 * Then greedy generate (llama_int.c:3067-3135) from a seeded prompt of
 * --prompt-len ids in [3, vocab) or an explicit --prompt "1,2,3", for
 * --max-new tokens.  Prints the token stream, --hash prints FNV-1a-64 of
 * each step's logits, and KPI lines named like llama_int's
 * (llama_int.c:271-285).  --write-mgw FILE exports the synthetic model.
 */
#include "q48_host.h"
#include "q48_synth.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void usage(void)
{
    fprintf(stderr,
            "usage: intllm_run (--tiny|--tinyllama|--model-dir DIR|--mgw FILE) [--seed N]\n"
            "                  [--prompt-len P | --prompt a,b,c] [--max-new N] [--max-seq S]\n"
            "                  [--threads T] [--device D] [--hash] [--write-mgw FILE]\n");
}

int main(int argc, char **argv)
{
    q48h_config cfg = {0};
    const char *mgw = NULL, *dir = NULL, *prompt_s = NULL, *write_mgw = NULL;
    int have_cfg = 0, plen = 16, max_new = 32, max_seq = 0, threads = 8, device = 0, hash = 0;
    uint64_t seed = 0x5EED;
    for (int i = 1; i < argc; ++i) {
        const char *a = argv[i];
        const char *v = i + 1 < argc ? argv[i + 1] : NULL;
        if (!strcmp(a, "--tiny")) {
            cfg = (q48h_config){256, 8, 2, 32, 2, 688, 512, 2048, 10000};
            have_cfg = 1;
        } else if (!strcmp(a, "--tinyllama")) {
            cfg = (q48h_config){2048, 32, 4, 64, 22, 5632, 32000, 2048, 10000};
            have_cfg = 1;
        } else if (!strcmp(a, "--model-dir") && v) {
            dir = v; ++i;
        } else if (!strcmp(a, "--mgw") && v) {
            mgw = v; ++i;
        } else if (!strcmp(a, "--seed") && v) {
            seed = strtoull(v, NULL, 0); ++i;
        } else if (!strcmp(a, "--prompt-len") && v) {
            plen = atoi(v); ++i;
        } else if (!strcmp(a, "--prompt") && v) {
            prompt_s = v; ++i;
        } else if (!strcmp(a, "--max-new") && v) {
            max_new = atoi(v); ++i;
        } else if (!strcmp(a, "--max-seq") && v) {
            max_seq = atoi(v); ++i;
        } else if (!strcmp(a, "--threads") && v) {
            threads = atoi(v); ++i;
        } else if (!strcmp(a, "--device") && v) {
            device = atoi(v); ++i;
        } else if (!strcmp(a, "--hash")) {
            hash = 1;
        } else if (!strcmp(a, "--write-mgw") && v) {
            write_mgw = v; ++i;
        } else {
            usage();
            return 2;
        }
    }
    if (dir) {
        int rc = q48h_config_from_json(dir, &cfg);
        if (rc) {
            fprintf(stderr, "config.json: %s (%d)\n", rc == -1 ? "not found" : "invalid", rc);
            return 1;
        }
        have_cfg = 1;
    }
    if (max_seq > 0 && have_cfg)
        cfg.max_seq = max_seq;
    if (write_mgw) {
        if (!have_cfg) {
            usage();
            return 2;
        }
        int rc = q48h_mgw_write_synth(write_mgw, &cfg, seed, threads);
        printf("wrote %s: %s\n", write_mgw, q48_strerror(rc));
        return rc ? 1 : 0;
    }
    if (!have_cfg && !mgw) {
        usage();
        return 2;
    }

    q48_ctx *ctx = NULL;
    int rc = q48_ctx_create(&ctx, device);
    if (rc) {
        fprintf(stderr, "q48_ctx_create: %s\n", q48_strerror(rc));
        return 1;
    }
    q48h_model *m = NULL;
    if (mgw)
        rc = q48h_model_load_mgw(&m, ctx, mgw, max_seq);
    else {
        rc = q48h_model_create(&m, ctx, &cfg);
        if (!rc)
            rc = q48h_model_synth(m, seed, threads);
    }
    if (rc) {
        fprintf(stderr, "model: %s\n", q48_strerror(rc));
        q48_ctx_destroy(ctx);
        return 1;
    }
    const q48h_config *c = q48h_model_config(m);

    int *prompt = (int *)calloc((size_t)c->max_seq + 1, sizeof(int));
    if (prompt_s) {
        plen = 0;
        for (const char *p = prompt_s; *p && plen < c->max_seq;) {
            prompt[plen++] = (int)strtol(p, (char **)&p, 10);
            while (*p == ',' || *p == ' ')
                p++;
        }
    } else {
        if (plen < 1 || plen > c->max_seq)
            plen = 1;
        q48s_tokens(prompt, plen, seed ^ 0x9E3779B97F4A7C15ULL, 3, c->vocab);
    }
    int cap = plen + (max_new > 0 ? max_new : 0) + 1;
    int *out = (int *)calloc((size_t)cap, sizeof(int));
    uint64_t *hs = hash ? (uint64_t *)calloc((size_t)cap, sizeof(uint64_t)) : NULL;
    int steps = 0;
    q48h_stats st = {0};
    int total = q48h_generate(m, prompt, plen, max_new, out, hs, &steps, &st);
    if (total < 0) {
        fprintf(stderr, "generate: %s\n", q48_strerror(total));
        rc = 1;
    } else {
        printf("Tokens: [");
        for (int i = 0; i < total; ++i)
            printf(i ? ", %d" : "%d", out[i]);
        printf("]\n");
        if (hs)
            for (int i = 0; i < steps; ++i)
                printf("step %d logits_fnv=%016llx\n", i, (unsigned long long)hs[i]);
        double pf = st.prefill_tokens ? 1e3 * st.prefill_s / st.prefill_tokens : 0;
        double dc = st.decode_tokens ? 1e3 * st.decode_s / st.decode_tokens : 0;
        printf("KPI:prefill_ms_per_tok=%.3f\n", pf);
        printf("KPI:decode_ms_per_tok=%.3f\n", dc);
        /* llama_int.c:283-285: prompt and generated tokens over the whole
         * generate() time */
        double gen_s = st.prefill_s + st.decode_s;
        int gen_tok = st.prefill_tokens + st.decode_tokens;
        printf("KPI:tok_per_sec=%.2f\n", gen_s > 0 ? gen_tok / gen_s : 0.0);
    }
    free(prompt);
    free(out);
    free(hs);
    q48h_model_free(m);
    q48_ctx_destroy(ctx);
    return rc;
}
