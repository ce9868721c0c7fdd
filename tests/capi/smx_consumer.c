/* smx_consumer.c -- a C99 program that uses libsmx.so only through include/smx.h, as a host
 * written in neither Python nor .NET would: it checks that the header is plain C (built with
 * -std=c99 -pedantic -Werror) and drives the library from a process of its own.
 *
 *   smx_consumer info MODEL.gguf
 *       no device work: version, block geometry, the file's configuration and tensor count
 *   smx_consumer generate MODEL.gguf N_NEW OUT.bin TOKEN...
 *       device 0: load the model, one session, greedy generation of N_NEW tokens after the
 *       prompt TOKEN...; OUT.bin receives the N_NEW tokens (int32) and their logits (float32,
 *       N_NEW x vocab).  Then a cancel requested before a second generation must stop it at
 *       its first check (SMX_ECANCELED, no tokens).
 *   smx_consumer suite MODEL.gguf TOKEN...
 *       device 0: the other host-heavy entry points on one model -- lockstep generation of
 *       three sessions, a continuous batcher with a greedy and a sampled member (one leaves
 *       between steps), sampled generation, and a Q8_0 weight through the host-memory operator
 *       (checked here against its own dequantization) -- printing what each produced.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "smx.h"

static void check(int rc, const char *what)
{
    if (rc != SMX_OK) {
        fprintf(stderr, "%s: status %d: %s\n", what, rc, smx_last_error());
        exit(2);
    }
}

static int info(const char *path)
{
    smx_model_config c;
    int64_t n = 0;
    printf("version %s\n", smx_version());
    printf("q4_k %d %d %lld\n", smx_type_block_elems(SMX_TYPE_Q4_K), smx_type_block_bytes(SMX_TYPE_Q4_K),
           (long long)smx_type_row_bytes(SMX_TYPE_Q4_K, 4096));
    check(smx_gguf_read_config(path, &c, &n), "smx_gguf_read_config");
    printf("config %d %d %d %d %d %d %d %d %.9g %.9g %lld\n", c.arch, c.vocab, c.ctx, c.d_model, c.n_layer,
           c.n_head, c.n_kv_head, c.d_ff, (double)c.rope_theta, (double)c.norm_eps, (long long)n);
    return 0;
}

static int generate(const char *path, int n_new, const char *out_path, int n_prompt, char **tokens)
{
    smx_context *ctx = NULL;
    smx_model *m = NULL;
    smx_session *s = NULL;
    smx_model_config c;
    smx_gen_stats st;
    int64_t n_tensors = 0;
    int32_t *prompt, *out;
    float *logits;
    FILE *f;
    int i, rc;

    if (n_new < 1 || n_prompt < 1) return 1;
    check(smx_gguf_read_config(path, &c, &n_tensors), "smx_gguf_read_config");
    prompt = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_prompt);
    out = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_new);
    logits = (float *)malloc(sizeof(float) * (size_t)n_new * (size_t)c.vocab);
    if (!prompt || !out || !logits) return 3;
    for (i = 0; i < n_prompt; i++) prompt[i] = (int32_t)atoi(tokens[i]);

    check(smx_context_create(0, &ctx), "smx_context_create");
    check(smx_model_load_gguf(ctx, path, &m), "smx_model_load_gguf");
    check(smx_session_create(m, n_prompt + n_new, &s), "smx_session_create");
    check(smx_session_generate(s, prompt, n_prompt, n_new, out, logits, &st), "smx_session_generate");
    printf("tokens");
    for (i = 0; i < n_new; i++) printf(" %d", out[i]);
    printf("\nsteps %d %d\n", st.n_prefill_steps, st.n_decode_steps);

    f = fopen(out_path, "wb");
    if (!f) return 4;
    if (fwrite(out, sizeof(int32_t), (size_t)n_new, f) != (size_t)n_new ||
        fwrite(logits, sizeof(float), (size_t)n_new * (size_t)c.vocab, f) != (size_t)n_new * (size_t)c.vocab)
        return 4;
    fclose(f);

    /* a cancel requested while no call runs stops the next generation at its first check */
    check(smx_session_reset(s), "smx_session_reset");
    check(smx_session_cancel(s), "smx_session_cancel");
    rc = smx_session_generate(s, prompt, n_prompt, n_new, out, NULL, &st);
    for (i = 0; i < n_new && out[i] == -1; i++) {
    }
    printf("cancel %d %d %d\n", rc, st.n_decode_steps, i == n_new);

    check(smx_session_destroy(s), "smx_session_destroy");
    check(smx_model_destroy(m), "smx_model_destroy");
    check(smx_context_destroy(ctx), "smx_context_destroy");
    free(prompt);
    free(out);
    free(logits);
    return 0;
}

static void print_row(const char *tag, const int32_t *t, int n)
{
    int i;
    printf("%s", tag);
    for (i = 0; i < n; i++) printf(" %d", t[i]);
    printf("\n");
}

static int suite(const char *path, int n_prompt, char **tokens)
{
    enum { NS = 3, NB = 16, NK = 256, NR = 64, NM = 5 };
    smx_context *ctx = NULL;
    smx_model *m = NULL;
    smx_session *s[NS];
    smx_batcher *b = NULL;
    smx_weight *w = NULL;
    smx_sampling sp;
    smx_gen_stats st;
    int32_t *prompts, lens[NS], out[NS * NB], steps[2 * 6];
    static uint8_t blocks[NR * (NK / 32) * 34];
    static float act[NM * NK], y[NM * NR], wf[NR * NK];
    double worst = 0.0;
    int i, j, r;

    prompts = (int32_t *)malloc(sizeof(int32_t) * (size_t)(NS * n_prompt));
    if (!prompts) return 3;
    for (i = 0; i < NS; i++) {   /* session i: the prompt rotated by i */
        lens[i] = n_prompt;
        for (j = 0; j < n_prompt; j++) prompts[i * n_prompt + j] = (int32_t)atoi(tokens[(i + j) % n_prompt]);
    }
    check(smx_context_create(0, &ctx), "smx_context_create");
    check(smx_model_load_gguf(ctx, path, &m), "smx_model_load_gguf");
    for (i = 0; i < NS; i++) check(smx_session_create(m, n_prompt + NB, &s[i]), "smx_session_create");

    check(smx_batch_generate(s, NS, prompts, lens, NB, out, &st), "smx_batch_generate");
    for (i = 0; i < NS; i++) print_row(i == 0 ? "batch0" : i == 1 ? "batch1" : "batch2", out + i * NB, NB);

    memset(&sp, 0, sizeof(sp));
    sp.temperature = 0.8f;
    sp.top_k = 40;
    sp.top_p = 0.95;
    sp.repetition_penalty = 1.1f;
    for (i = 0; i < NS; i++) check(smx_session_reset(s[i]), "smx_session_reset");
    check(smx_batcher_create(m, 2, n_prompt + NB, &b), "smx_batcher_create");
    check(smx_batcher_add(b, s[0], prompts, n_prompt), "smx_batcher_add");
    check(smx_batcher_add_sampled(b, s[1], prompts + n_prompt, n_prompt, &sp, 5), "smx_batcher_add_sampled");
    check(smx_batcher_step(b, 6, steps), "smx_batcher_step");
    print_row("batcher_greedy", steps, 6);
    print_row("batcher_sampled", steps + 6, 6);
    check(smx_batcher_remove(b, s[0]), "smx_batcher_remove");
    printf("batcher_count %d\n", smx_batcher_count(b));
    check(smx_batcher_step(b, 3, steps), "smx_batcher_step");
    print_row("batcher_after_leave", steps, 3);
    check(smx_batcher_destroy(b), "smx_batcher_destroy");

    check(smx_session_reset(s[2]), "smx_session_reset");
    check(smx_session_generate_sampled(s[2], prompts, n_prompt, 10, &sp, 9, out, NULL, &st), "smx_session_generate_sampled");
    print_row("sampled", out, 10);

    /* a Q8_0 weight [NR][NK]: scale 2^-7 (fp16 0x2000), codes from a fixed sequence */
    for (r = 0; r < NR * (NK / 32); r++) {
        uint8_t *blk = blocks + 34 * r;
        blk[0] = 0x00;
        blk[1] = 0x20;
        for (j = 0; j < 32; j++) blk[2 + j] = (uint8_t)((r * 37 + j * 11) % 255);
    }
    for (i = 0; i < NM * NK; i++) act[i] = (float)((i * 7919) % 200 - 100) / 64.0f;
    check(smx_weight_create(SMX_TYPE_Q8_0, NR, NK, blocks, 0, &w), "smx_weight_create");
    check(smx_weight_to_float32_host(w, wf), "smx_weight_to_float32_host");
    check(smx_weight_matmul_host(w, act, y, NM, NK, NR), "smx_weight_matmul_host");
    for (i = 0; i < NM; i++)
        for (r = 0; r < NR; r++) {
            double ref = 0.0, scale = 0.0;
            for (j = 0; j < NK; j++) {
                ref += (double)act[i * NK + j] * (double)wf[r * NK + j];
                scale += fabs((double)act[i * NK + j] * (double)wf[r * NK + j]);
            }
            if (scale > 0.0 && fabs((double)y[i * NR + r] - ref) / scale > worst) worst = fabs((double)y[i * NR + r] - ref) / scale;
        }
    printf("weight_matmul_host worst %.3g\n", worst);
    check(smx_weight_destroy(w), "smx_weight_destroy");

    for (i = 0; i < NS; i++) check(smx_session_destroy(s[i]), "smx_session_destroy");
    check(smx_model_destroy(m), "smx_model_destroy");
    check(smx_context_destroy(ctx), "smx_context_destroy");
    free(prompts);
    return 0;
}

int main(int argc, char **argv)
{
    setvbuf(stdout, NULL, _IOLBF, 0);   /* each result line leaves the process as it is printed */
    if (argc == 3 && !strcmp(argv[1], "info")) return info(argv[2]);
    if (argc >= 6 && !strcmp(argv[1], "generate")) return generate(argv[2], atoi(argv[3]), argv[4], argc - 5, argv + 5);
    if (argc >= 4 && !strcmp(argv[1], "suite")) return suite(argv[2], argc - 3, argv + 3);
    fprintf(stderr, "usage: smx_consumer info MODEL.gguf | generate MODEL.gguf N_NEW OUT.bin TOKEN... | suite MODEL.gguf TOKEN...\n");
    return 1;
}
