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
 */
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

int main(int argc, char **argv)
{
    if (argc == 3 && !strcmp(argv[1], "info")) return info(argv[2]);
    if (argc >= 6 && !strcmp(argv[1], "generate")) return generate(argv[2], atoi(argv[3]), argv[4], argc - 5, argv + 5);
    fprintf(stderr, "usage: smx_consumer info MODEL.gguf | generate MODEL.gguf N_NEW OUT.bin TOKEN...\n");
    return 1;
}
