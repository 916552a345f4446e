/*
 * consumer.c -- a C caller of libzinfer_hip through include/zinfer_hip.h
 * alone, standing in for the Zig shim that binds the same symbols with
 * `extern fn` (there is no Zig toolchain to build that shim here).  It drives
 * the host-row API the way src/gen.zig drives Sampler (src/sampler.zig:38-286):
 * init with params and a seed, accept the prompt, then per step sample one
 * host row and accept the token; plus argmaxWithMargin on the same rows.
 *
 * Input file (little-endian): u32 rows, u32 vocab, u32 seed, u32 n_prompt,
 * u32 prompt[n_prompt], f32 temp, u32 top_k, f32 top_p, f32 min_p,
 * f32 repeat_penalty, then rows x vocab f32 logits.
 * Output (stdout): one line per row: "<tok> <margin bits hex> <argmax tok> <argmax margin bits hex>".
 * Exit status: 0 on success, 2 on an ABI error (message on stderr).
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "zinfer_hip.h"

static int fail(const char *what, int32_t rc) {
    fprintf(stderr, "%s: status %d: %s\n", what, (int)rc, zi_last_error());
    return 2;
}

static int rd(FILE *f, void *p, size_t n) { return fread(p, 1, n, f) == n ? 0 : -1; }

static uint32_t bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}

int main(int argc, char **argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s input.bin\n", argv[0]);
        return 2;
    }
    FILE *f = fopen(argv[1], "rb");
    if (!f) {
        perror("open");
        return 2;
    }
    uint32_t rows, vocab, seed, n_prompt;
    if (rd(f, &rows, 4) || rd(f, &vocab, 4) || rd(f, &seed, 4) || rd(f, &n_prompt, 4)) return 2;
    uint32_t *prompt = malloc((size_t)n_prompt * 4 + 4);
    if (!prompt || rd(f, prompt, (size_t)n_prompt * 4)) return 2;
    zi_params p;
    zi_params_default(&p);
    if (rd(f, &p.temp, 4) || rd(f, &p.top_k, 4) || rd(f, &p.top_p, 4) || rd(f, &p.min_p, 4) ||
        rd(f, &p.repeat_penalty, 4))
        return 2;
    p.seed = seed;
    float *logits = malloc((size_t)rows * vocab * 4);
    float *row = malloc((size_t)vocab * 4);
    if (!logits || !row || rd(f, logits, (size_t)rows * vocab * 4)) return 2;
    fclose(f);

    zi_ctx *ctx = NULL;
    int32_t rc = zi_create(&ctx, 0, 16, (int32_t)vocab);
    if (rc) return fail("zi_create", rc);
    zi_sampler *s = NULL;
    rc = zi_sampler_init(&s, ctx, vocab, &p);
    if (rc) return fail("zi_sampler_init", rc);
    for (uint32_t i = 0; i < n_prompt; ++i) zi_sampler_accept(s, prompt[i]);
    for (uint32_t r = 0; r < rows; ++r) {
        uint32_t tok = 0, atok = 0;
        float margin = 0.0f, amargin = 0.0f;
        memcpy(row, logits + (size_t)r * vocab, (size_t)vocab * 4);
        rc = zi_argmax_with_margin(ctx, row, vocab, &atok, &amargin);
        if (rc) return fail("zi_argmax_with_margin", rc);
        rc = zi_sampler_sample_with_margin(s, row, vocab, &tok, &margin);
        if (rc) return fail("zi_sampler_sample_with_margin", rc);
        zi_sampler_accept(s, tok);
        printf("%u %08x %u %08x\n", tok, bits(margin), atok, bits(amargin));
    }
    zi_sampler_deinit(s);
    zi_destroy(ctx);
    free(prompt);
    free(logits);
    free(row);
    return 0;
}
