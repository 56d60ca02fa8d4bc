/* The oracle (oracle/oracle.c, compiled into this file) under AddressSanitizer
 * and UndefinedBehaviorSanitizer: every exported function on small ragged
 * shapes, each buffer allocated at exactly the size its function documents,
 * so a read or write past it (or any undefined behaviour) aborts the run.
 * Values are not checked here (the Python pins do that). */
#include "../../oracle/oracle.c"

#include <stdio.h>

static uint32_t lcg = 12345u;
static float frand(void) {
    lcg = lcg * 1664525u + 1013904223u;
    return ((float)(lcg >> 8) / (float)(1u << 24)) * 2.0f - 1.0f;
}
static void *xmalloc(size_t bytes) {
    void *p = malloc(bytes ? bytes : 1);
    if (!p) { fprintf(stderr, "malloc\n"); exit(2); }
    return p;
}
static uint16_t *rand16(size_t len) {
    uint16_t *p = xmalloc(len * 2);
    for (size_t i = 0; i < len; i++) p[i] = or_f32_to_f16(frand());
    return p;
}
static float *randf(size_t len) {
    float *p = xmalloc(len * 4);
    for (size_t i = 0; i < len; i++) p[i] = frand();
    return p;
}

int main(void) {
    const size_t shapes[][3] = {{1, 1, 1}, {3, 5, 7}, {2, 37, 70}, {4, 130, 33}, {1, 64, 257}};
    const size_t blocks[] = {16, 32, 64, 128};
    for (size_t si = 0; si < sizeof shapes / sizeof shapes[0]; si++) {
        const size_t m = shapes[si][0], n = shapes[si][1], k = shapes[si][2];
        for (size_t bi = 0; bi < 4; bi++) {
            const size_t block = blocks[bi], nbk = (k + block - 1) / block;
            float *w = randf(n * k);
            uint16_t *a = rand16(m * k);
            for (int layout = 0; layout < 2; layout++) {
                /* Q4: quantize, dequant (both forms), band pack, threaded matmul */
                for (int affine = 0; affine < 2; affine++) {
                    uint8_t *quants = xmalloc((k * n + 1) / 2);
                    uint16_t *scales = xmalloc(n * nbk * 2), *mins = affine ? xmalloc(n * nbk * 2) : NULL;
                    or_q4_quantize(w, layout, n, k, block, affine, quants, scales, mins);
                    uint16_t *deq = xmalloc(k * n * 2);
                    or_q4_dequant_f16(quants, scales, mins, n, k, block, deq);
                    or_q4_dequant_bf16(quants, scales, mins, n, k, block, deq);
                    size_t nib_len, sc_len;
                    or_q4_band_sizes(n, k, block, &nib_len, &sc_len);
                    uint8_t *nib = xmalloc(nib_len);
                    uint16_t *bsc = xmalloc(sc_len * 2), *bmn = affine ? xmalloc(sc_len * 2) : NULL;
                    or_q4_pack_band(quants, scales, mins, n, k, block, nib, bsc, bmn);
                    uint16_t *c = xmalloc(m * n * 2);
                    if (!affine && block >= 32 && or_matmul_mt(4, a, quants, scales, NULL, m, n, k, block, c, 3))
                        return 3;
                    free(quants); free(scales); free(mins); free(deq); free(nib); free(bsc); free(bmn); free(c);
                }
                /* Q2 and Q1: quantize, reference, dequant, band pack, threaded matmul */
                const int8_t cb[4] = {-1, 0, 1, 0};
                uint8_t *codes = xmalloc((k * n + 3) / 4), *signs = xmalloc((k * n + 7) / 8);
                uint16_t *s2 = xmalloc(n * nbk * 2), *s1 = xmalloc(n * nbk * 2);
                if (or_q2_quantize(w, layout, n, k, block, cb, codes, s2)) return 4;
                or_q1_quantize(w, layout, n, k, block, signs, s1);
                int8_t *sq = xmalloc(k);
                float *ss = xmalloc(nbk * 4);
                uint16_t *c = xmalloc(m * n * 2), *deq = xmalloc(k * n * 2);
                or_lowbit_reference(2, a, codes, s2, cb, 1, m, n, k, block, c, sq, ss);
                or_lowbit_reference(1, a, signs, s1, NULL, 0, m, n, k, block, c, sq, ss);
                or_lowbit_dequant_f16(2, codes, s2, cb, 1, n, k, block, deq);
                or_lowbit_dequant_f16(1, signs, s1, NULL, 0, n, k, block, deq);
                for (int kind = 1; kind <= 2; kind++) {
                    size_t codes_len, lsc_len;
                    or_lowbit_band_sizes(kind, n, k, block, &codes_len, &lsc_len);
                    uint8_t *packed = xmalloc(codes_len);
                    uint16_t *lsc = xmalloc(lsc_len * 2);
                    or_lowbit_pack_band(kind, kind == 2 ? codes : signs, kind == 2 ? s2 : s1, kind == 2, n, k,
                                        block, packed, lsc);
                    free(packed); free(lsc);
                }
                if (or_matmul_mt(2, a, codes, s2, cb, m, n, k, block, c, 2)) return 5;
                if (or_matmul_mt(1, a, signs, s1, NULL, m, n, k, block, c, 4)) return 6;
                or_quantize_row(a, k, block, sq, ss);
                free(codes); free(signs); free(s2); free(s1); free(sq); free(ss); free(c); free(deq);
            }
            free(w);
            free(a);
        }
        /* dense GEMMs (row- and column-major, strided with alpha), epilogue */
        uint16_t *a = rand16(m * k), *b = rand16(k * n), *c = xmalloc(m * n * 2);
        float *acc = xmalloc(n * 4);
        or_gemm_f16(m, n, k, c, a, b, 0x3C00, 0, acc);
        or_gemm_bf16(m, n, k, c, a, b, 0x3F80, 1, acc);
        or_gemm_strided(0, m, n, k, c, 1, m, a, 1, m, b, 1, k, 0x3800, 0x3C00, acc);
        uint16_t *row = rand16(m), *col = rand16(n), *ten = rand16(m * n);  /* ROW ops index i, COL ops j */
        OrEpNode nodes[4] = {{OP_ADD_ROW, 0, 0.0f, row, 0}, {OP_MUL_COL, 0, 0.0f, col, 0},
                             {OP_SUB_TENSOR, 0, 0.0f, ten, 0}, {OP_ACT, 3, 0.0f, NULL, 0}};
        or_apply_ep(c, m, n, n, 1, nodes, 4, 5, 0);
        free(a); free(b); free(c); free(acc); free(row); free(col); free(ten);
    }
    /* decode-block passes */
    {
        const size_t dim = 77, rows = 3, hd = 16, heads = 4, kv_heads = 2, len = 9;
        float *x = randf(rows * dim), *wn = randf(dim), *scratch = xmalloc(dim * 4);
        uint16_t *y = xmalloc(rows * dim * 2);
        or_rms_norm_f16(x, wn, rows, dim, 1e-5f, y, scratch);
        float *inv = xmalloc(hd / 2 * 4), *cs = xmalloc(hd / 2 * 4), *sn = xmalloc(hd / 2 * 4);
        or_rope_inv_freq(hd, 10000.0, inv);
        or_rope_angles(inv, hd / 2, 5, cs, sn);
        float *q = randf(heads * hd);
        or_rope_apply(q, heads * hd, cs, sn, hd / 2);
        uint16_t *kc = rand16(len * kv_heads * hd), *vc = rand16(len * kv_heads * hd);
        float *out = xmalloc(heads * hd * 4), *scores = xmalloc(len * 4), *qh = xmalloc(hd * 4);
        or_attention_kv_f16(q, kc, vc, len, heads, kv_heads, hd, 0.25f, out, scores, qh);
        uint16_t *both = rand16(rows * 2 * 45), *g = xmalloc(rows * 45 * 2);
        or_glu_f16(g, both, rows, 45, 0);
        or_glu_f16(g, both, rows, 45, 1);
        free(x); free(wn); free(scratch); free(y); free(inv); free(cs); free(sn); free(q);
        free(kc); free(vc); free(out); free(scores); free(qh); free(both); free(g);
    }
    /* conversions and activations over special values */
    const float sp[] = {0.0f, -0.0f, 1.0f, -1.0f, 65504.0f, 70000.0f, 1e-8f, -1e-8f, INFINITY, -INFINITY, NAN};
    for (size_t i = 0; i < sizeof sp / sizeof sp[0]; i++) {
        (void)or_f32_to_f16(sp[i]);
        (void)or_f32_to_bf16(sp[i]);
        (void)or_f64_to_f16((double)sp[i]);
        for (uint32_t kind = 1; kind <= 24; kind++) {
            (void)or_act_f64(kind, (double)sp[i], 0.1);
            (void)or_act_f32(kind, sp[i], 0.1f);
        }
    }
    for (uint32_t h = 0; h < 65536; h++) (void)or_f16_to_f32((uint16_t)h);
    puts("oracle asan ok");
    return 0;
}
