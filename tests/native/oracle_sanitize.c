/* Drives every function of the CPU oracle (oracle/glint_oracle.c) once on small inputs that
 * reach its edge paths: odd element counts (the pad nibble), a partial last block, a block
 * size that does not divide the row, zero blocks, NaN and infinite weights, a K that is not
 * a multiple of 64, every INT8 form and the K-major path. Built together with the oracle
 * under -fsanitize=address,undefined -fno-sanitize-recover=all by tests/test_native_checks.py,
 * so an out-of-bounds access, a use of uninitialised heap or undefined arithmetic in the
 * oracle ends the run with a report. It checks no values (the parity tests do); it prints
 * one checksum line and exits 0.
 * Build: gcc -O1 -g -fsanitize=address,undefined -fno-sanitize-recover=all -fopenmp
 *        -ffp-contract=off -I include oracle/glint_oracle.c tests/native/oracle_sanitize.c -lm */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

uint16_t oracle_f32_to_bf16_one(float f);
void oracle_f32_to_bf16(const float *in, int64_t n, uint16_t *out);
int oracle_encode_f32(const float *w, int64_t n, int bs, uint8_t *hole, uint8_t *plug, float *absmax);
int oracle_encode_bf16(const uint16_t *w, int64_t n, int bs, uint8_t *hole, uint8_t *plug, float *absmax,
                       float *scratch);
void oracle_expand_f32(const uint8_t *hole, const uint8_t *plug, const float *absmax, int64_t n, int bs, float *out);
void oracle_expand_bf16(const uint8_t *hole, const uint8_t *plug, const float *absmax, int64_t n, int bs,
                        uint16_t *out);
void oracle_htile_f32(const uint8_t *hole, const uint8_t *plug, const float *absmax, const uint16_t *x, float *y,
                      int M, int N, int K, int bs);
void oracle_htile_f64(const uint8_t *hole, const uint8_t *plug, const float *absmax, const uint16_t *x, double *y,
                      double *abs_sum, int M, int N, int K, int bs);
void oracle_quant_act(const uint16_t *x, int m, int k, int8_t *xq, float *sx);
void oracle_int8_mma_emu(const int8_t *xq, const float *sx, const int8_t *wq, const float *sw, int m, int n, int k,
                         float *y);
void oracle_unpack_res4(const uint8_t *q4, int64_t n, int8_t *out);
void oracle_int8_mma_plug_fused(const int8_t *xq, const float *sx, const int8_t *wq, const float *sw,
                                const int8_t *pq, const float *sp, int m, int n, int k, float *y);
void oracle_quant_act_resid(const uint16_t *x, const int8_t *xq, const float *sx, int m, int k, int8_t *rq,
                            float *sr);
void oracle_int8_gemm_i32(const int8_t *A, const int8_t *B, int M, int N, int K, int row0, int row1, int32_t *C);
void oracle_int8_scale_bf16(const int32_t *C, const float *sa, const float *sb, int M, int N, uint16_t *out);
void oracle_int8_pin_dequant_bf16(const int8_t *q, const float *scale, int64_t n, uint16_t *out);
void oracle_int8_tile_f64(const uint16_t *x, const int8_t *q, const float *scale, int M, int N, int K, double *y,
                          double *abs_sum);
void oracle_kmajor_pack(const uint8_t *hole, const uint8_t *plug, const float *absmax, int N, int K,
                        uint8_t *hole_k, uint8_t *plug_k, float *scales_k);
void oracle_gemv_km_fold(const uint8_t *hole_k, const float *scales_k, const uint16_t *x, int N, int K, int ksg,
                         float *y);
int oracle_select_price_key(const uint16_t *x, int K, int tkey);
int oracle_select_ex(const uint16_t *x, int K, int nsel, int tkey, int nfloor, int32_t *idx);
int oracle_select_topk(const uint16_t *x, int K, int nsel, int32_t *idx);
void oracle_apply_corr_km(const uint8_t *hole_k, const uint8_t *plug_k, const float *scales_k, const uint16_t *x,
                          const int32_t *idx, int cnt, int N, int K, int ks, float *y);

static uint32_t rng = 12345u;
static float frand(void) { /* uniform in [-1, 1) */
    rng = rng * 1664525u + 1013904223u;
    return (float)(rng >> 8) / 8388608.0f - 1.0f;
}
static double sum_f(const float *p, int64_t n) {
    double s = 0;
    for (int64_t i = 0; i < n; ++i)
        s += isfinite(p[i]) ? p[i] : 0.0;
    return s;
}
static double sum_u16(const uint16_t *p, int64_t n) {
    double s = 0;
    for (int64_t i = 0; i < n; ++i)
        s += p[i];
    return s;
}

/* encode -> expand on one weight vector of n elements, block size bs */
static double codec(int64_t n, int bs) {
    const int64_t nb = (n + bs - 1) / bs, np = (n + 1) / 2;
    float *w = malloc(n * sizeof(float)), *am = malloc(nb * sizeof(float)), *ef = malloc(n * sizeof(float));
    float *scratch = malloc(n * sizeof(float)), *am2 = malloc(nb * sizeof(float));
    uint16_t *wb = malloc(n * 2), *eb = malloc(n * 2);
    uint8_t *h = malloc(np), *p = malloc(np), *h2 = malloc(np), *p2 = malloc(np);
    for (int64_t i = 0; i < n; ++i)
        w[i] = 0.02f * frand();
    for (int64_t i = 0; i < bs && i < n; ++i)
        w[i] = 0.0f; /* a zero block */
    if (n > 3 * bs) {
        w[bs + 1] = NAN;
        w[2 * bs + 2] = INFINITY;
        w[2 * bs + 3] = -INFINITY;
    }
    oracle_f32_to_bf16(w, n, wb);
    double s = 0;
    if (oracle_encode_f32(w, n, bs, h, p, am) != 0 || oracle_encode_bf16(wb, n, bs, h2, p2, am2, scratch) != 0)
        s = -1e30;
    oracle_expand_f32(h, p, am, n, bs, ef);
    oracle_expand_bf16(h2, p2, am2, n, bs, eb);
    s += sum_f(ef, n) + sum_u16(eb, n) + h[np - 1] + p2[np - 1];
    free(w); free(am); free(ef); free(scratch); free(am2); free(wb); free(eb); free(h); free(p); free(h2); free(p2);
    return s;
}

static double htile(int M, int N, int K, int bs) {
    const int64_t n = (int64_t)N * K, nb = (n + bs - 1) / bs, np = (n + 1) / 2;
    float *w = malloc(n * sizeof(float)), *am = malloc(nb * sizeof(float)), *y = malloc((size_t)M * N * 4);
    double *y64 = malloc((size_t)M * N * 8), *as = malloc((size_t)M * N * 8);
    uint16_t *x = malloc((size_t)M * K * 2);
    uint8_t *h = malloc(np), *p = malloc(np);
    for (int64_t i = 0; i < n; ++i)
        w[i] = 0.02f * frand();
    for (int64_t i = 0; i < (int64_t)M * K; ++i)
        x[i] = oracle_f32_to_bf16_one(frand());
    oracle_encode_f32(w, n, bs, h, p, am);
    oracle_htile_f32(h, p, am, x, y, M, N, K, bs);
    oracle_htile_f64(h, p, am, x, y64, as, M, N, K, bs);
    double s = sum_f(y, (int64_t)M * N);
    for (int i = 0; i < M * N; ++i)
        s += (isfinite(y64[i]) ? y64[i] : 0.0) + (isfinite(as[i]) ? as[i] : 0.0);
    free(w); free(am); free(y); free(y64); free(as); free(x); free(h); free(p);
    return s;
}

static double int8(int m, int n, int k) {
    const int nkb = k / 64;
    uint16_t *x = malloc((size_t)m * k * 2), *yb = malloc((size_t)m * n * 2), *dq = malloc((size_t)n * k * 2);
    int8_t *xq = malloc((size_t)m * k), *wq = malloc((size_t)n * k), *pq = malloc((size_t)n * k);
    int8_t *rq = malloc((size_t)m * k);
    uint8_t *q4 = malloc((size_t)n * k / 2);
    float *sx = malloc((size_t)m * nkb * 4), *sw = malloc((size_t)n * nkb * 4), *sp = malloc((size_t)n * nkb * 4);
    float *sr = malloc((size_t)m * nkb * 4), *y = malloc((size_t)m * n * 4), *sa = malloc(m * 4), *sb = malloc(n * 4);
    int32_t *c = malloc((size_t)m * n * 4);
    double *y64 = malloc((size_t)m * n * 8), *as = malloc((size_t)m * n * 8);
    for (int i = 0; i < m * k; ++i)
        x[i] = oracle_f32_to_bf16_one(frand());
    x[1] = oracle_f32_to_bf16_one(NAN);
    for (int i = 0; i < 64; ++i)
        x[(int64_t)(m - 1) * k + i] = 0; /* a zero block of x */
    for (int i = 0; i < n * k; ++i)
        wq[i] = (int8_t)(int)(127 * frand());
    for (int i = 0; i < n * k / 2; ++i) {
        frand();
        q4[i] = (uint8_t)(rng >> 24);
    }
    for (int i = 0; i < n * nkb; ++i)
        sw[i] = sp[i] = 0.01f + 0.001f * (float)(i % 7);
    for (int i = 0; i < m; ++i)
        sa[i] = 0.5f;
    for (int i = 0; i < n; ++i)
        sb[i] = 0.25f;
    oracle_quant_act(x, m, k, xq, sx);
    oracle_int8_mma_emu(xq, sx, wq, sw, m, n, k, y);
    double s = sum_f(y, (int64_t)m * n);
    oracle_unpack_res4(q4, (int64_t)n * k, pq);
    oracle_int8_mma_plug_fused(xq, sx, wq, sw, pq, sp, m, n, k, y);
    oracle_quant_act_resid(x, xq, sx, m, k, rq, sr);
    oracle_int8_gemm_i32(xq, wq, m, n, k, 0, m, c);
    oracle_int8_scale_bf16(c, sa, sb, m, n, yb);
    oracle_int8_pin_dequant_bf16(wq, sw, (int64_t)n * k, dq);
    oracle_int8_tile_f64(x, wq, sw, m, n, k, y64, as);
    s += sum_f(y, (int64_t)m * n) + sum_u16(yb, (int64_t)m * n) + sum_u16(dq, (int64_t)n * k) + rq[0] + sr[0];
    for (int i = 0; i < m * n; ++i)
        s += c[i] + (isfinite(y64[i]) ? y64[i] : 0.0) + (isfinite(as[i]) ? as[i] : 0.0);
    free(x); free(yb); free(dq); free(xq); free(wq); free(pq); free(rq); free(q4); free(sx); free(sw); free(sp);
    free(sr); free(y); free(sa); free(sb); free(c); free(y64); free(as);
    return s;
}

static double kmajor(int N, int K, int ksg, int ks) {
    const int64_t n = (int64_t)N * K;
    float *w = malloc(n * 4), *am = malloc(n / 64 * 4), *sk = malloc(n / 64 * 4), *y = malloc(N * 4);
    uint8_t *h = malloc(n / 2), *p = malloc(n / 2), *hk = malloc(n / 2), *pk = malloc(n / 2);
    uint16_t *x = malloc(K * 2);
    int32_t *idx = malloc(K * 4);
    for (int64_t i = 0; i < n; ++i)
        w[i] = 0.02f * frand();
    for (int i = 0; i < K; ++i)
        x[i] = oracle_f32_to_bf16_one(frand());
    oracle_encode_f32(w, n, 64, h, p, am);
    oracle_kmajor_pack(h, p, am, N, K, hk, pk, sk);
    oracle_gemv_km_fold(hk, sk, x, N, K, ksg, y);
    const int key = oracle_select_price_key(x, K, 3);
    const int cnt = oracle_select_topk(x, K, K / 10, idx);
    const int cnt2 = oracle_select_ex(x, K, K / 10, 2, 4, idx);
    oracle_apply_corr_km(hk, pk, sk, x, idx, cnt2, N, K, ks, y);
    const double s = sum_f(y, N) + key + cnt + cnt2;
    free(w); free(am); free(sk); free(y); free(h); free(p); free(hk); free(pk); free(x); free(idx);
    return s;
}

int main(void) {
    double s = 0;
    s += codec(64 * 5 + 7, 64); /* odd n, partial last block */
    s += codec(1000, 7);        /* a block size that does not divide 64 */
    s += codec(1, 64);
    s += htile(3, 5, 70, 64);   /* K not a multiple of 64 */
    s += htile(2, 9, 64, 7);
    s += int8(3, 5, 128);
    s += kmajor(32, 256, 2, 2);
    printf("oracle under sanitizers: checksum %.6g\n", s);
    return 0;
}
