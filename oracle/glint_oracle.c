/* TEST INFRASTRUCTURE ONLY — the CPU oracle for GLINT's hot path.
 *
 * Plain-C restatement of the reference's arithmetic, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker. Nothing
 * in glint_amd/ links, loads or calls it. Every function cites the reference file:line
 * whose semantics it restates. Build: oracle/Makefile -> oracle/liboracle.so.
 *
 * Pinning (what checks each function, see tests/test_oracle.py):
 *   oracle_encode_*    known answers (gpu_ok vector, zero block, NaN, odd pad), the numpy
 *                      searchsorted restatement on the reference's own edge corpus, and a
 *                      pure-Python f64 restatement of glint_codec.encode on the
 *                      reference's seeded data;
 *   oracle_expand_*    a single f32 multiply; BF16 RNE known answers from
 *                      test_glint_tools.py:31-37; the -0.0 zero-block answer;
 *   oracle_htile_*     float64 brute force and the Python tile simulator order;
 *   oracle_quant_act / oracle_int8_*   exact integer brute force (numpy int64 matmul)
 *                      and rint ties-to-even known answers; the plug forms by nibble known
 *                      answers, a zero plug (equal to the base) and power-of-two scales on
 *                      small integers (every f32 step exact, so fused, two-pass and the
 *                      integer formula agree bit for bit); the residual by the rounding
 *                      bound |r - rq sr| <= sr / 2 and the sign of the reconstruction;
 *                      fmaf (the fused last step of the W8A8 epilogue and the residual)
 *                      against exact rational arithmetic, and the fused emulation against
 *                      the reference test's separate-step one within its 1e-5 gate;
 *   oracle_kmajor_pack / oracle_gemv_km_fold / oracle_select_topk / oracle_apply_corr_km
 *                      the K-major round trip against a numpy transpose; one-hot x (a single
 *                      term, so y is PARENT[h] * s or delta * s exactly); the selection
 *                      against a numpy sort (the nsel-th largest key, ties kept); two-hot x
 *                      whose exact answers differ between a run (round(P1 + P2) * s) and two
 *                      parts (round(P1 s) + round(P2 s)); fold plus the full correction
 *                      against the f64 H-TILE sum;
 *   oracle_int8_pin_* / oracle_int8_tile_f64   BF16 rounding known answers (ties to even on
 *                      exact halfway products), the flat scale index on k_in % 64 != 0
 *                      against a numpy restatement, and exact integer results for
 *                      power-of-two scales (numpy int64 matmul).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../include/glint_cells.h"

#define EXPORT __attribute__((visibility("default")))

static float bf16_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* f32 -> bf16 bits, round to nearest even, NaN -> (u >> 16) | 0x40
 * (glint_np.py:25-31, dtype_io.py:32-42). */
EXPORT uint16_t oracle_f32_to_bf16_one(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if (isnan(f))
        return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

EXPORT void oracle_f32_to_bf16(const float *in, int64_t n, uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        out[i] = oracle_f32_to_bf16_one(in[i]);
}

/* nearest16(): first index of the minimum |v - tab[k]|, strict '<'
 * (glint_encode.cu:67-79). */
static int nearest16(const float *tab, float v) {
    int best = 0;
    float bd = fabsf(v - tab[0]);
    for (int k = 1; k < 16; ++k) {
        const float d = fabsf(v - tab[k]);
        if (d < bd) {
            bd = d;
            best = k;
        }
    }
    return best;
}

/* Block absmax: max |w| over the block, NaN skipped because fabsf(NaN) > m is false
 * (glint_encode.cu:41-66, glint_np.py:32-40). */
static void block_absmax(const float *w, int64_t n, int bs, float *absmax) {
    const int64_t nb = (n + bs - 1) / bs;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nb; ++b) {
        float m = 0.f;
        const int64_t e = (b + 1) * bs < n ? (b + 1) * bs : n;
        for (int64_t i = b * bs; i < e; ++i) {
            const float a = fabsf(w[i]);
            if (a > m)
                m = a;
        }
        absmax[b] = m;
    }
}

/* Encode (glint_encode.cu:80-102): v = (s == 0) ? 0 : w / s in f32; hole = nearest
 * parent, plug = nearest child of that parent; element 2e in the low nibble of byte e,
 * 2e+1 in the high nibble, high pad nibble 0 for odd n. Returns 0, or -1 for bs <= 0. */
EXPORT int oracle_encode_f32(const float *w, int64_t n, int bs, uint8_t *hole, uint8_t *plug, float *absmax) {
    if (bs <= 0 || n < 0)
        return -1;
    block_absmax(w, n, bs, absmax);
    const int64_t npack = (n + 1) / 2;
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < npack; ++e) {
        int h[2] = {0, 0}, p[2] = {0, 0};
        for (int t = 0; t < 2; ++t) {
            const int64_t i = 2 * e + t;
            if (i >= n)
                break;
            const float s = absmax[i / bs];
            const float v = (s == 0.f) ? 0.f : (w[i] / s);
            h[t] = nearest16(GLINT_PARENT, v);
            p[t] = nearest16(GLINT_CELLS[h[t]], v);
        }
        hole[e] = (uint8_t)((h[0] & 15) | ((h[1] & 15) << 4));
        plug[e] = (uint8_t)((p[0] & 15) | ((p[1] & 15) << 4));
    }
    return 0;
}

/* BF16 input: widen (exact) then encode (glint_encode.cu:35-40, 182-204). `scratch`
 * holds n floats. */
EXPORT int oracle_encode_bf16(const uint16_t *w, int64_t n, int bs, uint8_t *hole, uint8_t *plug, float *absmax,
                              float *scratch) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        scratch[i] = bf16_to_f32(w[i]);
    return oracle_encode_f32(scratch, n, bs, hole, plug, absmax);
}

static inline int nib(const uint8_t *pk, int64_t i) { return (pk[i >> 1] >> (4 * (int)(i & 1))) & 15; }

/* out[i] = CELLS[h][p] * absmax[i / bs] (glint_encode.cu:103-114, glint_np.py:84-92). */
EXPORT void oracle_expand_f32(const uint8_t *hole, const uint8_t *plug, const float *absmax, int64_t n, int bs,
                              float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        out[i] = GLINT_CELLS[nib(hole, i)][nib(plug, i)] * absmax[i / bs];
}

/* Unpin to BF16: RNE of the f32 expand (glint_unpin.py:25-32). */
EXPORT void oracle_expand_bf16(const uint8_t *hole, const uint8_t *plug, const float *absmax, int64_t n, int bs,
                               uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        out[i] = oracle_f32_to_bf16_one(GLINT_CELLS[nib(hole, i)][nib(plug, i)] * absmax[i / bs]);
}

/* H-TILE, f32 in the reference kernel's order (glint_htile.cu:142-163,
 * glint_htile_sim.py:22-50): acc += (cell * absmax) * x for k ascending. */
EXPORT void oracle_htile_f32(const uint8_t *hole, const uint8_t *plug, const float *absmax, const uint16_t *x,
                             float *y, int M, int N, int K, int bs) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float acc = 0.f;
            for (int k = 0; k < K; ++k) {
                const int64_t i = (int64_t)n * K + k;
                const float wv = GLINT_CELLS[nib(hole, i)][nib(plug, i)] * absmax[i / bs];
                acc += wv * bf16_to_f32(x[(int64_t)m * K + k]);
            }
            y[(int64_t)m * N + n] = acc;
        }
}

/* Same sum in double (test_htile_k_bounds_device.cu:90-98); also returns
 * sum |terms| per output in `abs_sum` (may be NULL) for error bounds. */
EXPORT void oracle_htile_f64(const uint8_t *hole, const uint8_t *plug, const float *absmax, const uint16_t *x,
                             double *y, double *abs_sum, int M, int N, int K, int bs) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double acc = 0, aacc = 0;
            for (int k = 0; k < K; ++k) {
                const int64_t i = (int64_t)n * K + k;
                const double t = (double)(GLINT_CELLS[nib(hole, i)][nib(plug, i)] * absmax[i / bs]) *
                                 (double)bf16_to_f32(x[(int64_t)m * K + k]);
                acc += t;
                aacc += fabs(t);
            }
            y[(int64_t)m * N + n] = acc;
            if (abs_sum)
                abs_sum[(int64_t)m * N + n] = aacc;
        }
}

/* float -> int32 the way the reference's CUDA `(int)` cast converts (PTX cvt.rzi.s32.f32:
 * NaN -> 0, out-of-range values saturate); a plain C cast of NaN is undefined. */
static int cvt_s32(float f) {
    if (f != f)
        return 0;
    if (f >= 2147483648.0f)
        return 2147483647;
    if (f <= -2147483648.0f)
        return (int)0x80000000u;
    return (int)f;
}

/* Activation quantization per (row, 64-block): s = amax > 0 ? amax / 127 : 1,
 * q = clamp(rint(x / s), -127, 127) (int8_mma_gemm.cu:11-29). k % 64 == 0. */
EXPORT void oracle_quant_act(const uint16_t *x, int m, int k, int8_t *xq, float *sx) {
    const int nkb = k / 64;
#pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < m; ++r)
        for (int kb = 0; kb < nkb; ++kb) {
            const int64_t base = (int64_t)r * k + (int64_t)kb * 64;
            float am = 0.f;
            for (int t = 0; t < 64; ++t)
                am = fmaxf(am, fabsf(bf16_to_f32(x[base + t])));
            const float s = (am > 0.f) ? (am / 127.f) : 1.f;
            sx[(int64_t)r * nkb + kb] = s;
            for (int t = 0; t < 64; ++t) {
                int v = cvt_s32(rintf(bf16_to_f32(x[base + t]) / s));
                v = v > 127 ? 127 : (v < -127 ? -127 : v);
                xq[base + t] = (int8_t)v;
            }
        }
}

/* W8A8 per-64-slice arithmetic of the reference kernel (cuda/int8_mma_gemm.cu:105-118) as
 * its build compiles it (nvcc -O2, default --fmad=true, scripts/build_p7_kernels.sh:7):
 * ic = exact int32 sum over the slice; acc = fmaf(RN((float)ic * sx), sw, acc), kb
 * ascending. */
EXPORT void oracle_int8_mma_emu(const int8_t *xq, const float *sx, const int8_t *wq, const float *sw, int m, int n,
                                int k, float *y) {
    const int nkb = k / 64;
#pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j) {
            float acc = 0.f;
            for (int kb = 0; kb < nkb; ++kb) {
                int ic = 0;
                for (int t = 0; t < 64; ++t)
                    ic += (int)xq[(int64_t)i * k + kb * 64 + t] * (int)wq[(int64_t)j * k + kb * 64 + t];
                const float a = (float)ic * sx[(int64_t)i * nkb + kb];
                acc = fmaf(a, sw[(int64_t)j * nkb + kb], acc);
            }
            y[(int64_t)i * n + j] = acc;
        }
}

/* The reference test's host emulation (tests/test_int8_mma_gemm.cu:102-112): the same with
 * the last multiply and add separate, acc += ((float)ic * sx) * sw. Its gate against the
 * kernel is 1e-5 relative (test_int8_mma_gemm.cu:207). */
EXPORT void oracle_int8_mma_emu_sep(const int8_t *xq, const float *sx, const int8_t *wq, const float *sw, int m,
                                    int n, int k, float *y) {
    const int nkb = k / 64;
#pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j) {
            float acc = 0.f;
            for (int kb = 0; kb < nkb; ++kb) {
                int ic = 0;
                for (int t = 0; t < 64; ++t)
                    ic += (int)xq[(int64_t)i * k + kb * 64 + t] * (int)wq[(int64_t)j * k + kb * 64 + t];
                const float a = (float)ic * sx[(int64_t)i * nkb + kb];
                const float p = a * sw[(int64_t)j * nkb + kb];
                acc = acc + p;
            }
            y[(int64_t)i * n + j] = acc;
        }
}

/* fmaf over arrays (the oracle's fused multiply-add, pinned against exact rational
 * arithmetic in the tests) */
EXPORT void oracle_fmaf_n(const float *a, const float *b, const float *c, int64_t n, float *out) {
    for (int64_t i = 0; i < n; ++i)
        out[i] = fmaf(a[i], b[i], c[i]);
}

/* p7_plug_res4_v1 slice to int8 (cuda/int8_mma_gemm.cu:157-163): element i is nibble i of
 * the packed bytes, low nibble first, minus 8. */
EXPORT void oracle_unpack_res4(const uint8_t *q4, int64_t n, int8_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        out[i] = (int8_t)((int)((q4[i >> 1] >> ((i & 1) * 4)) & 15u) - 8);
}

/* Fused late plug (cuda/int8_mma_gemm.cu:105-124,224-240): per kb, the base term then the
 * plug term go into one accumulator: acc = fmaf(ic*sx, sw, acc); acc = fmaf(ip*sx, sp, acc). */
EXPORT void oracle_int8_mma_plug_fused(const int8_t *xq, const float *sx, const int8_t *wq, const float *sw,
                                       const int8_t *pq, const float *sp, int m, int n, int k, float *y) {
    const int nkb = k / 64;
#pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j) {
            float acc = 0.f;
            for (int kb = 0; kb < nkb; ++kb) {
                int ic = 0, ip = 0;
                for (int t = 0; t < 64; ++t) {
                    const int a = xq[(int64_t)i * k + kb * 64 + t];
                    ic += a * (int)wq[(int64_t)j * k + kb * 64 + t];
                    ip += a * (int)pq[(int64_t)j * k + kb * 64 + t];
                }
                const float xs = sx[(int64_t)i * nkb + kb];
                acc = fmaf((float)ic * xs, sw[(int64_t)j * nkb + kb], acc);
                acc = fmaf((float)ip * xs, sp[(int64_t)j * nkb + kb], acc);
            }
            y[(int64_t)i * n + j] = acc;
        }
}

/* Activation quantization residual re-quantized (cuda/int8_mma_gemm.cu:182-200): per (row,
 * 64-block) r = fmaf(-(float)xq, sx, x) (the reference's x - xq * sx under nvcc's default
 * contraction),
 * s = amax|r| > 0 ? amax / 127 : 1 (NaN skipped), rq = clamp(cvt(rint(r / s)), -127, 127). */
EXPORT void oracle_quant_act_resid(const uint16_t *x, const int8_t *xq, const float *sx, int m, int k, int8_t *rq,
                                   float *sr) {
    const int nkb = k / 64;
#pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < m; ++r)
        for (int kb = 0; kb < nkb; ++kb) {
            const int64_t base = (int64_t)r * k + (int64_t)kb * 64;
            const float s0 = sx[(int64_t)r * nkb + kb];
            float res[64], am = 0.f;
            for (int t = 0; t < 64; ++t) {
                res[t] = fmaf(-(float)xq[base + t], s0, bf16_to_f32(x[base + t]));
                am = fmaxf(am, fabsf(res[t]));
            }
            const float s = (am > 0.f) ? (am / 127.f) : 1.f;
            sr[(int64_t)r * nkb + kb] = s;
            for (int t = 0; t < 64; ++t) {
                int v = cvt_s32(rintf(res[t] / s));
                v = v > 127 ? 127 : (v < -127 ? -127 : v);
                rq[base + t] = (int8_t)v;
            }
        }
}

/* Raw INT8 GEMM: C[m,n] = sum_k A[m,k] * B[n,k] in int32 (exact: |C| <= K*127^2).
 * Only rows [row0, row1) are computed (a bounded sample for timing). */
EXPORT void oracle_int8_gemm_i32(const int8_t *A, const int8_t *B, int M, int N, int K, int row0, int row1,
                                 int32_t *C) {
    (void)M;
#pragma omp parallel for collapse(2) schedule(static)
    for (int i = row0; i < row1; ++i)
        for (int j = 0; j < N; ++j) {
            int32_t acc = 0;
            const int8_t *a = A + (int64_t)i * K, *b = B + (int64_t)j * K;
            for (int t = 0; t < K; ++t)
                acc += (int32_t)a[t] * (int32_t)b[t];
            C[(int64_t)i * N + j] = acc;
        }
}

/* Scaled output of the raw GEMM: bf16 RNE of ((float)C * sa[m]) * sb[n]. */
EXPORT void oracle_int8_scale_bf16(const int32_t *C, const float *sa, const float *sb, int M, int N, uint16_t *out) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j)
            out[(int64_t)i * N + j] = oracle_f32_to_bf16_one(((float)C[(int64_t)i * N + j] * sa[i]) * sb[j]);
}

/* W8A16 over an INT8 pin linear (int8_tile_gemm.h:10-27, test_int8_tile_gemm.cu:53-55,
 * 89-113): weight i = bf16 RNE((float)q[i] * scale[i / 64]) over the flat index
 * i = n * K + k; bits of every weight of W [N, K]. */
EXPORT void oracle_int8_pin_dequant_bf16(const int8_t *q, const float *scale, int64_t n, uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        out[i] = oracle_f32_to_bf16_one((float)q[i] * scale[i / 64]);
}

/* y[m, n] = sum_k x[m, k] * w[n, k] in double with w the BF16 dequant above, and the sum
 * of |terms| per output (the reference's check: |got - dot| <= 1e-4 * absdot). */
EXPORT void oracle_int8_tile_f64(const uint16_t *x, const int8_t *q, const float *scale, int M, int N, int K,
                                 double *y, double *abs_sum) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double acc = 0, aacc = 0;
            for (int k = 0; k < K; ++k) {
                const int64_t i = (int64_t)n * K + k;
                const float w = bf16_to_f32(oracle_f32_to_bf16_one((float)q[i] * scale[i / 64]));
                const double t = (double)bf16_to_f32(x[(int64_t)m * K + k]) * (double)w;
                acc += t;
                aacc += fabs(t);
            }
            y[(int64_t)m * N + n] = acc;
            abs_sum[(int64_t)m * N + n] = aacc;
        }
}

/* ---------------------------------------------------------------- K-major decode path
 * K-major layout (p7_glint_select_decode.mojo:126-142, p7_select_device.mojo:196-206):
 * hole_k[c * N/2 + r/2] holds element (r, c), even r in the low nibble; plug_k the same;
 * scales_k[(c / 64) * N + r] = absmax[r * K/64 + c / 64]. N even, K % 64 == 0, bs 64. */
EXPORT void oracle_kmajor_pack(const uint8_t *hole, const uint8_t *plug, const float *absmax, int N, int K,
                               uint8_t *hole_k, uint8_t *plug_k, float *scales_k) {
    const int64_t half = N / 2;
#pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < (int64_t)K * half; ++g) {
        const int64_t c = g / half, r0 = 2 * (g % half);
        const int64_t j0 = r0 * K + c, j1 = (r0 + 1) * K + c;
        hole_k[g] = (uint8_t)(nib(hole, j0) | (nib(hole, j1) << 4));
        plug_k[g] = (uint8_t)(nib(plug, j0) | (nib(plug, j1) << 4));
    }
    const int nb = K / 64;
#pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < (int64_t)N * nb; ++g)
        scales_k[(g % nb) * N + g / nb] = absmax[g];
}

static inline int nib_k(const uint8_t *pk, int64_t c, int64_t half, int r) {
    return (pk[c * half + (r >> 1)] >> (4 * (r & 1))) & 15;
}

/* Summation orders of the K-major fold and correction. The reference fixes the terms
 * (p7_glint_gemv_km.mojo:17-94: (PARENT[h] * scale) * x over slices of channels combined
 * in order) and states that its slice order is a choice validated on its gate; this build
 * fixes its own order, which the GPU kernels follow exactly:
 * - a list of channels is cut into KM_SUB equal parts per workgroup;
 * - each part is walked in order as runs of channels inside one 64-block:
 *   acc = fmaf(v, x[c], acc) over a run from 0, then t = fmaf(acc, scale(r, block), t);
 * - the KM_SUB part sums are added in order, then the outer slices in order. */
#define KM_SUB 8

/* t for channels [c0, c1) of row r; val(r, c) is PARENT[h] (fold) or CELLS[h][p] - PARENT[h]. */
static float km_runs(const uint8_t *hole_k, const uint8_t *plug_k, const float *scales_k, const uint16_t *x,
                     const int32_t *list, int i0, int i1, int N, int r, int corr) {
    const int64_t half = N / 2;
    float t = 0.f, acc = 0.f;
    int cur = -1;
    for (int i = i0; i < i1; ++i) {
        const int c = list ? list[i] : i;
        if ((c >> 6) != cur) {
            if (cur >= 0)
                t = fmaf(acc, scales_k[(int64_t)cur * N + r], t);
            cur = c >> 6;
            acc = 0.f;
        }
        const int h = nib_k(hole_k, c, half, r);
        const float v = corr ? GLINT_CELLS[h][nib_k(plug_k, c, half, r)] - GLINT_PARENT[h] : GLINT_PARENT[h];
        acc = fmaf(v, bf16_to_f32(x[c]), acc);
    }
    if (cur >= 0)
        t = fmaf(acc, scales_k[(int64_t)cur * N + r], t);
    return t;
}

/* Parent-only (fold) GEMV on the K-major hole: y[r] = sum_c PARENT[h] * scale * x[c] with
 * K cut into ksg outer slices of KM_SUB parts each, in the order above. */
EXPORT void oracle_gemv_km_fold(const uint8_t *hole_k, const float *scales_k, const uint16_t *x, int N, int K,
                                int ksg, float *y) {
    const int ksl = K / ksg, sub = ksl / KM_SUB;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < N; ++r) {
        float tot = 0.f;
        for (int g = 0; g < ksg; ++g) {
            float wg = 0.f;
            for (int q = 0; q < KM_SUB; ++q) {
                const int c0 = g * ksl + q * sub;
                const float t = km_runs(hole_k, NULL, scales_k, x, NULL, c0, c0 + sub, N, r, 0);
                wg = (q == 0) ? t : wg + t;
            }
            tot = (g == 0) ? wg : tot + wg;
        }
        y[r] = tot;
    }
}

/* Selection (p7_select_device.mojo:1-151): key = bf16 bits & 0x7FFF.
 *   rank(n): the largest 15-bit T with #{key >= T} >= n, found bit by bit from the top
 *            (:31-48); n <= 0 leaves every bit set (T = 32767), n > K leaves T = 0.
 *   T = rank(nsel) (the cap);
 *   tkey > 0: T = max(T, tkey) (price, :51-54);
 *   tkey < 0: tau = -tkey / 1024, m = mean |x| summed in f32 over 1024 thread ranges of
 *             ceil(K / 1024) channels and a pairwise tree (:55-77), t = m * tau as
 *             (sum / K) * (-tkey) / 1024 in f32, its key r = biased exponent << 7 | 7 mantissa
 *             bits by truncation, clamped to [1, 32767], 1 when t <= 0 (:78-92);
 *             T = max(T, r);
 *   nfloor > 0 and tkey != 0: T = max(cap, min(T, rank(nfloor))) (:93-114);
 *   nsel == 0: T = 32768, nothing kept (:115-117).
 * Writes the kept channels in ascending order, returns the count. */
static int sel_rank(const uint16_t *x, int K, int n) {
    int thr = 0;
    for (int bi = 0; bi < 15; ++bi) {
        const int cand = thr | (1 << (14 - bi));
        int cnt = 0;
        for (int i = 0; i < K; ++i)
            cnt += (x[i] & 0x7FFF) >= cand;
        if (cnt >= n)
            thr = cand;
    }
    return thr;
}

/* |x| of a key from its exponent and mantissa fields, 2^(e-134) clamped to
 * [2^-60, 2^40]; 0 for zero and subnormal keys (p7_select_device.mojo:60-74) */
static float sel_mag(int k) {
    const int ex = k >> 7;
    if (ex <= 0)
        return 0.0f;
    int n = ex - 134;
    n = n > 40 ? 40 : n < -60 ? -60 : n;
    return ldexpf((float)(128 + (k & 127)), n); /* exact: a power-of-two scale of an 8-bit integer */
}

EXPORT int oracle_select_price_key(const uint16_t *x, int K, int tkey) {
    enum { SB = 1024 };
    float red[SB];
    const int per = (K + SB - 1) / SB;
    for (int t = 0; t < SB; ++t) {
        const int lo = t * per, hi = lo + per < K ? lo + per : K;
        float acc = 0.0f;
        for (int i = lo; i < hi; ++i)
            acc += sel_mag(x[i] & 0x7FFF);
        red[t] = acc;
    }
    for (int off = SB / 2; off >= 1; off >>= 1)
        for (int t = 0; t < off; ++t)
            red[t] = red[t] + red[t + off];
    float tv = red[0] / (float)K * (float)(-tkey) / 1024.0f;
    int rk = 1;
    if (tv > 0.0f) {
        int e2 = 0;
        while (tv >= 2.0f && e2 < 100) {
            tv *= 0.5f;
            ++e2;
        }
        while (tv < 1.0f && e2 > -120) {
            tv *= 2.0f;
            --e2;
        }
        rk = ((e2 + 127) << 7) | (int)((tv - 1.0f) * 128.0f);
        rk = rk < 1 ? 1 : rk > 32767 ? 32767 : rk;
    }
    return rk;
}

EXPORT int oracle_select_threshold(const uint16_t *x, int K, int nsel, int tkey, int nfloor) {
    const int cap = sel_rank(x, K, nsel);
    int thr = cap;
    if (tkey > thr)
        thr = tkey;
    if (tkey < 0) {
        const int rk = oracle_select_price_key(x, K, tkey);
        if (rk > thr)
            thr = rk;
    }
    if (nfloor > 0 && tkey != 0) {
        const int thf = sel_rank(x, K, nfloor);
        if (thf < thr)
            thr = thf;
        if (thr < cap)
            thr = cap;
    }
    if (nsel == 0)
        thr = 32768;
    return thr;
}

EXPORT int oracle_select_ex(const uint16_t *x, int K, int nsel, int tkey, int nfloor, int32_t *idx) {
    const int thr = oracle_select_threshold(x, K, nsel, tkey, nfloor);
    int n = 0;
    for (int i = 0; i < K; ++i)
        if ((x[i] & 0x7FFF) >= thr)
            idx[n++] = i;
    return n;
}

EXPORT int oracle_select_topk(const uint16_t *x, int K, int nsel, int32_t *idx) {
    return oracle_select_ex(x, K, nsel, 0, 0, idx);
}

/* Plug correction over the selected channels (p7_select_device.mojo:208-236, 253-302):
 * y[r] = y[r] + sum_i (CELLS[h][p] - PARENT[h]) * scale * x[c_i]. The list is cut into
 * ks chunks of ceil(cnt / ks), each chunk into KM_SUB parts of ceil(chunk / KM_SUB), summed
 * in the order above; y is updated in place. */
EXPORT void oracle_apply_corr_km(const uint8_t *hole_k, const uint8_t *plug_k, const float *scales_k,
                                 const uint16_t *x, const int32_t *idx, int cnt, int N, int K, int ks, float *y) {
    (void)K;
    const int chunk = (cnt + ks - 1) / ks, sub = (chunk + KM_SUB - 1) / KM_SUB;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < N; ++r) {
        float tot = 0.f;
        for (int s = 0; s < ks; ++s) {
            const int lo = s * chunk, hi = lo + chunk < cnt ? lo + chunk : cnt;
            float wg = 0.f;
            for (int q = 0; q < KM_SUB; ++q) {
                const int i0 = lo + q * sub < hi ? lo + q * sub : hi;
                const int i1 = i0 + sub < hi ? i0 + sub : hi;
                const float t = km_runs(hole_k, plug_k, scales_k, x, idx, i0, i1, N, r, 1);
                wg = (q == 0) ? t : wg + t;
            }
            tot = (s == 0) ? wg : tot + wg;
        }
        y[r] = y[r] + tot;
    }
}

EXPORT int oracle_threads(void) {
#ifdef _OPENMP
    extern int omp_get_max_threads(void);
    return omp_get_max_threads();
#else
    return 1;
#endif
}
