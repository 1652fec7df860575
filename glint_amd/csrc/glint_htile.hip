/* GLINT H-TILE GEMV / GEMM for gfx950.
 *
 * y[m, n] = sum_k CELLS[h][p] * absmax[(n*K + k) / bs] * x[m, k]
 * (reference cuda/glint_htile.cu:124-164 and glint_htile_sim.py:22-50; f32 arithmetic).
 *
 * k_htile_gemv_b64 — decode (M = 1), bs = 64, K % 64 == 0: HBM-bound. A wave owns R
 *   weight rows; lane l reads 8 B of each plane per row per step (16 consecutive k inside
 *   one absmax block), so one wave load is 512 contiguous bytes. x is staged once per
 *   workgroup in LDS (bf16); the cell table sits in LDS as 32 bank-private copies, so the
 *   per-element lookups never conflict. Per row: 16 f32 FMAs per lane per step, then one
 *   FMA by the block absmax, then a wave reduction.
 * k_htile_mfma_b64 — prefill (M > 1, bf16 out, bs = 64): BF16 MFMA on LDS-dequantized
 *   weight tiles, f32 accumulation.
 * k_htile_generic — every other shape (any M, K, bs, alignment): 64x32 output tiles,
 *   weights decoded to f32 in LDS per 32-wide K step, f32 FMAs in k order.
 */
#include "glint_common.h"
#include "glint_htile.h"

/* ---------------------------------------------------------------- GEMV (M = 1) */
#define GEMV_THREADS 512
/* x (K bf16) + the 33 KiB tables stay within the default 64 KiB of LDS per block */
#define GEMV_MAX_K 15360

template <int R>
struct GemvRows {
    glint_u32x2 h[R], p[R];
    float a[R];
};

template <int R>
__device__ __forceinline__ void gemv_load(GemvRows<R> &s, const glint_u32x2 *__restrict__ hole,
                                          const glint_u32x2 *__restrict__ plug, const float *__restrict__ absmax,
                                          int n0, int N, int K, int j, bool ok) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = n0 + r;
        if (ok && n < N) {
            const int64_t cj = (int64_t)n * (K >> 4) + j; /* 16-element chunk index */
            s.h[r] = __builtin_nontemporal_load(&hole[cj]);
            s.p[r] = __builtin_nontemporal_load(&plug[cj]);
            s.a[r] = absmax[cj >> 2];
        } else {
            s.h[r] = glint_u32x2{0u, 0u};
            s.p[r] = glint_u32x2{0u, 0u};
            s.a[r] = 0.0f;
        }
    }
}

template <int R, bool OUT_BF16>
__global__ __launch_bounds__(GEMV_THREADS) void k_htile_gemv_b64(const glint_u32x2 *__restrict__ hole,
                                                                 const glint_u32x2 *__restrict__ plug,
                                                                 const float *__restrict__ absmax,
                                                                 const glint_u32x4 *__restrict__ x, void *__restrict__ y,
                                                                 int N, int K) {
    __shared__ float ltab[GLINT_LDS_CELLS_WORDS];
    __shared__ float stage[256];
    extern __shared__ glint_u32x4 xs[]; /* K bf16 */
    for (int i = threadIdx.x; i < (K >> 3); i += blockDim.x)
        xs[i] = x[i];
    glint_fill_cells_lds(ltab, stage);

    const int lane = threadIdx.x & 63;
    const uint32_t lb = lane & 31;
    const int nchunk = K >> 4;
    const int iters = (nchunk + 63) >> 6;
    const int waves_per_block = blockDim.x >> 6;
    const int64_t nwaves = (int64_t)gridDim.x * waves_per_block;
    for (int64_t g = (int64_t)blockIdx.x * waves_per_block + (threadIdx.x >> 6); g * R < N; g += nwaves) {
        const int n0 = (int)(g * R);
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            acc[r] = 0.0f;
        GemvRows<R> cur, nxt;
        gemv_load<R>(cur, hole, plug, absmax, n0, N, K, lane, lane < nchunk);
        for (int it = 0; it < iters; ++it) {
            const int j = it * 64 + lane;
            const bool ok = j < nchunk;
            if (it + 1 < iters)
                gemv_load<R>(nxt, hole, plug, absmax, n0, N, K, j + 64, j + 64 < nchunk);
            glint_u32x4 xa = glint_u32x4{0u, 0u, 0u, 0u}, xb = xa;
            if (ok) {
                xa = xs[2 * j];
                xb = xs[2 * j + 1];
            }
            const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            float xf[16];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                xf[2 * q] = glint_bf16lo(xw[q]);
                xf[2 * q + 1] = glint_bf16hi(xw[q]);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float part = 0.0f;
                const uint32_t H[2] = {cur.h[r].x, cur.h[r].y}, P[2] = {cur.p[r].x, cur.p[r].y};
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const uint32_t E = ((H[q] << 4) & 0xF0F0F0F0u) | (P[q] & 0x0F0F0F0Fu);
                    const uint32_t O = (H[q] & 0xF0F0F0F0u) | ((P[q] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        part = fmaf(ltab[(((E >> (8 * b)) & 0xFFu) << 5) | lb], xf[8 * q + 2 * b], part);
                        part = fmaf(ltab[(((O >> (8 * b)) & 0xFFu) << 5) | lb], xf[8 * q + 2 * b + 1], part);
                    }
                }
                acc[r] = fmaf(cur.a[r], part, acc[r]);
            }
            cur = nxt;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float t = glint_wave_sum(acc[r]);
            if (lane == r && n0 + r < N) {
                if (OUT_BF16)
                    ((uint16_t *)y)[n0 + r] = glint_f32_to_bf16(t);
                else
                    ((float *)y)[n0 + r] = t;
            }
        }
    }
}

/* ------------------------------------------------------------ generic f32 tiles */
#define GT_N 64
#define GT_M 32
#define GT_K 32

__device__ __forceinline__ uint32_t glint_nibble(const uint8_t *pk, int64_t i) {
    return (pk[i >> 1] >> ((uint32_t)(i & 1) * 4)) & 15u;
}

template <bool OUT_BF16>
__global__ __launch_bounds__(256) void k_htile_generic(const uint8_t *__restrict__ hole, const uint8_t *__restrict__ plug,
                                                       const float *__restrict__ absmax, const uint16_t *__restrict__ x,
                                                       void *__restrict__ y, int M, int N, int K, int bs) {
    __shared__ float ws[GT_K][GT_N + 1];
    __shared__ float xsh[GT_K][GT_M + 1];
    const int n0 = blockIdx.x * GT_N, m0 = blockIdx.y * GT_M;
    const int tid = threadIdx.x;
    const int tn = tid & 15, tm = tid >> 4; /* outputs n = n0 + tn + 16*i (i<4), m = m0 + tm + 16*j (j<2) */
    float acc[4][2] = {{0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}};
    for (int k0 = 0; k0 < K; k0 += GT_K) {
        for (int e = tid; e < GT_N * GT_K; e += 256) {
            const int r = e / GT_K, c = e % GT_K;
            const int n = n0 + r, k = k0 + c;
            float wv = 0.0f;
            if (n < N && k < K) {
                const int64_t i = (int64_t)n * K + k;
                wv = kCells[glint_nibble(hole, i)][glint_nibble(plug, i)] * absmax[i / bs];
            }
            ws[c][r] = wv;
        }
        for (int e = tid; e < GT_M * GT_K; e += 256) {
            const int r = e / GT_K, c = e % GT_K;
            const int m = m0 + r, k = k0 + c;
            xsh[c][r] = (m < M && k < K) ? __uint_as_float((uint32_t)x[(int64_t)m * K + k] << 16) : 0.0f;
        }
        __syncthreads();
        const int kend = min(GT_K, K - k0);
        for (int c = 0; c < kend; ++c) {
            float wv[4], xv[2];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                wv[i] = ws[c][tn + 16 * i];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                xv[j] = xsh[c][tm + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = fmaf(wv[i], xv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + tn + 16 * i, m = m0 + tm + 16 * j;
            if (n < N && m < M) {
                if (OUT_BF16)
                    ((uint16_t *)y)[(int64_t)m * N + n] = glint_f32_to_bf16(acc[i][j]);
                else
                    ((float *)y)[(int64_t)m * N + n] = acc[i][j];
            }
        }
}

/* ---------------------------------------------------- prefill GEMM on BF16 MFMA */
/* y[M, N] (bf16) = x[M, K] W^T for bs = 64, K % 64 == 0. Block tile BM x 128 x 64 (K);
 * 4 waves in 2 x 2, wave tile (BM/2) x 64 = (BM/32) x 4 MFMA tiles of 16x16
 * (v_mfma_f32_16x16x32_bf16, two K halves per step). Per K step each thread turns 32
 * packed weights of one row (16 B of each plane) into BF16 RNE(cell * absmax) through
 * the bank-private LDS table and writes them to the W tile; the next step's planes and
 * x tile are loaded from HBM while the MFMAs run. LDS rows are padded by 8 BF16 so the
 * 16 rows read by one MFMA operand load fall in distinct bank groups. */
typedef __bf16 glint_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 glint_bf16x2 __attribute__((ext_vector_type(2)));
typedef float glint_f32x2 __attribute__((ext_vector_type(2)));

#define MF_BN 128
#define MF_LDW 72 /* 64 + 8 bf16 per LDS row */

__device__ __forceinline__ uint32_t glint_cvt_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(glint_f32x2{lo, hi}, glint_bf16x2));
}

template <int BM>
__global__ __launch_bounds__(256) void k_htile_mfma_b64(const glint_u32x4 *__restrict__ hole,
                                                        const glint_u32x4 *__restrict__ plug,
                                                        const float *__restrict__ absmax, const uint16_t *__restrict__ x,
                                                        uint16_t *__restrict__ y, int M, int N, int K) {
    constexpr int WM = BM / 2, TM = WM / 16, XV = BM / 32; /* x u32x4 loads per thread */
    __shared__ float ltab[GLINT_LDS_CELLS_WORDS];
    __shared__ float stage[256];
    __shared__ __attribute__((aligned(16))) uint16_t sX[BM * MF_LDW];
    __shared__ __attribute__((aligned(16))) uint16_t sW[MF_BN * MF_LDW];
    glint_fill_cells_lds(ltab, stage);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * MF_BN;
    const uint32_t lb = lane & 31;
    const int nK = K >> 6;
    /* staging roles: weights row wr = tid >> 1, K half wh = tid & 1 (32 elements) */
    const int wr = tid >> 1, wh = tid & 1;
    const int wn_row = n0 + wr;
    glint_f32x4 acc[TM][4];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
            acc[a][b] = glint_f32x4{0.f, 0.f, 0.f, 0.f};

    glint_u32x4 hv, pv, xv[XV];
    float av;
    auto gload = [&](int kb) {
        if (wn_row < N) {
            const int64_t q = (int64_t)wn_row * (K >> 5) + kb * 2 + wh; /* 32-element groups */
            hv = __builtin_nontemporal_load(&hole[q]);
            pv = __builtin_nontemporal_load(&plug[q]);
            av = absmax[(int64_t)wn_row * (K >> 6) + kb];
        } else {
            hv = pv = glint_u32x4{0u, 0u, 0u, 0u};
            av = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int idx = tid + 256 * i, xr = idx >> 3, xc = idx & 7;
            const int m = m0 + xr;
            xv[i] = (m < M) ? *(const glint_u32x4 *)(x + (int64_t)m * K + (int64_t)kb * 64 + xc * 8)
                            : glint_u32x4{0u, 0u, 0u, 0u};
        }
    };
    gload(0);
    for (int kb = 0; kb < nK; ++kb) {
        /* dequantize this thread's 32 weights and stage x */
        {
            const uint32_t H[4] = {hv.x, hv.y, hv.z, hv.w}, P[4] = {pv.x, pv.y, pv.z, pv.w};
            uint32_t packed[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t E = ((H[q] << 4) & 0xF0F0F0F0u) | (P[q] & 0x0F0F0F0Fu);
                const uint32_t O = (H[q] & 0xF0F0F0F0u) | ((P[q] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const float ve = ltab[(((E >> (8 * b)) & 0xFFu) << 5) | lb] * av;
                    const float vo = ltab[(((O >> (8 * b)) & 0xFFu) << 5) | lb] * av;
                    packed[4 * q + b] = glint_cvt_bf16x2(ve, vo);
                }
            }
            glint_u32x4 *dst = (glint_u32x4 *)(sW + wr * MF_LDW + wh * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                dst[i] = glint_u32x4{packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]};
#pragma unroll
            for (int i = 0; i < XV; ++i) {
                const int idx = tid + 256 * i, xr = idx >> 3, xc = idx & 7;
                *(glint_u32x4 *)(sX + xr * MF_LDW + xc * 8) = xv[i];
            }
        }
        __syncthreads();
        if (kb + 1 < nK)
            gload(kb + 1);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int kofs = ks * 32 + (lane >> 4) * 8;
            glint_bf16x8 af[TM], bfr[4];
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[a] = __builtin_bit_cast(glint_bf16x8,
                                           *(const glint_u32x4 *)(sX + (wm * WM + a * 16 + (lane & 15)) * MF_LDW + kofs));
#pragma unroll
            for (int b = 0; b < 4; ++b)
                bfr[b] = __builtin_bit_cast(glint_bf16x8,
                                            *(const glint_u32x4 *)(sW + (wn * 64 + b * 16 + (lane & 15)) * MF_LDW + kofs));
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[a], bfr[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + wm * WM + a * 16 + (lane >> 4) * 4 + i;
                const int n = n0 + wn * 64 + b * 16 + (lane & 15);
                if (m < M && n < N)
                    y[(int64_t)m * N + n] = glint_f32_to_bf16(acc[a][b][i]);
            }
}

/* ------------------------------------------------------------------ dispatch */
template <bool OUT_BF16>
static int htile_launch(const uint8_t *hole, const uint8_t *plug, const float *absmax, const void *x, void *y, int M,
                        int N, int K, int bs, hipStream_t st) {
    if (!hole || !plug || !absmax || !x || !y)
        return -1;
    if (bs <= 0 || K < 1)
        return -2;
    if (M <= 0 || N <= 0)
        return 0;
    const bool gemv_ok = M == 1 && bs == 64 && (K % 64) == 0 && glint_aligned(hole, 8) && glint_aligned(plug, 8) &&
                         glint_aligned(absmax, 4) && glint_aligned(x, 16) &&
                         K <= GEMV_MAX_K;
    const bool mfma_ok = OUT_BF16 && M > 1 && bs == 64 && (K % 64) == 0 && glint_aligned(hole, 16) &&
                         glint_aligned(plug, 16) && glint_aligned(absmax, 4) && glint_aligned(x, 16);
    if (mfma_ok) {
        const unsigned gx = (unsigned)((N + MF_BN - 1) / MF_BN);
        if (M <= 64) {
            k_htile_mfma_b64<64><<<dim3(gx, (M + 63) / 64), 256, 0, st>>>(
                (const glint_u32x4 *)hole, (const glint_u32x4 *)plug, absmax, (const uint16_t *)x, (uint16_t *)y, M, N, K);
        } else {
            k_htile_mfma_b64<128><<<dim3(gx, (M + 127) / 128), 256, 0, st>>>(
                (const glint_u32x4 *)hole, (const glint_u32x4 *)plug, absmax, (const uint16_t *)x, (uint16_t *)y, M, N, K);
        }
    } else if (gemv_ok) {
        constexpr int R = 4;
        const int64_t groups = ((int64_t)N + R - 1) / R;
        const int waves = GEMV_THREADS / 64;
        const unsigned grid = (unsigned)((groups + waves - 1) / waves);
        k_htile_gemv_b64<R, OUT_BF16><<<grid, GEMV_THREADS, (size_t)K * 2, st>>>(
            (const glint_u32x2 *)hole, (const glint_u32x2 *)plug, absmax, (const glint_u32x4 *)x, y, N, K);
    } else {
        dim3 grid((N + GT_N - 1) / GT_N, (M + GT_M - 1) / GT_M);
        k_htile_generic<OUT_BF16><<<grid, 256, 0, st>>>(hole, plug, absmax, (const uint16_t *)x, y, M, N, K, bs);
    }
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

GLINT_API int launch_glint_htile_s3_f32_stream(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                                               const void *d_x, float *d_y, int M, int N, int K, int bs,
                                               struct ihipStream_t *stream) {
    return htile_launch<false>(d_hole, d_plug, d_absmax, d_x, d_y, M, N, K, bs, (hipStream_t)stream);
}

GLINT_API int launch_glint_htile_s3_f32(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                                        const void *d_x, float *d_y, int M, int N, int K, int bs) {
    return htile_launch<false>(d_hole, d_plug, d_absmax, d_x, d_y, M, N, K, bs, 0);
}

GLINT_API int launch_glint_htile_bf16_stream(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                                             const void *d_x, uint16_t *d_y, int M, int N, int K, int bs,
                                             struct ihipStream_t *stream) {
    return htile_launch<true>(d_hole, d_plug, d_absmax, d_x, d_y, M, N, K, bs, (hipStream_t)stream);
}
