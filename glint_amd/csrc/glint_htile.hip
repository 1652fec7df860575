/* GLINT H-TILE GEMV / GEMM for gfx950.
 *
 * y[m, n] = sum_k CELLS[h][p] * absmax[(n*K + k) / bs] * x[m, k]
 * (reference cuda/glint_htile.cu:124-164 and glint_htile_sim.py:22-50; f32 arithmetic).
 *
 * k_htile_gemv_b64 — decode (M = 1), bs = 64, K % 64 == 0: HBM-bound. A wave owns R
 *   weight rows; lane l reads 8 B of each plane per row per step (16 consecutive k inside
 *   one absmax block), so one wave load is 512 contiguous bytes, and keeps D steps of
 *   loads in flight. x is staged once per workgroup in LDS (bf16); the cell table sits in
 *   LDS as 64 lane-private copies, so lookups never conflict and each lookup address is
 *   one v_perm_b32. Per element: 0.5 op to form code bytes, 1 perm, 1 LDS read, 1 f32
 *   FMA; then one FMA by the block absmax per 16 elements and a wave reduction.
 * k_htile_mfma_b64 — prefill (M > 1, bf16 out, bs = 64): BF16 MFMA on LDS-dequantized
 *   weight tiles, f32 accumulation.
 * k_htile_generic — every other shape (any M, K, bs, alignment): 64x32 output tiles,
 *   weights decoded to f32 in LDS per 32-wide K step, f32 FMAs in k order.
 */
#include "glint_common.h"
#include "glint_htile.h"

/* ---------------------------------------------------------------- GEMV (M = 1) */
#ifndef GEMV_R
#define GEMV_R 2 /* weight rows per wave */
#endif
#ifndef GEMV_D
#define GEMV_D 2 /* row-steps of loads in flight per wave */
#endif
#ifndef GEMV_T
#define GEMV_T 1024 /* threads per workgroup for K <= 8192 */
#endif
/* x (K f32) + the 65 KiB of tables fit in the 160 KiB of LDS */
#define GEMV_MAX_K 16384
#define GEMV_LDS_BYTES(K) ((size_t)(K) * 4 + 64) /* dynamic part: x as f32 + one zero chunk */
/* x is stored as 4 planes of (K/16 + 1) float4: plane q holds floats 4q..4q+3 of every
 * 16-element chunk, so the 64 lanes of one ds_read_b128 read 64 consecutive float4. */

/* Wave task: rows [n0, n0 + R). Step i covers 16-element chunk j = 64 i + lane of every
 * row (8 B of each plane, inside one absmax block). Loads run D steps ahead in a ring of
 * registers (slot d holds steps d, d + D, ...), issued for the first task before the
 * LDS tables are filled. */
template <int R>
__device__ __forceinline__ void gemv_load_step(const glint_u32x2 *__restrict__ hole, const glint_u32x2 *__restrict__ plug,
                                               const float *__restrict__ absmax, int n0, int N, int nch, int it,
                                               int lane, glint_u32x2 (&h)[R], glint_u32x2 (&p)[R], float (&a)[R]) {
    /* unconditional loads: a lane past the row end reads the row's last chunk, gets
     * absmax 0 and x = 0, so it adds exactly 0 */
    const int jr = it * 64 + lane;
    const bool ok = jr < nch;
    const uint32_t j = (uint32_t)min(jr, nch - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        /* row base: wave-uniform (scalar) arithmetic; rows past N reuse row N-1 */
        const int64_t n = min(n0 + r, N - 1);
        h[r] = __builtin_nontemporal_load(hole + n * nch + j);
        p[r] = __builtin_nontemporal_load(plug + n * nch + j);
        const float av = absmax[n * (nch >> 2) + (j >> 2)];
        a[r] = ok ? av : 0.0f;
    }
}

template <int R, int D, int THREADS, bool OUT_BF16>
__global__ __launch_bounds__(THREADS, 4) void k_htile_gemv_b64(const glint_u32x2 *__restrict__ hole,
                                                               const glint_u32x2 *__restrict__ plug,
                                                               const float *__restrict__ absmax,
                                                               const glint_u32x4 *__restrict__ x, void *__restrict__ y,
                                                               int N, int K) {
    __shared__ __attribute__((aligned(16))) float ltab[GLINT_LDS_CELLS64_WORDS]; /* 64 KiB at LDS offset 0 */
    __shared__ float stage[256];
    extern __shared__ __attribute__((aligned(16))) glint_f32x4 xs[]; /* K f32 */

    const int lane = threadIdx.x & 63;
    const uint32_t lane4 = (uint32_t)lane * 4u;
    const int nch = K >> 4;
    const int iters = (nch + 63) >> 6;
    const int wpb = THREADS / 64;
    const int nwaves = gridDim.x * wpb;
    /* wave-uniform task index, so row arithmetic stays in scalar registers */
    int g = blockIdx.x * wpb + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ntasks = (N + R - 1) / R;

    glint_u32x2 rh[D][R], rp[D][R];
    float ra[D][R];
    if (g < ntasks) {
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (d < iters)
                gemv_load_step<R>(hole, plug, absmax, g * R, N, nch, d, lane, rh[d], rp[d], ra[d]);
    }
    const int xplane = nch + 1;
    for (int i = threadIdx.x; i < (K >> 3); i += THREADS) { /* i: 8 bf16 = half a chunk */
        const glint_u32x4 v = x[i];
        const int jj = i >> 1, q0 = (i & 1) * 2;
        xs[q0 * xplane + jj] = glint_f32x4{glint_bf16lo(v.x), glint_bf16hi(v.x), glint_bf16lo(v.y), glint_bf16hi(v.y)};
        xs[(q0 + 1) * xplane + jj] = glint_f32x4{glint_bf16lo(v.z), glint_bf16hi(v.z), glint_bf16lo(v.w), glint_bf16hi(v.w)};
    }
    if (threadIdx.x < 4)
        xs[threadIdx.x * xplane + nch] = glint_f32x4{0.f, 0.f, 0.f, 0.f}; /* chunk nch: zeros */
    glint_fill_cells_lds64(ltab, stage);

    for (; g < ntasks; g += nwaves) {
        const int n0 = g * R;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            acc[r] = 0.0f;
        for (int base = 0; base < iters; base += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const int it = base + d;
                if (it < iters) {
                    /* x of chunk j; lanes past the row end read the zero chunk */
                    const int jc = min(it * 64 + lane, nch);
                    float xf[16];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const glint_f32x4 v = xs[q * xplane + jc];
                        xf[4 * q] = v.x;
                        xf[4 * q + 1] = v.y;
                        xf[4 * q + 2] = v.z;
                        xf[4 * q + 3] = v.w;
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float part = 0.0f;
                        const uint32_t H[2] = {rh[d][r].x, rh[d][r].y}, P[2] = {rp[d][r].x, rp[d][r].y};
#pragma unroll
                        for (int q = 0; q < 2; ++q) {
                            const uint32_t E = glint_codes_even(H[q], P[q]);
                            const uint32_t O = glint_codes_odd(H[q], P[q]);
                            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<0>(E, lane4)), xf[8 * q + 0], part);
                            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<0>(O, lane4)), xf[8 * q + 1], part);
                            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<1>(E, lane4)), xf[8 * q + 2], part);
                            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<1>(O, lane4)), xf[8 * q + 3], part);
                            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<2>(E, lane4)), xf[8 * q + 4], part);
                            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<2>(O, lane4)), xf[8 * q + 5], part);
                            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<3>(E, lane4)), xf[8 * q + 6], part);
                            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<3>(O, lane4)), xf[8 * q + 7], part);
                        }
                        acc[r] = fmaf(ra[d][r], part, acc[r]);
                        /* keep the next row's lookups after this row's FMAs: bounds live registers */
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    if (it + D < iters)
                        gemv_load_step<R>(hole, plug, absmax, n0, N, nch, it + D, lane, rh[d], rp[d], ra[d]);
                }
            }
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
        if (g + nwaves < ntasks) {
#pragma unroll
            for (int d = 0; d < D; ++d)
                if (d < iters)
                    gemv_load_step<R>(hole, plug, absmax, (g + nwaves) * R, N, nch, d, lane, rh[d], rp[d], ra[d]);
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
/* One resident wave of workgroups (every CU filled to its occupancy limit), or fewer if
 * there are fewer wave tasks; the waves then loop over their tasks. */
static unsigned gemv_grid(const void *kern, int threads, size_t lds, int64_t tasks) {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    const int64_t resident = (int64_t)cus * glint_resident_blocks(kern, threads, lds);
    const int64_t needed = (tasks + threads / 64 - 1) / (threads / 64);
    return (unsigned)(needed < resident ? needed : resident);
}

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
        constexpr int R = GEMV_R, D = GEMV_D;
        const size_t lds = GEMV_LDS_BYTES(K);
        const int64_t tasks = ((int64_t)N + R - 1) / R;
        if (K <= 8192) {
            constexpr int T = GEMV_T;
            auto kern = k_htile_gemv_b64<R, D, T, OUT_BF16>;
            if (glint_set_lds_limit((const void *)kern, lds) != 0)
                return -3;
            const unsigned grid = gemv_grid((const void *)kern, T, lds, tasks);
            kern<<<grid, T, lds, st>>>((const glint_u32x2 *)hole, (const glint_u32x2 *)plug, absmax,
                                      (const glint_u32x4 *)x, y, N, K);
        } else {
            constexpr int T = 1024;
            auto kern = k_htile_gemv_b64<R, D, T, OUT_BF16>;
            if (glint_set_lds_limit((const void *)kern, lds) != 0)
                return -3;
            const unsigned grid = gemv_grid((const void *)kern, T, lds, tasks);
            kern<<<grid, T, lds, st>>>((const glint_u32x2 *)hole, (const glint_u32x2 *)plug, absmax,
                                      (const glint_u32x4 *)x, y, N, K);
        }
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
