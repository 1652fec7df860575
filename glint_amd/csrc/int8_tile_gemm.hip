/* W8A16 tile GEMM over an INT8 pin linear on gfx950 (reference cuda/int8_tile_gemm.cu).
 *
 * y[m, n] = sum_k x[m, k] * bf16(q[n, k] * scale[(n * k_in + k) / 64]), f32 out.
 *
 * k_tile_mfma<..., Int8PinTileProducer, TileOutF32> (tile_mfma.h) — k_in % 64 == 0 with
 *   16-B aligned x and q: each thread turns 16 int8 weights of one row (one 16-B load) into
 *   BF16 RNE((float)q * scale) in LDS, and v_mfma_f32_16x16x32_bf16 accumulates in f32.
 *   Tiles: 256 x 128 over 8 waves for m >= 256, 128 x 64 for m > 64, 64 x 64 below.
 * k_i8tile_generic — any k_in and alignment: 64 (n) x 32 (m) output tiles, weights
 *   dequantized to BF16 and widened to f32 in LDS per 32-wide K step, f32 FMAs in k order.
 *   A row's scale index is the flat (n * k_in + k) / 64, so a K step may span two blocks.
 */
#include <algorithm>

#include "glint_common.h"
#include "int8_tile_gemm.h"
#include "tile_mfma.h"

#define I8G_N 64
#define I8G_M 32
#define I8G_K 32
#define I8_MAX_YBLOCKS 65535 /* grid.y limit: M tiles per launch */

__device__ __forceinline__ float i8_dequant_bf16(int8_t q, float s) {
    return __uint_as_float((uint32_t)glint_f32_to_bf16((float)q * s) << 16);
}

__global__ __launch_bounds__(256) void k_i8tile_generic(const uint16_t *__restrict__ x, const int8_t *__restrict__ q,
                                                        const float *__restrict__ scale, float *__restrict__ y, int M,
                                                        int N, int K) {
    __shared__ float ws[I8G_K][I8G_N + 1];
    __shared__ float xsh[I8G_K][I8G_M + 1];
    const int n0 = blockIdx.x * I8G_N, m0 = blockIdx.y * I8G_M;
    const int tid = threadIdx.x;
    const int tn = tid & 15, tm = tid >> 4; /* outputs n = n0 + tn + 16 i (i < 4), m = m0 + tm + 16 j (j < 2) */
    float acc[4][2] = {{0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}};
    for (int k0 = 0; k0 < K; k0 += I8G_K) {
        for (int e = tid; e < I8G_N * I8G_K; e += 256) {
            const int r = e / I8G_K, c = e % I8G_K;
            const int n = n0 + r, k = k0 + c;
            float wv = 0.0f;
            if (n < N && k < K) {
                const int64_t i = (int64_t)n * K + k;
                wv = i8_dequant_bf16(q[i], scale[i / INT8_PIN_BLOCK]);
            }
            ws[c][r] = wv;
        }
        for (int e = tid; e < I8G_M * I8G_K; e += 256) {
            const int r = e / I8G_K, c = e % I8G_K;
            const int m = m0 + r, k = k0 + c;
            xsh[c][r] = (m < M && k < K) ? __uint_as_float((uint32_t)x[(int64_t)m * K + k] << 16) : 0.0f;
        }
        __syncthreads();
        const int kend = min(I8G_K, K - k0);
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
            if (n < N && m < M)
                y[(int64_t)m * N + n] = acc[i][j];
        }
}

template <int BM, int BN, int WM, int WN>
static void i8tile_launch_fast(const uint16_t *x, const Int8PinLinear &w, float *y, int m, hipStream_t st) {
    const Int8PinTileProducer p{(const glint_u32x4 *)w.q, w.scale, w.n_out, w.k_in};
    const unsigned gx = (unsigned)((w.n_out + BN - 1) / BN);
    for (int64_t r0 = 0; r0 < m; r0 += (int64_t)I8_MAX_YBLOCKS * BM) {
        const int mm = (int)std::min<int64_t>((int64_t)I8_MAX_YBLOCKS * BM, m - r0);
        k_tile_mfma<BM, BN, WM, WN, Int8PinTileProducer, TileOutF32><<<dim3(gx, (mm + BM - 1) / BM), 64 * WM * WN, 0, st>>>(
            p, x + r0 * w.k_in, y + r0 * w.n_out, mm, w.n_out, w.k_in);
    }
}

GLINT_API int int8_tile_gemm_bf16(const void *x_bf16, Int8PinLinear w, float *y, int m, hipStream_t stream) {
    const hipError_t pending = hipGetLastError();
    if (pending != hipSuccess)
        return (int)pending;
    if (m < 0 || w.n_out <= 0 || w.k_in <= 0 || !x_bf16 || !w.q || !w.scale || !y)
        return (int)hipErrorInvalidValue;
    if (m == 0)
        return (int)hipSuccess;
    const uint16_t *x = (const uint16_t *)x_bf16;
    const bool fast = (w.k_in % INT8_PIN_BLOCK) == 0 && glint_aligned(x, 16) && glint_aligned(w.q, 16) &&
                      glint_aligned(w.scale, 4);
    if (fast) {
        if (m >= 256)
            i8tile_launch_fast<256, 128, 4, 2>(x, w, y, m, stream);
        else if (m > 64)
            i8tile_launch_fast<128, 64, 2, 2>(x, w, y, m, stream);
        else
            i8tile_launch_fast<64, 64, 2, 2>(x, w, y, m, stream);
    } else {
        const unsigned gx = (unsigned)((w.n_out + I8G_N - 1) / I8G_N);
        for (int64_t r0 = 0; r0 < m; r0 += (int64_t)I8_MAX_YBLOCKS * I8G_M) {
            const int mm = (int)std::min<int64_t>((int64_t)I8_MAX_YBLOCKS * I8G_M, m - r0);
            k_i8tile_generic<<<dim3(gx, (mm + I8G_M - 1) / I8G_M), 256, 0, stream>>>(
                x + r0 * w.k_in, w.q, w.scale, y + r0 * w.n_out, mm, w.n_out, w.k_in);
        }
    }
    return (int)hipGetLastError();
}
