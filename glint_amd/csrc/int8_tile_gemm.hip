/* W8A16 tile GEMM over an INT8 pin linear on gfx950 (reference cuda/int8_tile_gemm.cu).
 *
 * y[m, n] = sum_k x[m, k] * bf16(q[n, k] * scale[(n * k_in + k) / 64]), f32 out.
 *
 * k_tile_mfma / k_tile_ss<..., Int8PinTileProducer, TileOutF32> (tile_mfma.h) — k_in % 64
 *   == 0 with 16-B aligned x and q, m > 4: threads turn 16 int8 weights of one row into
 *   BF16 RNE((float)q * scale) in LDS, and v_mfma_f32_16x16x32_bf16 accumulates in f32;
 *   K is split across workgroups (fixed-order reduction) when the tiles leave CUs idle.
 *   Tiles: 256 x 128 over 8 waves for m >= 256 (k_tile_mfma), 128 x 64 for m > 64 and
 *   64 x 64 below (k_tile_ss: weight loads cover whole 128-B lines).
 * k_i8tile_gemv<MR> — m <= 4, k_in % 2048 == 0: the GEMV-shaped kernel, v_dot2_f32_bf16.
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
#ifndef I8_SS_PER_CU
#define I8_SS_PER_CU 2 /* k_tile_ss<64> split-K plan: workgroups per CU to fill. Its LDS (80 KB)
                        * and its register cap (256, two waves per SIMD) let two be resident:
                        * m = 64 14336 x 4096 32.6 -> 29.3 us. The 128-row tile (369 VGPRs) got
                        * slower with two, so it keeps one. */
#endif

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

/* ---------------------------------------------------------- small m: GEMV-shaped */
/* m <= 4, k_in % 2048 == 0, k_in / 2048 <= 8 (the decode shapes). Like the GLINT decode
 * GEMV: the row is cut into S = k_in / 2048 slices, wave (s, g) keeps slice s of the m
 * activation rows in registers (32 f32 per lane per row) and streams weight rows
 * r0 + g, r0 + g + G, ... of its workgroup's row range: per row each lane reads 32 int8,
 * vectors l and 64 + l of the slice (two 16-B loads, each instruction 1 KiB contiguous;
 * two 64-blocks, so two scales). Weights are rounded to BF16 exactly as the
 * tile kernels do (v_cvt_pk_bf16_f32 of q * scale); each BF16 weight pair meets the BF16 x
 * pair in one v_dot2_f32_bf16 (both products exact in f32, added into the f32 partial).
 * Against unpacking the pair and two f32 FMAs, with the grid capped at 16 waves per CU
 * (the dot form needs fewer registers, so more workgroups would fit): 14336 x 4096 m = 1
 * 14.5 -> 14.1 us, m = 4 22.6 -> 19.4; 4096 x 14336 m = 1 15.6 -> 13.4, m = 4 25.2 -> 20.7;
 * 8192 x 8192 m = 1 18.4 -> 16.0. Without the cap m = 2 was slower (16.1 -> 17.1).
 * Two rows are in flight per wave (one at m = 2); loads are unconditional (rows clamped at
 * the end).
 * A row's S slice sums (DPP within the wave) meet in LDS and are added in slice order. */
#ifndef I8V_THREADS
#define I8V_THREADS 512
#endif
#ifndef I8V_DEPTH
#define I8V_DEPTH 2 /* rows of loads in flight per wave (I8V_DEPTH_M1 for m = 1, k_in <= 4096; I8V_DEPTH_M2 at m = 2) */
#endif
#ifndef I8V_DEPTH_M1
#define I8V_DEPTH_M1 1
#endif
#ifndef I8V_DEPTH_M2
#define I8V_DEPTH_M2 1 /* rows in flight at m = 2 */
#endif
#define I8V_RED_MAX 8192 /* floats of row partials a workgroup may park in LDS */
#ifndef I8V_WAVES_CU
#define I8V_WAVES_CU 16 /* most waves per CU the grid is sized for (4 per SIMD) */
#endif
#ifndef I8V_GRID_DIV
#define I8V_GRID_DIV 2 /* m = 1, one row group per workgroup (k_in >= 10240): launch the resident grid / this */
#endif

struct I8Row {
    glint_u32x4 q0, q1;
    float s, s1; /* the scales of q0's and q1's 64-blocks */
};
#ifndef I8V_LINE
#define I8V_LINE 1 /* lane l loads vectors l and 64 + l of its slice (1 KiB contiguous per load) */
#endif
#ifndef I8V_DOT2
#define I8V_DOT2 1 /* products of the BF16 weight pair and the BF16 x pair by v_dot2_f32_bf16 */
#endif
typedef __bf16 i8v_bf16x2_t __attribute__((ext_vector_type(2)));

template <int MR, int DEPTH>
__global__ __launch_bounds__(I8V_THREADS) void k_i8tile_gemv(const glint_u32x4 *__restrict__ q,
                                                             const float *__restrict__ scale,
                                                             const glint_u32x4 *__restrict__ x, float *__restrict__ y,
                                                             int N, int K, int G, int rows_per_wg) {
    extern __shared__ __attribute__((aligned(16))) float red[]; /* [rows][S][MR] */
    const int lane = threadIdx.x & 63;
    const int S = K >> 11;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int s = w % S, g = w / S;
    const int r0 = blockIdx.x * rows_per_wg;
    const int nrows = max(min(rows_per_wg, N - r0), 0);
    const int my = g < nrows ? (nrows - g + G - 1) / G : 0;
    const int64_t kv = K >> 4;                     /* 16-B vectors per weight row */
    /* this lane's two 16-B vectors in a row: 1 KiB contiguous per load instruction
     * (I8V_LINE), or two adjacent vectors */
    const int64_t v0 = I8V_LINE ? (int64_t)s * 128 + lane : (int64_t)(s * 64 + lane) * 2;
    const int64_t v1 = I8V_LINE ? v0 + 64 : v0 + 1;
    auto row_of = [&](int i) -> int64_t { return (int64_t)min(r0 + g + min(i, max(my - 1, 0)) * G, N - 1); };
    auto load = [&](int i, I8Row &r) {
        const int64_t n = row_of(i);
        r.q0 = __builtin_nontemporal_load(&q[n * kv + v0]);
        r.q1 = __builtin_nontemporal_load(&q[n * kv + v1]);
        r.s = scale[n * (K >> 6) + (v0 >> 2)];
        r.s1 = scale[n * (K >> 6) + (v1 >> 2)];
    };
    /* x: this lane's 32 activations of each of the MR rows: as BF16 pairs (I8V_DOT2) or f32 */
    uint32_t xw[MR][16];
    float xr[I8V_DOT2 ? 1 : MR][I8V_DOT2 ? 1 : 32];
#pragma unroll
    for (int mr = 0; mr < MR; ++mr)
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const glint_u32x4 v = x[(int64_t)mr * (K >> 3) + (h < 2 ? 2 * v0 + h : 2 * v1 + h - 2)];
            const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                xw[mr][4 * h + e] = d[e];
                if constexpr (!I8V_DOT2) {
                    xr[mr][8 * h + 2 * e] = glint_bf16lo(d[e]);
                    xr[mr][8 * h + 2 * e + 1] = glint_bf16hi(d[e]);
                }
            }
        }
    I8Row buf[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
        load(d, buf[d]);
    auto compute = [&](int i, const I8Row &r) {
        const uint32_t W[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        float part[MR];
#pragma unroll
        for (int mr = 0; mr < MR; ++mr)
            part[mr] = 0.0f;
        auto accumulate = [&](auto weights) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    float lo, hi;
                    weights(W[e], e >> 2, b, lo, hi);
                    const uint32_t pk = glint_cvt_bf16x2(lo, hi);
                    if constexpr (I8V_DOT2) {
                        /* both BF16 products are exact in f32; one instruction adds them */
#pragma unroll
                        for (int mr = 0; mr < MR; ++mr)
                            part[mr] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(i8v_bf16x2_t, pk),
                                                                       __builtin_bit_cast(i8v_bf16x2_t, xw[mr][2 * e + b]),
                                                                       part[mr], false);
                    } else {
                        const float wl = glint_bf16lo(pk), wh = glint_bf16hi(pk);
#pragma unroll
                        for (int mr = 0; mr < MR; ++mr) {
                            part[mr] = fmaf(wl, xr[mr][4 * e + 2 * b], part[mr]);
                            part[mr] = fmaf(wh, xr[mr][4 * e + 2 * b + 1], part[mr]);
                        }
                    }
                }
        };
        /* q s as fma(q + 128, s, -128 s): q + 128 is an unsigned byte (flip the sign bit,
         * then v_cvt_f32_ubyte) and -128 s is exact, so the one rounding gives the f32
         * product q s exactly as a multiply would. When -128 s is not finite (s infinite,
         * NaN or above 2^120) the lane multiplies instead. */
        const float sv[2] = {r.s, r.s1}, ns[2] = {-128.0f * r.s, -128.0f * r.s1};
        if (__builtin_isfinite(ns[0]) && __builtin_isfinite(ns[1])) {
            accumulate([&](uint32_t w, int hv, int b, float &lo, float &hi) {
                const uint32_t u = w ^ 0x80808080u;
                lo = fmaf((float)((u >> (16 * b)) & 0xFFu), sv[hv], ns[hv]);
                hi = fmaf((float)((u >> (16 * b + 8)) & 0xFFu), sv[hv], ns[hv]);
            });
        } else {
            accumulate([&](uint32_t w, int hv, int b, float &lo, float &hi) {
                lo = (float)(int8_t)(w >> (16 * b)) * sv[hv];
                hi = (float)(int8_t)(w >> (16 * b + 8)) * sv[hv];
            });
        }
#pragma unroll
        for (int mr = 0; mr < MR; ++mr) {
            float v = glint_row16_sum(part[mr]);
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            if (lane == 0)
                red[((g + i * G) * S + s) * MR + mr] = v;
        }
    };
    int i = 0;
    for (; i + DEPTH <= my; i += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            compute(i + d, buf[d]);
            load(i + d + DEPTH, buf[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d)
        if (i + d < my)
            compute(i + d, buf[d]);
    __syncthreads();
    for (int t = threadIdx.x; t < nrows * MR; t += blockDim.x) {
        const int row = t / MR, mr = t % MR;
        float sum = red[(row * S) * MR + mr];
        for (int k = 1; k < S; ++k)
            sum += red[(row * S + k) * MR + mr];
        y[(int64_t)mr * N + r0 + row] = sum;
    }
}

template <int MR>
static void i8tile_launch_gemv(const uint16_t *x, const Int8PinLinear &w, float *y, hipStream_t st) {
    const int S = w.k_in / 2048, G = (I8V_THREADS / 64) / S, threads = 64 * S * G;
    /* rows in flight (with the dot form and the 16-wave cap): m = 1 at k_in <= 4096 one
     * with the 1-KiB loads (14336 x 4096 12.5 against 13.5 us with two; with adjacent vectors
     * per lane two had been best, 13.6 against 14.0 for four); m = 2 one (14336 x 4096 15.4 against
     * 15.6, 4096 x 14336 16.4 against 16.9, 8192 x 8192 17.3 against 17.9); otherwise two
     * (one was 8-35% slower at m = 1, k_in > 4096 and at m = 4, three 1-7% slower) */
    auto kern = (MR == 1 && S <= 2) ? k_i8tile_gemv<MR, I8V_DEPTH_M1>
                                    : (MR == 2 ? k_i8tile_gemv<MR, I8V_DEPTH_M2> : k_i8tile_gemv<MR, I8V_DEPTH>);
    /* m = 1 with one row group per workgroup (G == 1: S = k_in / 2048 >= 5, k_in >= 10240):
     * half the resident grid (twice the rows per wave) measured 16.5 -> 15.4 us on
     * 4096 x 14336; at k_in = 4096 or m = 4 it was slower, and k_in = 6144 / 8192 (G = 2)
     * were not measured, so they keep the full grid */
    const int div = (MR == 1 && G == 1) ? I8V_GRID_DIV : 1;
    int64_t resident = glint_resident_grid((const void *)kern, threads, I8V_RED_MAX * 4);
    resident = std::min<int64_t>(resident, (int64_t)glint_cu_count() * std::max(I8V_WAVES_CU / (threads / 64), 1));
    resident = std::max<int64_t>(resident / div, 1);
    const int64_t per_wave = ((int64_t)w.n_out + G * resident - 1) / (G * resident);
    int64_t rows_per_wg = G * per_wave;
    const int64_t cap = (I8V_RED_MAX / (S * MR)) / G * G;
    if (rows_per_wg > cap)
        rows_per_wg = cap;
    const unsigned grid = (unsigned)((w.n_out + rows_per_wg - 1) / rows_per_wg);
    const size_t lds = (size_t)rows_per_wg * S * MR * sizeof(float);
    glint_set_lds_limit((const void *)kern, I8V_RED_MAX * 4);
    kern<<<grid, threads, lds, st>>>((const glint_u32x4 *)w.q, w.scale, (const glint_u32x4 *)x, y, w.n_out, w.k_in, G,
                                     (int)rows_per_wg);
}

template <int BM, int BN, int WM, int WN, int R>
static void i8tile_launch_fast(const uint16_t *x, const Int8PinLinear &w, float *y, int m, hipStream_t st) {
    const Int8PinTileProducer p{(const glint_u32x4 *)w.q, w.scale, w.n_out, w.k_in};
    for (int64_t r0 = 0; r0 < m; r0 += (int64_t)I8_MAX_YBLOCKS * BM) {
        const int mm = (int)std::min<int64_t>((int64_t)I8_MAX_YBLOCKS * BM, m - r0);
        tile_mfma_launch<BM, BN, WM, WN, R, Int8PinTileProducer, TileOutF32>(p, x + r0 * w.k_in, y + r0 * w.n_out, mm,
                                                                            w.n_out, w.k_in, st);
    }
}

/* The 256 x 256 prefill tile (x straight into LDS), where it has enough tiles */
static bool i8tile_launch_big(const uint16_t *x, const Int8PinLinear &w, float *y, int m, hipStream_t st) {
    if (!TILE_BIG || !tile_big_fits(std::min(m, I8_MAX_YBLOCKS * 256), w.n_out, w.k_in) ||
        !tile_big_pays(std::min(m, I8_MAX_YBLOCKS * 256), w.n_out))
        return false;
    const Int8PinTileProducer p{(const glint_u32x4 *)w.q, w.scale, w.n_out, w.k_in};
    for (int64_t r0 = 0; r0 < m; r0 += (int64_t)I8_MAX_YBLOCKS * 256) {
        const int mm = (int)std::min<int64_t>((int64_t)I8_MAX_YBLOCKS * 256, m - r0);
        if (tile_big_pays(mm, w.n_out))
            tile_big_launch<2, Int8PinTileProducer, TileOutF32>(p, x + r0 * w.k_in, y + r0 * w.n_out, mm, w.n_out,
                                                                w.k_in, st);
        else
            tile_mfma_launch<256, 128, 4, 2, 2, Int8PinTileProducer, TileOutF32>(p, x + r0 * w.k_in,
                                                                                y + r0 * w.n_out, mm, w.n_out,
                                                                                w.k_in, st);
    }
    return true;
}

template <int BM>
static void i8tile_launch_ss(const uint16_t *x, const Int8PinLinear &w, float *y, int m, hipStream_t st) {
    const Int8PinTileProducer p{(const glint_u32x4 *)w.q, w.scale, w.n_out, w.k_in};
    for (int64_t r0 = 0; r0 < m; r0 += (int64_t)I8_MAX_YBLOCKS * BM) {
        const int mm = (int)std::min<int64_t>((int64_t)I8_MAX_YBLOCKS * BM, m - r0);
        tile_ss_launch<BM, 64, 4, Int8PinTileProducer, TileOutF32>(p, x + r0 * w.k_in, y + r0 * w.n_out, mm, w.n_out,
                                                               w.k_in, st, BM == 64 ? I8_SS_PER_CU : 1);
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
    if (fast && m <= 4 && (w.k_in % 2048) == 0 && w.k_in / 2048 <= I8V_THREADS / 64) {
        if (m == 1)
            i8tile_launch_gemv<1>(x, w, y, stream);
        else if (m == 2)
            i8tile_launch_gemv<2>(x, w, y, stream);
        else if (m == 3)
            i8tile_launch_gemv<3>(x, w, y, stream);
        else
            i8tile_launch_gemv<4>(x, w, y, stream);
    } else if (fast) {
        if (m >= 256 && i8tile_launch_big(x, w, y, m, stream))
            ;
        else if (m >= 256)
            i8tile_launch_fast<256, 128, 4, 2, 2>(x, w, y, m, stream);
        else if (m > 64)
            i8tile_launch_ss<128>(x, w, y, m, stream);
        else
            i8tile_launch_ss<64>(x, w, y, m, stream);
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

GLINT_API int int8_tile_gemm_workspace_release(hipStream_t stream) { return glint_split_ws_release(stream); }
