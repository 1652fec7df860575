/* INT8 GEMMs on gfx950 i8 MFMA (v_mfma_i32_16x16x64_i8: one 64-wide K slice per
 * instruction, exact int32 accumulation).
 *
 * int8_mma_gemm — the attach ABI (reference cuda/int8_mma_gemm.cu:11-155): activations
 *   quantized per (row, 64-block) (s = amax > 0 ? amax / 127 : 1, q = clamp(rint(x / s))),
 *   then per 64-slice kb: ic = exact int32 dot product, acc += ((float)ic * sx) * sw,
 *   kb ascending, as separate f32 multiplies and add (bit-identical to the CPU emulation).
 * glint_int8_gemm_i32 / _scaled_bf16 — the plain INT8 GEMM C = A B^T with int32
 *   accumulation over all of K (|C| <= K * 127^2 < 2^31 for K < 133152), optionally
 *   scaled to BF16 RNE(((float)C * sa[m]) * sb[n]).
 *
 * MFMA operand layout (16x16x64 i8): lane l holds row (l % 16), K bytes
 * [(l / 16) * 16, +16) of A (and the same for B's row = output column); the 4 int32
 * results of lane l are D[(l / 16) * 4 + i][l % 16], i = 0..3.
 */
#include "glint_common.h"
#include "int8_mma_gemm.h"

typedef int glint_i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ glint_i32x4 glint_mfma_i8(glint_i32x4 a, glint_i32x4 b, glint_i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

/* ------------------------------------------------------------ activation quantization */
typedef unsigned short glint_u16x2 __attribute__((ext_vector_type(2)));
typedef short glint_i16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ glint_i16x2 q_mag_key(uint32_t d) {
    const glint_u16x2 m = __builtin_bit_cast(glint_u16x2, d & 0x7FFF7FFFu) + (glint_u16x2)(0x7F);
    return __builtin_bit_cast(glint_i16x2, m);
}

/* One lane per 8 values, 8 lanes per 64-block; blocks are the flat array's 64-element
 * groups (k_in % 64 == 0, so a block never crosses a row). The block max ignores NaN
 * like the reference's fmaxf reduction (an all-NaN block gives amax 0 here and NaN
 * there; both give s = 1). */
__global__ __launch_bounds__(256) void k_quant_act(const glint_u32x4 *__restrict__ x, int64_t nchunk8,
                                                   glint_u32x2 *__restrict__ xq, float *__restrict__ sx) {
    /* nchunk8 and the stride are multiples of 8, so the 8 lanes of a block always run the
     * same iterations and the DPP max sees the whole block */
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < nchunk8; t += stride) {
        const glint_u32x4 d = x[t];
        glint_i16x2 k = __builtin_elementwise_max(q_mag_key(d.x), q_mag_key(d.y));
        k = __builtin_elementwise_max(k, __builtin_elementwise_max(q_mag_key(d.z), q_mag_key(d.w)));
        /* floor at key 0x7F (magnitude 0) so an all-NaN lane contributes 0 */
        const int m16 = glint_max8(max(max((int)k.x, (int)k.y), 0x7F) - 0x7F);
        const float am = __uint_as_float((uint32_t)m16 << 16);
        const float s = (am > 0.0f) ? (am / 127.0f) : 1.0f;
        const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
        uint32_t packed[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float w = (j & 1) ? glint_bf16hi(dw[j >> 1]) : glint_bf16lo(dw[j >> 1]);
            /* float -> int as the reference's CUDA cast: NaN -> 0, saturating */
            int v = (int)rintf(w / s);
            v = v > 127 ? 127 : (v < -127 ? -127 : v);
            packed[j >> 2] |= ((uint32_t)v & 0xFFu) << (8 * (j & 3));
        }
        xq[t] = glint_u32x2{packed[0], packed[1]};
        if ((threadIdx.x & 7) == 0)
            sx[t >> 3] = s;
    }
}

/* ------------------------------------------------------------ W8A8 (attach ABI) */
#define Q_BM 64
#define Q_BN 64
#define Q_LDS_ROW 80 /* 64 bytes + 16 of padding: 8 consecutive rows hit 8 disjoint bank quads */

/* 256 threads = 4 waves in 2x2; wave (wm, wn) owns rows [32 wm, +32) x cols [32 wn, +32) of
 * the 64x64 tile = 2x2 MFMA tiles. */
__global__ __launch_bounds__(256) void k_int8_mma_gemm(const int8_t *__restrict__ xq, const float *__restrict__ sx,
                                                       const int8_t *__restrict__ wq, const float *__restrict__ sw,
                                                       float *__restrict__ y, int m, int n, int k_in) {
    __shared__ __attribute__((aligned(16))) int8_t sA[Q_BM * Q_LDS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t sB[Q_BN * Q_LDS_ROW];
    __shared__ float sSx[Q_BM], sSw[Q_BN];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * Q_BM, n0 = blockIdx.x * Q_BN;
    const int nkb = k_in / 64;
    float acc[2][2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[a][b][i] = 0.0f;
    /* staging: thread t copies 16 B of A row (t >> 2) and of B row (t >> 2), K bytes (t & 3) * 16 */
    const int sr = tid >> 2, sc = (tid & 3) * 16;
    for (int kb = 0; kb < nkb; ++kb) {
        glint_u32x4 va = glint_u32x4{0u, 0u, 0u, 0u}, vb = va;
        if (m0 + sr < m)
            va = *(const glint_u32x4 *)(xq + (int64_t)(m0 + sr) * k_in + (int64_t)kb * 64 + sc);
        if (n0 + sr < n)
            vb = *(const glint_u32x4 *)(wq + (int64_t)(n0 + sr) * k_in + (int64_t)kb * 64 + sc);
        *(glint_u32x4 *)(sA + sr * Q_LDS_ROW + sc) = va;
        *(glint_u32x4 *)(sB + sr * Q_LDS_ROW + sc) = vb;
        if (tid < Q_BM)
            sSx[tid] = (m0 + tid < m) ? sx[(int64_t)(m0 + tid) * nkb + kb] : 0.0f;
        else if (tid < Q_BM + Q_BN)
            sSw[tid - Q_BM] = (n0 + tid - Q_BM < n) ? sw[(int64_t)(n0 + tid - Q_BM) * nkb + kb] : 0.0f;
        __syncthreads();
        glint_i32x4 af[2], bf[2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
            af[a] = *(const glint_i32x4 *)(sA + (wm * 32 + a * 16 + (lane & 15)) * Q_LDS_ROW + (lane >> 4) * 16);
#pragma unroll
        for (int b = 0; b < 2; ++b)
            bf[b] = *(const glint_i32x4 *)(sB + (wn * 32 + b * 16 + (lane & 15)) * Q_LDS_ROW + (lane >> 4) * 16);
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const glint_i32x4 ic = glint_mfma_i8(af[a], bf[b], glint_i32x4{0, 0, 0, 0});
                const float swv = sSw[wn * 32 + b * 16 + (lane & 15)];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float sxv = sSx[wm * 32 + a * 16 + (lane >> 4) * 4 + i];
                    const float t = (float)ic[i] * sxv;
                    acc[a][b][i] = acc[a][b][i] + t * swv;
                }
            }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = m0 + wm * 32 + a * 16 + (lane >> 4) * 4 + i;
                const int c = n0 + wn * 32 + b * 16 + (lane & 15);
                if (r < m && c < n)
                    y[(int64_t)r * n + c] = acc[a][b][i];
            }
}

/* ------------------------------------------------------------ plain INT8 GEMM */
#define G_BM 128
#define G_BN 128
#define G_LDS_ROW 80

/* 256 threads = 4 waves in 2x2, each wave a 64x64 output block = 4x4 MFMA tiles; int32
 * accumulation over all of K; A and B tiles double-buffered in LDS. */
template <bool SCALED>
__global__ __launch_bounds__(256) void k_int8_gemm(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                   const float *__restrict__ sa, const float *__restrict__ sb,
                                                   void *__restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) int8_t sA[2][G_BM * G_LDS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][G_BN * G_LDS_ROW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * G_BM, n0 = blockIdx.x * G_BN;
    const int nkb = K / 64;
    glint_i32x4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
            acc[a][b] = glint_i32x4{0, 0, 0, 0};
    /* staging: 128 rows x 64 B per operand = 512 x 16 B; thread t copies rows (t >> 2) and
     * (t >> 2) + 64, K bytes (t & 3) * 16 */
    const int sr = tid >> 2, sc = (tid & 3) * 16;
    glint_u32x4 ra[2], rb[2];
    auto gload = [&](int kb) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = sr + 64 * h;
            ra[h] = (m0 + r < M) ? *(const glint_u32x4 *)(A + (int64_t)(m0 + r) * K + (int64_t)kb * 64 + sc)
                                 : glint_u32x4{0u, 0u, 0u, 0u};
            rb[h] = (n0 + r < N) ? *(const glint_u32x4 *)(B + (int64_t)(n0 + r) * K + (int64_t)kb * 64 + sc)
                                 : glint_u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            *(glint_u32x4 *)(sA[buf] + (sr + 64 * h) * G_LDS_ROW + sc) = ra[h];
            *(glint_u32x4 *)(sB[buf] + (sr + 64 * h) * G_LDS_ROW + sc) = rb[h];
        }
    };
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        const int cur = kb & 1;
        if (kb + 1 < nkb)
            gload(kb + 1);
        glint_i32x4 af[4], bf[4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
            af[a] = *(const glint_i32x4 *)(sA[cur] + (wm * 64 + a * 16 + (lane & 15)) * G_LDS_ROW + (lane >> 4) * 16);
#pragma unroll
        for (int b = 0; b < 4; ++b)
            bf[b] = *(const glint_i32x4 *)(sB[cur] + (wn * 64 + b * 16 + (lane & 15)) * G_LDS_ROW + (lane >> 4) * 16);
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                acc[a][b] = glint_mfma_i8(af[a], bf[b], acc[a][b]);
        if (kb + 1 < nkb)
            lstore(cur ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = m0 + wm * 64 + a * 16 + (lane >> 4) * 4 + i;
                const int c = n0 + wn * 64 + b * 16 + (lane & 15);
                if (r < M && c < N) {
                    if (SCALED)
                        ((uint16_t *)C)[(int64_t)r * N + c] = glint_f32_to_bf16(((float)acc[a][b][i] * sa[r]) * sb[c]);
                    else
                        ((int32_t *)C)[(int64_t)r * N + c] = acc[a][b][i];
                }
            }
}

/* ------------------------------------------------------------------ C ABI */
GLINT_API int int8_mma_gemm(const void *x, Int8MmaLinear w, float *y, int m, int8_t *xq, float *sx,
                            struct ihipStream_t *stream) {
    if (!x || !y || !xq || !sx || !w.q || !w.scale || m < 1 || w.n_out < 1 || w.k_in < 64 || (w.k_in % 64) != 0)
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    if (!glint_aligned(x, 16) || !glint_aligned(xq, 16) || !glint_aligned(w.q, 16))
        return (int)hipErrorInvalidValue;
    const int64_t nchunk8 = (int64_t)m * w.k_in / 8;
    int64_t grid = (nchunk8 + 255) / 256;
    if (grid > 4096)
        grid = 4096;
    k_quant_act<<<(unsigned)grid, 256, 0, st>>>((const glint_u32x4 *)x, nchunk8, (glint_u32x2 *)xq, sx);
    dim3 g2((w.n_out + Q_BN - 1) / Q_BN, (m + Q_BM - 1) / Q_BM);
    k_int8_mma_gemm<<<g2, 256, 0, st>>>(xq, sx, w.q, w.scale, y, m, w.n_out, w.k_in);
    return (int)hipGetLastError();
}

GLINT_API int glint_int8_gemm_i32(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K,
                                  struct ihipStream_t *stream) {
    if (!A || !B || !C || M < 1 || N < 1 || K < 64 || (K % 64) != 0 || !glint_aligned(A, 16) || !glint_aligned(B, 16))
        return (int)hipErrorInvalidValue;
    dim3 g((N + G_BN - 1) / G_BN, (M + G_BM - 1) / G_BM);
    k_int8_gemm<false><<<g, 256, 0, (hipStream_t)stream>>>(A, B, nullptr, nullptr, C, M, N, K);
    return (int)hipGetLastError();
}

GLINT_API int glint_int8_gemm_scaled_bf16(const int8_t *A, const int8_t *B, const float *sa, const float *sb,
                                          uint16_t *out, int M, int N, int K, struct ihipStream_t *stream) {
    if (!A || !B || !sa || !sb || !out || M < 1 || N < 1 || K < 64 || (K % 64) != 0 || !glint_aligned(A, 16) ||
        !glint_aligned(B, 16))
        return (int)hipErrorInvalidValue;
    dim3 g((N + G_BN - 1) / G_BN, (M + G_BM - 1) / G_BM);
    k_int8_gemm<true><<<g, 256, 0, (hipStream_t)stream>>>(A, B, sa, sb, out, M, N, K);
    return (int)hipGetLastError();
}
