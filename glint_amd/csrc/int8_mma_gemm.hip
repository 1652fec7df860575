/* INT8 GEMMs on gfx950 i8 MFMA (v_mfma_i32_16x16x64_i8: one 64-wide K slice per
 * instruction, exact int32 accumulation).
 *
 * int8_mma_gemm — the attach ABI (reference cuda/int8_mma_gemm.cu:11-155): activations
 *   quantized per (row, 64-block) (s = amax > 0 ? amax / 127 : 1, q = clamp(rint(x / s))),
 *   then per 64-slice kb: ic = exact int32 dot product, acc = fma(RN((float)ic * sx), sw,
 *   acc), kb ascending. That is the reference kernel's statement acc += ((float)ic * x0) * w0
 *   (cuda/int8_mma_gemm.cu:115-124) as its build compiles it: nvcc -O2 with the default
 *   --fmad=true (scripts/build_p7_kernels.sh:7) contracts the last multiply and add into one
 *   fused multiply-add. The reference's host emulation keeps them separate and its test
 *   allows for exactly that difference (1e-5, "only fp32 contraction order may differ",
 *   tests/test_int8_mma_gemm.cu:207).
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
 * the 64x64 tile = 2x2 MFMA tiles. Per 64-slice kb: ic = exact int32 dot product (one MFMA
 * with zero C), acc = fma((float)ic * sx, sw, acc). PLUG adds, per kb and right after the
 * base term, a p7_plug_res4_v1 slice read from its nibbles (element 2i in the low nibble,
 * value nibble - 8) with its own block scales: acc = fma((float)ip * sx, sp, acc). ACCUM
 * stores y + acc instead of acc (the second pass of the two-pass forms). */
template <bool PLUG, bool ACCUM>
__global__ __launch_bounds__(256) void k_int8_mma_gemm(const int8_t *__restrict__ xq, const float *__restrict__ sx,
                                                       const int8_t *__restrict__ wq, const float *__restrict__ sw,
                                                       float *__restrict__ y, int m, int n, int k_in,
                                                       const uint8_t *__restrict__ pq4, const float *__restrict__ psc) {
    /* two LDS buffers per operand: slice kb runs from buffer kb & 1 while slice kb + 1, loaded
     * into registers during slice kb's MFMAs, is written to the other; one barrier per slice */
    __shared__ __attribute__((aligned(16))) int8_t sA[2][Q_BM * Q_LDS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][Q_BN * Q_LDS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t sP[2][PLUG ? Q_BN * Q_LDS_ROW : 16];
    __shared__ float sSx[2][Q_BM], sSw[2][Q_BN], sSp[2][PLUG ? Q_BN : 1];
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
    /* staging: thread t copies 16 B of A row (t >> 2) and of B row (t >> 2), K bytes (t & 3) * 16;
     * the plug slice is 8 B of nibbles per thread, widened to the same 16 B; threads 0-63 load
     * the slice's sx, 64-127 its sw, 128-191 its plug scales */
    const int sr = tid >> 2, sc = (tid & 3) * 16;
    struct Stage {
        glint_u32x4 a, b;
        uint32_t nib[2];
        float s;
    };
    auto gload = [&](int kb, Stage &g) {
        g.a = glint_u32x4{0u, 0u, 0u, 0u};
        g.b = g.a;
        if (m0 + sr < m)
            g.a = *(const glint_u32x4 *)(xq + (int64_t)(m0 + sr) * k_in + (int64_t)kb * 64 + sc);
        if (n0 + sr < n)
            g.b = *(const glint_u32x4 *)(wq + (int64_t)(n0 + sr) * k_in + (int64_t)kb * 64 + sc);
        if (PLUG) {
            /* rows past n read as nibble 8 (value 0); k_in is even, so a row's nibbles start on a byte */
            g.nib[0] = g.nib[1] = 0x88888888u;
            if (n0 + sr < n) {
                const uint8_t *src = pq4 + (((int64_t)(n0 + sr) * k_in + (int64_t)kb * 64 + sc) >> 1);
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    g.nib[h] = (uint32_t)src[4 * h] | (uint32_t)src[4 * h + 1] << 8 | (uint32_t)src[4 * h + 2] << 16 |
                               (uint32_t)src[4 * h + 3] << 24;
            }
        }
        g.s = 0.0f;
        if (tid < Q_BM) {
            if (m0 + tid < m)
                g.s = sx[(int64_t)(m0 + tid) * nkb + kb];
        } else if (tid < Q_BM + Q_BN) {
            if (n0 + tid - Q_BM < n)
                g.s = sw[(int64_t)(n0 + tid - Q_BM) * nkb + kb];
        } else if (PLUG && tid < Q_BM + 2 * Q_BN) {
            if (n0 + tid - Q_BM - Q_BN < n)
                g.s = psc[(int64_t)(n0 + tid - Q_BM - Q_BN) * nkb + kb];
        }
    };
    auto lstore = [&](int buf, const Stage &g) {
        *(glint_u32x4 *)(sA[buf] + sr * Q_LDS_ROW + sc) = g.a;
        *(glint_u32x4 *)(sB[buf] + sr * Q_LDS_ROW + sc) = g.b;
        if (PLUG) {
            uint32_t out[4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                /* bytes 4h..4h+3 hold elements 8h..8h+7: low nibble first; value = nibble - 8 */
                const uint32_t lo = g.nib[h] & 0x0F0F0F0Fu, hi = (g.nib[h] >> 4) & 0x0F0F0F0Fu;
                const uint32_t e0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u); /* elements 0..3 */
                const uint32_t e1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u); /* elements 4..7 */
                /* per byte: nibble - 8 mod 256; setting bit 7 of every byte first keeps the
                 * subtraction's borrow inside the byte, the xor clears it again */
                out[2 * h] = ((e0 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
                out[2 * h + 1] = ((e1 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
            }
            *(glint_u32x4 *)(sP[buf] + sr * Q_LDS_ROW + sc) = glint_u32x4{out[0], out[1], out[2], out[3]};
        }
        if (tid < Q_BM)
            sSx[buf][tid] = g.s;
        else if (tid < Q_BM + Q_BN)
            sSw[buf][tid - Q_BM] = g.s;
        else if (PLUG && tid < Q_BM + 2 * Q_BN)
            sSp[buf][tid - Q_BM - Q_BN] = g.s;
    };
    Stage st;
    gload(0, st);
    lstore(0, st);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        const int cur = kb & 1;
        if (kb + 1 < nkb)
            gload(kb + 1, st);
        glint_i32x4 af[2], bf[2], pf[2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
            af[a] = *(const glint_i32x4 *)(sA[cur] + (wm * 32 + a * 16 + (lane & 15)) * Q_LDS_ROW + (lane >> 4) * 16);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            bf[b] = *(const glint_i32x4 *)(sB[cur] + (wn * 32 + b * 16 + (lane & 15)) * Q_LDS_ROW + (lane >> 4) * 16);
            if (PLUG)
                pf[b] = *(const glint_i32x4 *)(sP[cur] + (wn * 32 + b * 16 + (lane & 15)) * Q_LDS_ROW + (lane >> 4) * 16);
        }
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const glint_i32x4 ic = glint_mfma_i8(af[a], bf[b], glint_i32x4{0, 0, 0, 0});
                glint_i32x4 ip = glint_i32x4{0, 0, 0, 0};
                if (PLUG)
                    ip = glint_mfma_i8(af[a], pf[b], glint_i32x4{0, 0, 0, 0});
                const int col = wn * 32 + b * 16 + (lane & 15);
                const float swv = sSw[cur][col];
                const float spv = PLUG ? sSp[cur][col] : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float sxv = sSx[cur][wm * 32 + a * 16 + (lane >> 4) * 4 + i];
                    acc[a][b][i] = __builtin_fmaf((float)ic[i] * sxv, swv, acc[a][b][i]);
                    if (PLUG)
                        acc[a][b][i] = __builtin_fmaf((float)ip[i] * sxv, spv, acc[a][b][i]);
                }
            }
        if (kb + 1 < nkb)
            lstore(cur ^ 1, st);
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
                if (r < m && c < n) {
                    float *dst = y + (int64_t)r * n + c;
                    *dst = ACCUM ? *dst + acc[a][b][i] : acc[a][b][i];
                }
            }
}

/* p7_plug_res4_v1 slice to int8: element i = nibble i (low nibble first) - 8. */
__global__ __launch_bounds__(256) void k_unpack_res4(const uint8_t *__restrict__ q4, int8_t *__restrict__ out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = (int8_t)((int)((q4[i >> 1] >> ((i & 1) * 4)) & 15u) - 8);
}

/* Quantization residual of the activation, quantized again by the same rule: per (row,
 * 64-block), r = fma(-(float)xq, sx, x) (the reference's x - xq * sx under nvcc's
 * default contraction), s = amax|r| > 0 ?
 * amax / 127 : 1, rq = clamp(rint(r / s), -127, 127). One wave per block, one element per
 * lane. Reference cuda/int8_mma_gemm.cu:172-190. */
__global__ __launch_bounds__(256) void k_quant_act_resid(const uint16_t *__restrict__ x, const int8_t *__restrict__ xq,
                                                         const float *__restrict__ sx, int64_t nblocks,
                                                         int8_t *__restrict__ rq, float *__restrict__ sr) {
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * (blockDim.x / 64);
    for (int64_t b = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); b < nblocks; b += waves) {
        const int64_t i = b * 64 + lane;
        const float r = __builtin_fmaf(-(float)xq[i], sx[b], __uint_as_float((uint32_t)x[i] << 16));
        const float am = glint_wave_max(fabsf(r));
        const float s = (am > 0.0f) ? (am / 127.0f) : 1.0f;
        int v = (int)rintf(r / s);
        v = v > 127 ? 127 : (v < -127 ? -127 : v);
        rq[i] = (int8_t)v;
        if (lane == 0)
            sr[b] = s;
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

/* Large tiles: block 256 x 256 x 64 (K), 512 threads = 8 waves in 2 (M) x 4 (N), each wave a
 * 128 x 64 output block = 8 x 4 MFMA tiles (128 int32 accumulators per lane). Per K step a
 * wave reads 12 operand fragments from LDS for 32 MFMAs (the 64 x 64 wave tile above reads
 * 8 for 16), and the block reads each operand byte from L2 once per 256 outputs instead of
 * 128. Two LDS buffers per operand: step kb runs from buffer kb & 1 while the threads write
 * step kb + 1 into the other, then one barrier. Loads run three steps ahead: two register
 * sets alternate (even and odd steps), so a load issued at the end of step kb - 3 is
 * written to LDS at the end of step kb - 1, two steps of compute later (one step ahead
 * measured 13% slower, four steps ahead no faster). Rows past M or N are clamped into the
 * matrix (outputs not stored) and steps past the end reload the last one, so every load is
 * unconditional and the wait counter counts loads in flight. */
#define G2_BM 256
#define G2_BN 256
/* 64-byte LDS rows, 16-byte chunk c of row r stored at chunk c ^ f(r) with
 * f(r) = ((r >> 1) ^ ((r >> 3) & 1)) & 3. In a fragment read (16 consecutive rows from a
 * multiple of 16, one chunk) every group of 8 lanes, and every group of 16, then covers
 * distinct banks; a staging store (whole rows) does too. f does not change when r moves
 * by a multiple of 16. Against 80-byte padded rows: 40% fewer bank-conflict cycles, 3%
 * faster. */
#define G2_LDS_ROW 64
__device__ __forceinline__ int g2_lds_ofs(int r, int c) {
    return r * G2_LDS_ROW + ((c ^ (((r >> 1) ^ ((r >> 3) & 1)) & 3)) << 4);
}

template <bool SCALED>
__global__ __launch_bounds__(512) void k_int8_gemm_256(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                        const float *__restrict__ sa, const float *__restrict__ sb,
                                                        void *__restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) int8_t sA[2][G2_BM * G2_LDS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][G2_BN * G2_LDS_ROW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int m0 = blockIdx.y * G2_BM, n0 = blockIdx.x * G2_BN;
    const int nkb = K / 64;
    glint_i32x4 acc[8][4];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
            acc[a][b] = glint_i32x4{0, 0, 0, 0};
    const int sr = tid >> 2, sc = (tid & 3) * 16;
    const int64_t arow[2] = {(int64_t)min(m0 + sr, M - 1) * K + sc, (int64_t)min(m0 + sr + 128, M - 1) * K + sc};
    const int64_t brow[2] = {(int64_t)min(n0 + sr, N - 1) * K + sc, (int64_t)min(n0 + sr + 128, N - 1) * K + sc};
    struct Regs {
        glint_u32x4 a[2], b[2];
    };
    Regs r0, r1;
    auto gload = [&](int kb, Regs &r) {
        kb = min(kb, nkb - 1);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            r.a[h] = *(const glint_u32x4 *)(A + arow[h] + (int64_t)kb * 64);
            r.b[h] = *(const glint_u32x4 *)(B + brow[h] + (int64_t)kb * 64);
        }
    };
    /* the chunk this thread stages (t % 4) lands at g2_chunk(row, t % 4); rows sr and sr + 128
     * have the same swizzle */
    const int st_ofs = g2_lds_ofs(sr, tid & 3);
    auto lstore = [&](int buf, const Regs &r) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            *(glint_u32x4 *)(sA[buf] + 128 * h * G2_LDS_ROW + st_ofs) = r.a[h];
            *(glint_u32x4 *)(sB[buf] + 128 * h * G2_LDS_ROW + st_ofs) = r.b[h];
        }
    };
    /* fragment rows are (16-row tile base) + lane % 16, chunk lane / 16 */
    const int fr_ofs = g2_lds_ofs(lane & 15, lane >> 4);
    /* step kb: MFMAs from buffer kb & 1; step kb + 1's data (in `next`) goes to the other
     * buffer, then `next` is refilled with step kb + 3 */
    auto step = [&](int kb, Regs &next) {
        const int cur = kb & 1;
        glint_i32x4 af[8], bf[4];
#pragma unroll
        for (int a = 0; a < 8; ++a)
            af[a] = *(const glint_i32x4 *)(sA[cur] + (wm * 128 + a * 16) * G2_LDS_ROW + fr_ofs);
#pragma unroll
        for (int b = 0; b < 4; ++b)
            bf[b] = *(const glint_i32x4 *)(sB[cur] + (wn * 64 + b * 16) * G2_LDS_ROW + fr_ofs);
#pragma unroll
        for (int a = 0; a < 8; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                acc[a][b] = glint_mfma_i8(af[a], bf[b], acc[a][b]);
        lstore(cur ^ 1, next);
        gload(kb + 3, next);
        __syncthreads();
    };
    gload(0, r0);
    lstore(0, r0);
    gload(1, r1);
    gload(2, r0);
    __syncthreads();
    int kb = 0;
    for (; kb + 2 <= nkb; kb += 2) {
        step(kb, r1);     /* writes step kb + 1 (odd, in r1), loads kb + 3 into r1 */
        step(kb + 1, r0); /* writes step kb + 2 (even, in r0), loads kb + 4 into r0 */
    }
    if (kb < nkb)
        step(kb, r1);
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = m0 + wm * 128 + a * 16 + (lane >> 4) * 4 + i;
                const int c = n0 + wn * 64 + b * 16 + (lane & 15);
                if (r < M && c < N) {
                    if (SCALED)
                        ((uint16_t *)C)[(int64_t)r * N + c] = glint_f32_to_bf16(((float)acc[a][b][i] * sa[r]) * sb[c]);
                    else
                        ((int32_t *)C)[(int64_t)r * N + c] = acc[a][b][i];
                }
            }
}

/* The same 256 x 256 tile and wave layout with both operands going HBM -> LDS directly
 * (buffer loads with the lds bit), through a ring of G3_NBUF K-step buffers: the loads of
 * step kb + G3_NBUF - 1 go out at the start of step kb, into the buffer step kb - 1 used.
 * No staging registers and no LDS store instructions; each DMA instruction writes 1 KB of
 * consecutive LDS (16 rows, every lane the 16-B chunk the row swizzle puts in its slot).
 * Per step a wave waits for its own loads of the step (s_waitcnt), then the barrier makes
 * every wave's visible. Byte offsets are 32-bit: M * K and N * K < 2^31 (the host checks).
 * The four A and four B buffers are separate arrays, so the compiler sees that a DMA into
 * one does not alias fragment reads of another. */
#define G3_NBUF 4
#ifndef G3_PREFETCH
#define G3_PREFETCH 1
#endif
#ifndef G3_THREADS
#define G3_THREADS 512
#endif
template <bool SCALED>
__global__ __launch_bounds__(G3_THREADS) void k_int8_gemm_dma(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                        const float *__restrict__ sa, const float *__restrict__ sb,
                                                        void *__restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) int8_t sA0[G2_BM * G2_LDS_ROW], sA1[G2_BM * G2_LDS_ROW],
        sA2[G2_BM * G2_LDS_ROW], sA3[G2_BM * G2_LDS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t sB0[G2_BN * G2_LDS_ROW], sB1[G2_BN * G2_LDS_ROW],
        sB2[G2_BN * G2_LDS_ROW], sB3[G2_BN * G2_LDS_ROW];
    auto bufA = [&](int i) { return i == 0 ? sA0 : (i == 1 ? sA1 : (i == 2 ? sA2 : sA3)); };
    auto bufB = [&](int i) { return i == 0 ? sB0 : (i == 1 ? sB1 : (i == 2 ? sB2 : sB3)); };
    /* NW waves in 2 (M) x NW / 2 (N); wave tile 128 x TN * 16; each wave loads RPW rows of
     * each operand per step in QN instructions */
    constexpr int T = G3_THREADS;
    constexpr int NW = T / 64, WNW = NW / 2, TM = 8, TN = 16 / WNW, RPW = 256 / NW, QN = RPW / 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WNW, wn = wave % WNW;
    const int m0 = blockIdx.y * G2_BM, n0 = blockIdx.x * G2_BN;
    const int nkb = K / 64;
    glint_i32x4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
            acc[a][b] = glint_i32x4{0, 0, 0, 0};
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void *)A, (short)0, (int)((uint32_t)M * (uint32_t)K), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void *)B, (short)0, (int)((uint32_t)N * (uint32_t)K), GLINT_BUF_DWORD3);
    /* wave w, instruction q: rows RPW w + 16 q .. +15 of both tiles; lane l takes row
     * RPW w + 16 q + l / 4, LDS slot l % 4, i.e. logical chunk (l % 4) ^ f(row) */
    uint32_t avo[QN], bvo[QN];
#pragma unroll
    for (int q = 0; q < QN; ++q) {
        const int r = RPW * wave + 16 * q + (lane >> 2);
        const int c = (lane & 3) ^ (((r >> 1) ^ ((r >> 3) & 1)) & 3);
        avo[q] = (uint32_t)min(m0 + r, M - 1) * (uint32_t)K + (uint32_t)c * 16u;
        bvo[q] = (uint32_t)min(n0 + r, N - 1) * (uint32_t)K + (uint32_t)c * 16u;
    }
    /* step kb's 2 QN loads per wave into ring slot buf; steps past the end reload the last */
    auto dma = [&](int kb, int buf) {
        const uint32_t so = (uint32_t)min(kb, nkb - 1) * 64u;
#pragma unroll
        for (int q = 0; q < QN; ++q) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void *)(bufA(buf) + (RPW * wave + 16 * q) * G2_LDS_ROW), 16,
                avo[q], so, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void *)(bufB(buf) + (RPW * wave + 16 * q) * G2_LDS_ROW), 16,
                bvo[q], so, 0, 0);
        }
    };
    const int fr_ofs = g2_lds_ofs(lane & 15, lane >> 4);
#if G3_PREFETCH
    /* Fragments one step ahead: step kb multiplies fragments read during step kb - 1 while
     * it reads step kb + 1's, so no LDS read latency sits between MFMAs. Two register sets
     * alternate with the step's parity. */
    struct Frags {
        glint_i32x4 a[TM], b[TN];
    };
    Frags fr[2];
    auto read_frags = [&](int u, Frags &f) {
        const int8_t *ta = bufA(u), *tb = bufB(u);
#pragma unroll
        for (int b = 0; b < TN; ++b)
            f.b[b] = *(const glint_i32x4 *)(tb + (wn * TN * 16 + b * 16) * G2_LDS_ROW + fr_ofs);
#pragma unroll
        for (int a = 0; a < TM; ++a)
            f.a[a] = *(const glint_i32x4 *)(ta + (wm * 128 + a * 16) * G2_LDS_ROW + fr_ofs);
    };
    auto step = [&](int kb, int u) {
        /* this wave's loads of step kb + 1 are done once only step kb + 2's 2 QN remain, and
         * its fragment reads of step kb are done; after the barrier every wave's are, and
         * slot (u + 3) % 4, last read during step kb - 2, is free */
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT_LGKM0(2 * QN * (G3_NBUF - 3)));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "global");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "global");
        dma(kb + G3_NBUF - 1, (u + G3_NBUF - 1) % G3_NBUF);
        __builtin_amdgcn_sched_barrier(0); /* issue the loads first, not after the MFMAs */
        Frags &f = fr[u & 1];
        read_frags((u + 1) % G3_NBUF, fr[(u + 1) & 1]); /* past the end: clamped data nobody uses */
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b)
                acc[a][b] = glint_mfma_i8(f.a[a], f.b[b], acc[a][b]);
        /* the next step's reads spread over the first MFMAs, one read per two MFMAs */
#pragma unroll
        for (int i = 0; i < TM + TN; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); /* LDS read */
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0); /* MFMA */
        }
    };
#pragma unroll
    for (int i = 0; i < G3_NBUF - 1; ++i)
        dma(i, i);
    /* step 0's loads (only steps 1 and 2's remain), then its fragments */
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT_LGKM0(2 * QN * (G3_NBUF - 2)));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "global");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "global");
    read_frags(0, fr[0]);
#else
    /* step kb from ring slot u = kb % G3_NBUF (a constant after unrolling) */
    auto step = [&](int kb, int u) {
        /* this wave's loads of step kb are done once only the later steps' 2 QN each remain,
         * and its fragment reads of step kb - 1 are done (their slot is refilled next) */
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT_LGKM0(2 * QN * (G3_NBUF - 2)));
        /* A barrier with fences that order global memory only. __syncthreads() orders LDS as
         * well, and the compiler then waits for every LDS DMA in flight (vmcnt(0)) at each
         * step, which empties the ring. The fences still keep the compiler from moving memory
         * accesses across the barrier; the explicit wait above gives the LDS ordering. */
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "global");
        __builtin_amdgcn_s_barrier(); /* every wave's loads of step kb landed; slot (u + 3) % 4 is free */
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "global");
        dma(kb + G3_NBUF - 1, (u + G3_NBUF - 1) % G3_NBUF);
        __builtin_amdgcn_sched_barrier(0); /* issue the loads first, not after the MFMAs */
        const int8_t *ta = bufA(u), *tb = bufB(u);
        glint_i32x4 bf[TN];
#pragma unroll
        for (int b = 0; b < TN; ++b)
            bf[b] = *(const glint_i32x4 *)(tb + (wn * TN * 16 + b * 16) * G2_LDS_ROW + fr_ofs);
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const glint_i32x4 af = *(const glint_i32x4 *)(ta + (wm * 128 + a * 16) * G2_LDS_ROW + fr_ofs);
#pragma unroll
            for (int b = 0; b < TN; ++b)
                acc[a][b] = glint_mfma_i8(af, bf[b], acc[a][b]);
        }
    };
#pragma unroll
    for (int i = 0; i < G3_NBUF - 1; ++i)
        dma(i, i);
#endif
    int kb = 0;
    for (; kb + G3_NBUF <= nkb; kb += G3_NBUF) {
#pragma unroll
        for (int u = 0; u < G3_NBUF; ++u)
            step(kb + u, u);
    }
#pragma unroll
    for (int u = 0; u + 1 < G3_NBUF; ++u)
        if (kb + u < nkb)
            step(kb + u, u);
    /* the ring's last loads (reloads past the end) must land before the workgroup's LDS is
     * released */
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0);
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = m0 + wm * 128 + a * 16 + (lane >> 4) * 4 + i;
                const int c = n0 + wn * TN * 16 + b * 16 + (lane & 15);
                if (r < M && c < N) {
                    if (SCALED)
                        ((uint16_t *)C)[(int64_t)r * N + c] = glint_f32_to_bf16(((float)acc[a][b][i] * sa[r]) * sb[c]);
                    else
                        ((int32_t *)C)[(int64_t)r * N + c] = acc[a][b][i];
                }
            }
}

/* k_int8_gemm_dma with a 5-slot ring and one barrier per two K steps. A per-step timeline
 * of k_int8_gemm_dma (s_memtime stamps in a timing copy) showed each SIMD's older wave done
 * issuing its step in about 780 clocks and the younger in about 1320, the older then
 * waiting at the barrier: per step the MFMA pipe idles through the wait and the barrier
 * (about 250 clocks) besides the 1024 clocks of MFMAs. Here an even step kb waits for its
 * own loads of steps up to kb + 2, passes the barrier, and loads steps kb + 4 and kb + 5
 * into the slots of steps kb - 1 and kb (whose fragments every wave has read); an odd step
 * only multiplies and reads the next step's fragments, which the even step's barrier
 * already made visible. Loads still run two steps ahead of the wait that needs them. The
 * 5 slots are the whole 160 KiB of LDS. */
template <bool SCALED>
__global__ __launch_bounds__(512) void k_int8_gemm_dma5(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                        const float *__restrict__ sa, const float *__restrict__ sb,
                                                        void *__restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) int8_t sA0[G2_BM * G2_LDS_ROW], sA1[G2_BM * G2_LDS_ROW],
        sA2[G2_BM * G2_LDS_ROW], sA3[G2_BM * G2_LDS_ROW], sA4[G2_BM * G2_LDS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t sB0[G2_BN * G2_LDS_ROW], sB1[G2_BN * G2_LDS_ROW],
        sB2[G2_BN * G2_LDS_ROW], sB3[G2_BN * G2_LDS_ROW], sB4[G2_BN * G2_LDS_ROW];
    auto bufA = [&](int i) { return i == 0 ? sA0 : (i == 1 ? sA1 : (i == 2 ? sA2 : (i == 3 ? sA3 : sA4))); };
    auto bufB = [&](int i) { return i == 0 ? sB0 : (i == 1 ? sB1 : (i == 2 ? sB2 : (i == 3 ? sB3 : sB4))); };
    constexpr int NW = 8, WNW = 4, TM = 8, TN = 4, RPW = 32, QN = 2, NS = 5;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WNW, wn = wave % WNW;
    const int m0 = blockIdx.y * G2_BM, n0 = blockIdx.x * G2_BN;
    const int nkb = K / 64;
    glint_i32x4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
            acc[a][b] = glint_i32x4{0, 0, 0, 0};
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void *)A, (short)0, (int)((uint32_t)M * (uint32_t)K), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void *)B, (short)0, (int)((uint32_t)N * (uint32_t)K), GLINT_BUF_DWORD3);
    uint32_t avo[QN], bvo[QN];
#pragma unroll
    for (int q = 0; q < QN; ++q) {
        const int r = RPW * wave + 16 * q + (lane >> 2);
        const int c = (lane & 3) ^ (((r >> 1) ^ ((r >> 3) & 1)) & 3);
        avo[q] = (uint32_t)min(m0 + r, M - 1) * (uint32_t)K + (uint32_t)c * 16u;
        bvo[q] = (uint32_t)min(n0 + r, N - 1) * (uint32_t)K + (uint32_t)c * 16u;
    }
    auto dma = [&](int kb, int buf) {
        const uint32_t so = (uint32_t)min(kb, nkb - 1) * 64u;
#pragma unroll
        for (int q = 0; q < QN; ++q) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void *)(bufA(buf) + (RPW * wave + 16 * q) * G2_LDS_ROW), 16,
                avo[q], so, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void *)(bufB(buf) + (RPW * wave + 16 * q) * G2_LDS_ROW), 16,
                bvo[q], so, 0, 0);
        }
    };
    const int fr_ofs = g2_lds_ofs(lane & 15, lane >> 4);
    struct Frags {
        glint_i32x4 a[TM], b[TN];
    };
    Frags fr[2];
    auto read_frags = [&](int u, Frags &f) {
        const int8_t *ta = bufA(u), *tb = bufB(u);
#pragma unroll
        for (int b = 0; b < TN; ++b)
            f.b[b] = *(const glint_i32x4 *)(tb + (wn * TN * 16 + b * 16) * G2_LDS_ROW + fr_ofs);
#pragma unroll
        for (int a = 0; a < TM; ++a)
            f.a[a] = *(const glint_i32x4 *)(ta + (wm * 128 + a * 16) * G2_LDS_ROW + fr_ofs);
    };
    /* step kb in slot u = kb % NS, fragments in set p = kb % 2 (constants after unrolling) */
    auto step = [&](int kb, int u, int p) {
        if (p == 0) {
            __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT_LGKM0(2 * QN)); /* only step kb + 3's remain */
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "global");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "global");
            dma(kb + 4, (u + 4) % NS);
            dma(kb + 5, u);
            __builtin_amdgcn_sched_barrier(0);
        }
        Frags &f = fr[p];
        read_frags((u + 1) % NS, fr[p ^ 1]); /* past the end: clamped data nobody uses */
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b)
                acc[a][b] = glint_mfma_i8(f.a[a], f.b[b], acc[a][b]);
#pragma unroll
        for (int i = 0; i < TM + TN; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); /* LDS read */
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0); /* MFMA */
        }
    };
#pragma unroll
    for (int i = 0; i < 4; ++i)
        dma(i, i);
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT_LGKM0(2 * QN * 2)); /* steps 0 and 1 landed */
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "global");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "global");
    read_frags(0, fr[0]);
    int kb = 0;
    for (; kb + 2 * NS <= nkb; kb += 2 * NS) {
#pragma unroll
        for (int i = 0; i < 2 * NS; ++i)
            step(kb + i, i % NS, i & 1);
    }
#pragma unroll
    for (int i = 0; i + 1 < 2 * NS; ++i)
        if (kb + i < nkb)
            step(kb + i, i % NS, i & 1);
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0); /* the ring's last (clamped) loads land first */
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = m0 + wm * 128 + a * 16 + (lane >> 4) * 4 + i;
                const int c = n0 + wn * TN * 16 + b * 16 + (lane & 15);
                if (r < M && c < N) {
                    if (SCALED)
                        ((uint16_t *)C)[(int64_t)r * N + c] = glint_f32_to_bf16(((float)acc[a][b][i] * sa[r]) * sb[c]);
                    else
                        ((int32_t *)C)[(int64_t)r * N + c] = acc[a][b][i];
                }
            }
}

/* The attach ABI's W8A8 GEMM on the same 256 x 256 DMA ring (int8_mma_gemm at the shapes
 * with at least 3/4 as many 256 x 256 tiles as CUs). Per 64-slice kb the wave's 32 MFMAs
 * run with zero C (ic = the slice's exact int32 dot products), and each A tile's 4 results
 * go straight into the f32 accumulators as acc = fma((float)ic * sx[m, kb], sw[n, kb], acc)
 * (kb ascending: bit-identical to the 64 x 64 kernel). A third ring carries the slice's
 * scales: 256 sx (rows of the tile) and 256 sw (columns), one 4-byte DMA per wave per step
 * (waves 0-3 rows, 4-7 columns). That epilogue is 3 VALU ops per output per slice (convert,
 * multiply, fused multiply-add) against one MFMA per 16 x 16 x 64, so the kernel is
 * VALU-bound: at 2048 x 8192 x 8192 about 164 us of VALU issue on 256 CUs.
 * ACCUM stores y + acc (the second pass of the two-pass forms). Offsets are 32-bit:
 * M K, N K, M K / 16 and N K / 16 < 2^31 (the host checks). */
template <bool ACCUM>
__global__ __launch_bounds__(512) void k_int8_mma_dma(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                      const float *__restrict__ sx, const float *__restrict__ sw,
                                                      float *__restrict__ y, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) int8_t sA0[G2_BM * G2_LDS_ROW], sA1[G2_BM * G2_LDS_ROW],
        sA2[G2_BM * G2_LDS_ROW], sA3[G2_BM * G2_LDS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t sB0[G2_BN * G2_LDS_ROW], sB1[G2_BN * G2_LDS_ROW],
        sB2[G2_BN * G2_LDS_ROW], sB3[G2_BN * G2_LDS_ROW];
    /* scales of a slice: [0, 256) sx of the tile's rows, [256, 512) sw of its columns */
    __shared__ __attribute__((aligned(16))) float sS0[512], sS1[512], sS2[512], sS3[512];
    auto bufA = [&](int i) { return i == 0 ? sA0 : (i == 1 ? sA1 : (i == 2 ? sA2 : sA3)); };
    auto bufB = [&](int i) { return i == 0 ? sB0 : (i == 1 ? sB1 : (i == 2 ? sB2 : sB3)); };
    auto bufS = [&](int i) { return i == 0 ? sS0 : (i == 1 ? sS1 : (i == 2 ? sS2 : sS3)); };
    constexpr int NW = 8, WNW = 4, TM = 8, TN = 4, RPW = 32, QN = 2;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WNW, wn = wave % WNW;
    const int m0 = blockIdx.y * G2_BM, n0 = blockIdx.x * G2_BN;
    const int nkb = K / 64;
    float acc[TM][TN][4];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[a][b][i] = 0.0f;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void *)A, (short)0, (int)((uint32_t)M * (uint32_t)K), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void *)B, (short)0, (int)((uint32_t)N * (uint32_t)K), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rs = wave < 4
        ? __builtin_amdgcn_make_buffer_rsrc((void *)sx, (short)0, (int)((uint32_t)M * (uint32_t)nkb * 4u), GLINT_BUF_DWORD3)
        : __builtin_amdgcn_make_buffer_rsrc((void *)sw, (short)0, (int)((uint32_t)N * (uint32_t)nkb * 4u), GLINT_BUF_DWORD3);
    uint32_t avo[QN], bvo[QN];
#pragma unroll
    for (int q = 0; q < QN; ++q) {
        const int r = RPW * wave + 16 * q + (lane >> 2);
        const int c = (lane & 3) ^ (((r >> 1) ^ ((r >> 3) & 1)) & 3);
        avo[q] = (uint32_t)min(m0 + r, M - 1) * (uint32_t)K + (uint32_t)c * 16u;
        bvo[q] = (uint32_t)min(n0 + r, N - 1) * (uint32_t)K + (uint32_t)c * 16u;
    }
    /* scale lane: wave w < 4 row m0 + 64 w + l, else column n0 + 64 (w - 4) + l (clamped) */
    const uint32_t svo = (wave < 4 ? (uint32_t)min(m0 + 64 * wave + lane, M - 1)
                                   : (uint32_t)min(n0 + 64 * (wave - 4) + lane, N - 1)) *
                         (uint32_t)nkb * 4u;
    auto dma = [&](int kb, int buf) {
        const uint32_t kc = (uint32_t)min(kb, nkb - 1);
#pragma unroll
        for (int q = 0; q < QN; ++q) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void *)(bufA(buf) + (RPW * wave + 16 * q) * G2_LDS_ROW), 16,
                avo[q], kc * 64u, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void *)(bufB(buf) + (RPW * wave + 16 * q) * G2_LDS_ROW), 16,
                bvo[q], kc * 64u, 0, 0);
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(bufS(buf) + 64 * wave),
                                                 4, svo, kc * 4u, 0, 0);
    };
    const int fr_ofs = g2_lds_ofs(lane & 15, lane >> 4);
    auto step = [&](int kb, int u) {
        /* own loads of step kb landed (later steps' 2 QN + 1 each remain), own reads of step
         * kb - 1 done; then the barrier with global-only fences (see k_int8_gemm_dma) */
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT_LGKM0((2 * QN + 1) * (G3_NBUF - 2)));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "global");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "global");
        dma(kb + G3_NBUF - 1, (u + G3_NBUF - 1) % G3_NBUF);
        __builtin_amdgcn_sched_barrier(0);
        const int8_t *ta = bufA(u), *tb = bufB(u);
        const float *ts = bufS(u);
        glint_i32x4 bf[TN];
        float swv[TN];
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            bf[b] = *(const glint_i32x4 *)(tb + (wn * TN * 16 + b * 16) * G2_LDS_ROW + fr_ofs);
            swv[b] = ts[256 + wn * TN * 16 + b * 16 + (lane & 15)];
        }
        /* A tile a's MFMAs go out before tile a - 2's epilogue, which then runs while they
         * complete instead of waiting for its own results (2048 x 8192 x 8192: 334 -> 320 us
         * one tile behind, 311 us two behind; three or four behind 385-392 us) */
        constexpr int PD = 2;
        glint_i32x4 ic[PD + 1][TN];
        glint_f32x4 sxv[PD + 1];
        auto epi = [&](int a, const glint_i32x4 (&c)[TN], const glint_f32x4 &sv) {
#pragma unroll
            for (int b = 0; b < TN; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[a][b][i] = __builtin_fmaf((float)c[b][i] * sv[i], swv[b], acc[a][b][i]);
        };
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const glint_i32x4 af = *(const glint_i32x4 *)(ta + (wm * 128 + a * 16) * G2_LDS_ROW + fr_ofs);
            sxv[a % (PD + 1)] = *(const glint_f32x4 *)(ts + wm * 128 + a * 16 + (lane >> 4) * 4);
#pragma unroll
            for (int b = 0; b < TN; ++b)
                ic[a % (PD + 1)][b] = glint_mfma_i8(af, bf[b], glint_i32x4{0, 0, 0, 0});
            if (a >= PD)
                epi(a - PD, ic[(a - PD) % (PD + 1)], sxv[(a - PD) % (PD + 1)]);
        }
#pragma unroll
        for (int a = TM - PD; a < TM; ++a)
            epi(a, ic[a % (PD + 1)], sxv[a % (PD + 1)]);
    };
#pragma unroll
    for (int i = 0; i < G3_NBUF - 1; ++i)
        dma(i, i);
    int kb = 0;
    for (; kb + G3_NBUF <= nkb; kb += G3_NBUF) {
#pragma unroll
        for (int u = 0; u < G3_NBUF; ++u)
            step(kb + u, u);
    }
#pragma unroll
    for (int u = 0; u + 1 < G3_NBUF; ++u)
        if (kb + u < nkb)
            step(kb + u, u);
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0); /* the ring's last (clamped) loads land first */
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = m0 + wm * 128 + a * 16 + (lane >> 4) * 4 + i;
                const int c = n0 + wn * TN * 16 + b * 16 + (lane & 15);
                if (r < M && c < N) {
                    float *dst = y + (int64_t)r * N + c;
                    *dst = ACCUM ? *dst + acc[a][b][i] : acc[a][b][i];
                }
            }
}

/* The attach ABI's W8A8 GEMM for the shapes with few 256 x 256 tiles (small m: a decode or
 * short prefill): 64 x 64 tiles, 4 waves in 2 x 2 (32 x 32 each), operands and scales
 * through a ring of Q_NBUF slice buffers filled by LDS DMA, loads Q_NBUF - 1 slices ahead.
 * The slices of an output must be added in order, so a tile walks all of K; with few
 * tiles per CU the time per slice is the load latency, and the deep ring spreads it over
 * Q_NBUF - 1 slices. Each wave issues 3 loads per slice (16 rows of A, 16 of B, 64 scales:
 * wave 0 the tile's sx, wave 1 its sw, waves 2-3 copies of both into spare slots, so every
 * wave's wait count is the same). Epilogue as k_int8_mma_dma. */
#ifndef Q_NBUF
#define Q_NBUF 8
#endif
#ifndef Q_NARROW
#define Q_NARROW 1
#endif
#ifndef Q_RING8
#define Q_RING8 1 /* the narrow tiles on 8 waves (k_int8_mma_ring8) */
#endif
#ifndef Q_RING8_WIDE
#define Q_RING8_WIDE 0 /* the 64 x 64 tiles on 8 waves too (slower: 128 x 14336 x 4096 49.5 -> 62.5 us,
                        * 256 x 4096 x 4096 24.2 -> 27.7) */
#endif
#ifndef Q_PER_STEP
#define Q_PER_STEP 2 /* K slices per barrier (1 or 2) */
#endif
template <bool ACCUM, int NB>
__global__ __launch_bounds__(256) void k_int8_mma_ring(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                       const float *__restrict__ sx, const float *__restrict__ sw,
                                                       float *__restrict__ y, int M, int N, int K) {
    /* one array per ring slot: the compiler then sees that a DMA into one slot does not
     * alias fragment reads of another (with one array it waits for every DMA in flight,
     * vmcnt(0), before each step's reads, which empties the ring) */
    static_assert(Q_NBUF == 8, "ring slots are declared one by one");
#define Q_SLOT(i) __shared__ __attribute__((aligned(16))) int8_t sA##i[Q_BM * G2_LDS_ROW], sB##i[Q_BN * G2_LDS_ROW]; \
    __shared__ __attribute__((aligned(16))) float sS##i[256]; /* [0, 64) sx, [64, 128) sw */
    Q_SLOT(0) Q_SLOT(1) Q_SLOT(2) Q_SLOT(3) Q_SLOT(4) Q_SLOT(5) Q_SLOT(6) Q_SLOT(7)
#undef Q_SLOT
    auto slotA = [&](int i) -> int8_t * {
        switch (i) { case 0: return sA0; case 1: return sA1; case 2: return sA2; case 3: return sA3;
                     case 4: return sA4; case 5: return sA5; case 6: return sA6; default: return sA7; }
    };
    auto slotB = [&](int i) -> int8_t * {
        switch (i) { case 0: return sB0; case 1: return sB1; case 2: return sB2; case 3: return sB3;
                     case 4: return sB4; case 5: return sB5; case 6: return sB6; default: return sB7; }
    };
    auto slotS = [&](int i) -> float * {
        switch (i) { case 0: return sS0; case 1: return sS1; case 2: return sS2; case 3: return sS3;
                     case 4: return sS4; case 5: return sS5; case 6: return sS6; default: return sS7; }
    };
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * Q_BM, n0 = blockIdx.x * (32 * NB); /* NB 16-column blocks per wave */
    const int nkb = K / 64;
    float acc[2][NB][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[a][b][i] = 0.0f;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void *)A, (short)0, (int)((uint32_t)M * (uint32_t)K), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void *)B, (short)0, (int)((uint32_t)N * (uint32_t)K), GLINT_BUF_DWORD3);
    const bool rows = (wave & 1) == 0; /* waves 0, 2: sx; 1, 3: sw */
    const __amdgpu_buffer_rsrc_t rs = rows
        ? __builtin_amdgcn_make_buffer_rsrc((void *)sx, (short)0, (int)((uint32_t)M * (uint32_t)nkb * 4u), GLINT_BUF_DWORD3)
        : __builtin_amdgcn_make_buffer_rsrc((void *)sw, (short)0, (int)((uint32_t)N * (uint32_t)nkb * 4u), GLINT_BUF_DWORD3);
    /* wave w: rows 16 w .. +15 of both tiles; lane l takes row 16 w + l / 4, LDS slot l % 4 */
    const int r = 16 * wave + (lane >> 2);
    const int c = (lane & 3) ^ (((r >> 1) ^ ((r >> 3) & 1)) & 3);
    const uint32_t avo = (uint32_t)min(m0 + r, M - 1) * (uint32_t)K + (uint32_t)c * 16u;
    const uint32_t bvo = (uint32_t)min(n0 + r, N - 1) * (uint32_t)K + (uint32_t)c * 16u;
    const uint32_t svo = (rows ? (uint32_t)min(m0 + lane, M - 1) : (uint32_t)min(n0 + lane, N - 1)) * (uint32_t)nkb * 4u;
    auto dma = [&](int kb, int buf) {
        const uint32_t kc = (uint32_t)min(kb, nkb - 1);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            ra, (__attribute__((address_space(3))) void *)(slotA(buf) + 16 * wave * G2_LDS_ROW), 16, avo, kc * 64u, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rb, (__attribute__((address_space(3))) void *)(slotB(buf) + 16 * wave * G2_LDS_ROW), 16, bvo, kc * 64u, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(slotS(buf) + 64 * wave),
                                                 4, svo, kc * 4u, 0, 0);
    };
    const int fr_ofs = g2_lds_ofs(lane & 15, lane >> 4);
    auto slice = [&](int u) {
        const int8_t *ta = slotA(u), *tb = slotB(u);
        const float *ts = slotS(u);
        glint_i32x4 af[2], bf[NB];
        float swv[NB];
#pragma unroll
        for (int a = 0; a < 2; ++a)
            af[a] = *(const glint_i32x4 *)(ta + (wm * 32 + a * 16) * G2_LDS_ROW + fr_ofs);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            bf[b] = *(const glint_i32x4 *)(tb + (wn * 16 * NB + b * 16) * G2_LDS_ROW + fr_ofs);
            swv[b] = ts[64 + wn * 16 * NB + b * 16 + (lane & 15)];
        }
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            const glint_f32x4 sxv = *(const glint_f32x4 *)(ts + wm * 32 + a * 16 + (lane >> 4) * 4);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const glint_i32x4 ic = glint_mfma_i8(af[a], bf[b], glint_i32x4{0, 0, 0, 0});
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[a][b][i] = __builtin_fmaf((float)ic[i] * sxv[i], swv[b], acc[a][b][i]);
            }
        }
    };
    /* Q_PER_STEP slices per barrier; Q_NBUF - Q_PER_STEP slices in flight ahead */
    constexpr int PS = Q_PER_STEP, AHEAD = Q_NBUF - PS;
    auto step = [&](int kb, int u) {
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT_LGKM0(3 * (AHEAD - PS)));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "global");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "global");
#pragma unroll
        for (int v = 0; v < PS; ++v)
            dma(kb + AHEAD + v, (u + AHEAD + v) % Q_NBUF);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int v = 0; v < PS; ++v)
            if (v == 0 || kb + v < nkb) /* the last step of an odd count has one slice */
                slice((u + v) % Q_NBUF);
    };
#pragma unroll
    for (int i = 0; i < AHEAD; ++i)
        dma(i, i);
    int kb = 0;
    for (; kb + Q_NBUF <= nkb; kb += Q_NBUF) {
#pragma unroll
        for (int u = 0; u < Q_NBUF; u += PS)
            step(kb + u, u);
    }
#pragma unroll
    for (int u = 0; u < Q_NBUF; u += PS)
        if (kb + u < nkb)
            step(kb + u, u);
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0); /* the ring's last (clamped) loads land first */
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rr = m0 + wm * 32 + a * 16 + (lane >> 4) * 4 + i;
                const int cc = n0 + wn * 16 * NB + b * 16 + (lane & 15);
                if (rr < M && cc < N) {
                    float *dst = y + (int64_t)rr * N + cc;
                    *dst = ACCUM ? *dst + acc[a][b][i] : acc[a][b][i];
                }
            }
}

#ifndef G3_DMA
#define G3_DMA 1
#endif
#ifndef G3_RING5
#define G3_RING5 1 /* the plain GEMM on k_int8_gemm_dma5 (5-slot ring, a barrier every two steps) */
#endif
static inline bool g3_fits(int M, int N, int K) {
    return G3_DMA && (int64_t)M * K < ((int64_t)1 << 31) && (int64_t)N * K < ((int64_t)1 << 31);
}
#ifndef G2_MIN_FILL
#define G2_MIN_FILL 1
#endif
/* The 256 x 256 tiles need at least 3/4 as many tiles as CUs; with fewer, the 128 x 128
 * kernel's 4x more tiles fill the device better (512 x 8192 x 8192: 64 tiles of 256 x 256
 * on 256 CUs). */
static inline bool g2_pays(int M, int N) {
    if (M < G2_BM || N < G2_BN)
        return false;
    return !G2_MIN_FILL ||
           (int64_t)((M + G2_BM - 1) / G2_BM) * ((N + G2_BN - 1) / G2_BN) * 4 >= (int64_t)3 * glint_cu_count();
}

/* ------------------------------------------------------------------ C ABI */
static bool q_args_ok(const void *x, const void *y, const void *xq, const void *sx, const Int8MmaLinear &w, int m) {
    return x && y && xq && sx && w.q && w.scale && m >= 1 && w.n_out >= 1 && w.k_in >= 64 && (w.k_in % 64) == 0 &&
           glint_aligned(x, 16) && glint_aligned(xq, 16) && glint_aligned(w.q, 16);
}

static void q_launch_quant(const void *x, int m, int k_in, int8_t *xq, float *sx, hipStream_t st) {
    const int64_t nchunk8 = (int64_t)m * k_in / 8;
    int64_t grid = (nchunk8 + 255) / 256;
    if (grid > 4096)
        grid = 4096;
    k_quant_act<<<(unsigned)grid, 256, 0, st>>>((const glint_u32x4 *)x, nchunk8, (glint_u32x2 *)xq, sx);
}

/* k_int8_mma_ring over 8 waves, two per SIMD: 64 x 32 NB tiles, wave w computes rows
 * 16 (w / 2) .. +15 and NB 16-column blocks from column 16 NB (w % 2). Every wave issues the
 * same number of DMAs per slice, so the wait counts are uniform: NB = 1 one (waves 0-3 16
 * rows of A each, waves 4-5 16 rows of B, wave 6 the tile's 64 sx, wave 7 64 sw of which 32
 * are used: only the W rows the tile uses are staged); NB = 2 two (waves 0-3 16 rows of A,
 * waves 4-7 16 rows of B, wave 0 sx, wave 1 sw and the others copies of them into spare
 * slots). Against the 4-wave form (32 x 16 NB per wave): M 70 N 4096 K 3072 (NB = 1) 17.4 ->
 * 15.0 us for the whole call (quantization included), bit-identical; at NB = 2 it was slower
 * (Q_RING8_WIDE). Epilogue as k_int8_mma_dma. */
template <bool ACCUM, int NB>
__global__ __launch_bounds__(512) void k_int8_mma_ring8(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                        const float *__restrict__ sx, const float *__restrict__ sw,
                                                        float *__restrict__ y, int M, int N, int K) {
    static_assert(Q_NBUF == 8, "ring slots are declared one by one");
    static_assert(NB == 1 || NB == 2, "16-column blocks per wave");
    constexpr int BR = 32 * NB;         /* W rows of a tile */
    constexpr int ND = NB;              /* DMAs per wave per slice */
    constexpr int SW = NB == 1 ? 128 : 512; /* scale floats per slot: sx, sw (and the copies) */
#define Q_SLOT(i) __shared__ __attribute__((aligned(16))) int8_t sA##i[64 * G2_LDS_ROW], sB##i[BR * G2_LDS_ROW]; \
    __shared__ __attribute__((aligned(16))) float sS##i[SW];
    Q_SLOT(0) Q_SLOT(1) Q_SLOT(2) Q_SLOT(3) Q_SLOT(4) Q_SLOT(5) Q_SLOT(6) Q_SLOT(7)
#undef Q_SLOT
    auto slotA = [&](int i) -> int8_t * {
        switch (i) { case 0: return sA0; case 1: return sA1; case 2: return sA2; case 3: return sA3;
                     case 4: return sA4; case 5: return sA5; case 6: return sA6; default: return sA7; }
    };
    auto slotB = [&](int i) -> int8_t * {
        switch (i) { case 0: return sB0; case 1: return sB1; case 2: return sB2; case 3: return sB3;
                     case 4: return sB4; case 5: return sB5; case 6: return sB6; default: return sB7; }
    };
    auto slotS = [&](int i) -> float * {
        switch (i) { case 0: return sS0; case 1: return sS1; case 2: return sS2; case 3: return sS3;
                     case 4: return sS4; case 5: return sS5; case 6: return sS6; default: return sS7; }
    };
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * BR;
    const int nkb = K / 64;
    float acc[NB][4];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            acc[b][i] = 0.0f;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void *)A, (short)0, (int)((uint32_t)M * (uint32_t)K), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void *)B, (short)0, (int)((uint32_t)N * (uint32_t)K), GLINT_BUF_DWORD3);
    /* operand rows: waves 0-3 A rows 16 w, waves 4 .. 4 + BR / 16 - 1 B rows 16 (w - 4) */
    const bool opA = wave < 4, opB = !opA && wave < 4 + BR / 16;
    const int r = (opA ? 16 * wave : 16 * (wave - 4)) + (lane >> 2);
    const int c = (lane & 3) ^ (((r >> 1) ^ ((r >> 3) & 1)) & 3);
    const uint32_t ovo = opA ? (uint32_t)min(m0 + r, M - 1) * (uint32_t)K + (uint32_t)c * 16u
                             : (uint32_t)min(n0 + r, N - 1) * (uint32_t)K + (uint32_t)c * 16u;
    /* scales: NB = 1 waves 6 (sx) and 7 (sw); NB = 2 even waves sx, odd waves sw, wave w
     * into 64-float region w (regions 0 and 1 are the ones read) */
    const bool srow = NB == 1 ? wave == 6 : (wave & 1) == 0;
    const __amdgpu_buffer_rsrc_t rs = srow
        ? __builtin_amdgcn_make_buffer_rsrc((void *)sx, (short)0, (int)((uint32_t)M * (uint32_t)nkb * 4u), GLINT_BUF_DWORD3)
        : __builtin_amdgcn_make_buffer_rsrc((void *)sw, (short)0, (int)((uint32_t)N * (uint32_t)nkb * 4u), GLINT_BUF_DWORD3);
    const uint32_t svo = (srow ? (uint32_t)min(m0 + lane, M - 1) : (uint32_t)min(n0 + lane, N - 1)) * (uint32_t)nkb * 4u;
    const int sreg = NB == 1 ? 64 * (wave - 6) : 64 * wave;
    auto dma = [&](int kb, int buf) {
        const uint32_t kc = (uint32_t)min(kb, nkb - 1);
        if (opA)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void *)(slotA(buf) + 16 * wave * G2_LDS_ROW), 16, ovo, kc * 64u, 0, 0);
        else if (opB)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void *)(slotB(buf) + 16 * (wave - 4) * G2_LDS_ROW), 16, ovo, kc * 64u,
                0, 0);
        if (NB == 2 || (!opA && !opB))
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(slotS(buf) + sreg), 4, svo,
                                                     kc * 4u, 0, 0);
    };
    const int fr_ofs = g2_lds_ofs(lane & 15, lane >> 4);
    auto slice = [&](int u) {
        const int8_t *ta = slotA(u), *tb = slotB(u);
        const float *ts = slotS(u);
        const glint_i32x4 af = *(const glint_i32x4 *)(ta + (wm * 16) * G2_LDS_ROW + fr_ofs);
        const glint_f32x4 sxv = *(const glint_f32x4 *)(ts + wm * 16 + (lane >> 4) * 4);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const glint_i32x4 bf = *(const glint_i32x4 *)(tb + (wn * 16 * NB + b * 16) * G2_LDS_ROW + fr_ofs);
            const float swv = ts[64 + wn * 16 * NB + b * 16 + (lane & 15)];
            const glint_i32x4 ic = glint_mfma_i8(af, bf, glint_i32x4{0, 0, 0, 0});
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[b][i] = __builtin_fmaf((float)ic[i] * sxv[i], swv, acc[b][i]);
        }
    };
    constexpr int PS = Q_PER_STEP, AHEAD = Q_NBUF - PS;
    auto step = [&](int kb, int u) {
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT_LGKM0(ND * (AHEAD - PS)));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "global");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "global");
#pragma unroll
        for (int v = 0; v < PS; ++v)
            dma(kb + AHEAD + v, (u + AHEAD + v) % Q_NBUF);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int v = 0; v < PS; ++v)
            if (v == 0 || kb + v < nkb)
                slice((u + v) % Q_NBUF);
    };
#pragma unroll
    for (int i = 0; i < AHEAD; ++i)
        dma(i, i);
    int kb = 0;
    for (; kb + Q_NBUF <= nkb; kb += Q_NBUF) {
#pragma unroll
        for (int u = 0; u < Q_NBUF; u += PS)
            step(kb + u, u);
    }
#pragma unroll
    for (int u = 0; u < Q_NBUF; u += PS)
        if (kb + u < nkb)
            step(kb + u, u);
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rr = m0 + wm * 16 + (lane >> 4) * 4 + i;
            const int cc = n0 + wn * 16 * NB + b * 16 + (lane & 15);
            if (rr < M && cc < N) {
                float *dst = y + (int64_t)rr * N + cc;
                *dst = ACCUM ? *dst + acc[b][i] : acc[b][i];
            }
        }
}

/* The W8A8 product: the 256 x 256 DMA-ring kernel where there are enough tiles, else the
 * 64 x 64 DMA-ring kernel (both need their 32-bit offsets to fit); the fused plug (and an
 * operand past 2 GiB) takes the 64 x 64 register-staged kernel. */
template <bool PLUG, bool ACCUM>
static void q_launch_gemm(const int8_t *xq, const float *sx, const int8_t *wq, const float *sw, float *y, int m,
                          int n, int k_in, const uint8_t *pq4, const float *psc, hipStream_t st) {
    if (!PLUG && g2_pays(m, n) && g3_fits(m, n, k_in)) {
        k_int8_mma_dma<ACCUM><<<dim3((n + G2_BN - 1) / G2_BN, (m + G2_BM - 1) / G2_BM), 512, 0, st>>>(
            xq, wq, sx, sw, y, m, n, k_in);
        return;
    }
    if (!PLUG && g3_fits(m, n, k_in)) {
        /* 64 x 32 output tiles (each wave one 16-column block; the loader still stages 64 W
         * rows, half of them unused) where 64 x 64 tiles would leave CUs idle */
        const int64_t tiles64 = (int64_t)((n + Q_BN - 1) / Q_BN) * ((m + Q_BM - 1) / Q_BM);
        const bool narrow = Q_NARROW && tiles64 < glint_cu_count();
        if (narrow && Q_RING8)
            k_int8_mma_ring8<ACCUM, 1><<<dim3((n + 31) / 32, (m + Q_BM - 1) / Q_BM), 512, 0, st>>>(xq, wq, sx, sw, y, m,
                                                                                                  n, k_in);
        else if (narrow)
            k_int8_mma_ring<ACCUM, 1><<<dim3((n + 31) / 32, (m + Q_BM - 1) / Q_BM), 256, 0, st>>>(xq, wq, sx, sw, y, m,
                                                                                                  n, k_in);
        else if (Q_RING8_WIDE)
            k_int8_mma_ring8<ACCUM, 2><<<dim3((n + Q_BN - 1) / Q_BN, (m + Q_BM - 1) / Q_BM), 512, 0, st>>>(xq, wq, sx, sw,
                                                                                                          y, m, n, k_in);
        else
            k_int8_mma_ring<ACCUM, 2><<<dim3((n + Q_BN - 1) / Q_BN, (m + Q_BM - 1) / Q_BM), 256, 0, st>>>(xq, wq, sx, sw,
                                                                                                          y, m, n, k_in);
        return;
    }
    dim3 g((n + Q_BN - 1) / Q_BN, (m + Q_BM - 1) / Q_BM);
    k_int8_mma_gemm<PLUG, ACCUM><<<g, 256, 0, st>>>(xq, sx, wq, sw, y, m, n, k_in, pq4, psc);
}

static void q_launch_unpack(const uint8_t *q4, int8_t *out, int64_t n, hipStream_t st) {
    int64_t grid = (n + 255) / 256;
    if (grid > 8192)
        grid = 8192;
    k_unpack_res4<<<(unsigned)grid, 256, 0, st>>>(q4, out, n);
}

GLINT_API int int8_mma_gemm(const void *x, Int8MmaLinear w, float *y, int m, int8_t *xq, float *sx,
                            struct ihipStream_t *stream) {
    if (!q_args_ok(x, y, xq, sx, w, m))
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    q_launch_quant(x, m, w.k_in, xq, sx, st);
    q_launch_gemm<false, false>(xq, sx, w.q, w.scale, y, m, w.n_out, w.k_in, nullptr, nullptr, st);
    return (int)hipGetLastError();
}

GLINT_API int int8_mma_gemm_plug(const void *x, Int8MmaLinear w, const uint8_t *plug_q4, const float *plug_scale,
                                 float *y, int m, int8_t *xq, float *sx, int8_t *plug_i8,
                                 struct ihipStream_t *stream) {
    if (!q_args_ok(x, y, xq, sx, w, m) || !plug_q4 || !plug_scale || !plug_i8 || !glint_aligned(plug_i8, 16))
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    q_launch_quant(x, m, w.k_in, xq, sx, st);
    q_launch_gemm<false, false>(xq, sx, w.q, w.scale, y, m, w.n_out, w.k_in, nullptr, nullptr, st);
    q_launch_unpack(plug_q4, plug_i8, (int64_t)w.n_out * w.k_in, st);
    q_launch_gemm<false, true>(xq, sx, plug_i8, plug_scale, y, m, w.n_out, w.k_in, nullptr, nullptr, st);
    return (int)hipGetLastError();
}

GLINT_API int int8_mma_gemm_plug_fused(const void *x, Int8MmaLinear w, const uint8_t *plug_q4,
                                       const float *plug_scale, float *y, int m, int8_t *xq, float *sx,
                                       struct ihipStream_t *stream) {
    if (!q_args_ok(x, y, xq, sx, w, m) || !plug_q4 || !plug_scale)
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    q_launch_quant(x, m, w.k_in, xq, sx, st);
    q_launch_gemm<true, false>(xq, sx, w.q, w.scale, y, m, w.n_out, w.k_in, plug_q4, plug_scale, st);
    return (int)hipGetLastError();
}

GLINT_API int int8_mma_gemm_resolve(const void *x, Int8MmaLinear w, const uint8_t *plug_q4, const float *plug_scale,
                                    float *y, int m, int8_t *xq, float *sx, int8_t *rq, float *sr, int8_t *plug_i8,
                                    struct ihipStream_t *stream) {
    const bool plug = plug_q4 != nullptr;
    if (!q_args_ok(x, y, xq, sx, w, m) || !rq || !sr || !glint_aligned(rq, 16) || plug != (plug_i8 != nullptr) ||
        plug != (plug_scale != nullptr) || (plug && !glint_aligned(plug_i8, 16)))
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const int64_t nblocks = (int64_t)m * (w.k_in / 64);
    q_launch_quant(x, m, w.k_in, xq, sx, st);
    int64_t grid = (nblocks + 3) / 4;
    if (grid > 8192)
        grid = 8192;
    k_quant_act_resid<<<(unsigned)grid, 256, 0, st>>>((const uint16_t *)x, xq, sx, nblocks, rq, sr);
    q_launch_gemm<false, false>(xq, sx, w.q, w.scale, y, m, w.n_out, w.k_in, nullptr, nullptr, st);
    q_launch_gemm<false, true>(rq, sr, w.q, w.scale, y, m, w.n_out, w.k_in, nullptr, nullptr, st);
    if (plug) {
        q_launch_unpack(plug_q4, plug_i8, (int64_t)w.n_out * w.k_in, st);
        q_launch_gemm<false, true>(xq, sx, plug_i8, plug_scale, y, m, w.n_out, w.k_in, nullptr, nullptr, st);
        q_launch_gemm<false, true>(rq, sr, plug_i8, plug_scale, y, m, w.n_out, w.k_in, nullptr, nullptr, st);
    }
    return (int)hipGetLastError();
}

GLINT_API int glint_int8_gemm_i32(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K,
                                  struct ihipStream_t *stream) {
    if (!A || !B || !C || M < 1 || N < 1 || K < 64 || (K % 64) != 0 || !glint_aligned(A, 16) || !glint_aligned(B, 16))
        return (int)hipErrorInvalidValue;
    const bool big = g2_pays(M, N);
    if (big && g3_fits(M, N, K) && G3_RING5)
        k_int8_gemm_dma5<false><<<dim3((N + G2_BN - 1) / G2_BN, (M + G2_BM - 1) / G2_BM), 512, 0, (hipStream_t)stream>>>(
            A, B, nullptr, nullptr, C, M, N, K);
    else if (big && g3_fits(M, N, K))
        k_int8_gemm_dma<false><<<dim3((N + G2_BN - 1) / G2_BN, (M + G2_BM - 1) / G2_BM), G3_THREADS, 0,
                                             (hipStream_t)stream>>>(
            A, B, nullptr, nullptr, C, M, N, K);
    else if (big)
        k_int8_gemm_256<false><<<dim3((N + G2_BN - 1) / G2_BN, (M + G2_BM - 1) / G2_BM), 512, 0, (hipStream_t)stream>>>(
            A, B, nullptr, nullptr, C, M, N, K);
    else
        k_int8_gemm<false><<<dim3((N + G_BN - 1) / G_BN, (M + G_BM - 1) / G_BM), 256, 0, (hipStream_t)stream>>>(
            A, B, nullptr, nullptr, C, M, N, K);
    return (int)hipGetLastError();
}

GLINT_API int glint_int8_gemm_scaled_bf16(const int8_t *A, const int8_t *B, const float *sa, const float *sb,
                                          uint16_t *out, int M, int N, int K, struct ihipStream_t *stream) {
    if (!A || !B || !sa || !sb || !out || M < 1 || N < 1 || K < 64 || (K % 64) != 0 || !glint_aligned(A, 16) ||
        !glint_aligned(B, 16))
        return (int)hipErrorInvalidValue;
    const bool big = g2_pays(M, N);
    if (big && g3_fits(M, N, K) && G3_RING5)
        k_int8_gemm_dma5<true><<<dim3((N + G2_BN - 1) / G2_BN, (M + G2_BM - 1) / G2_BM), 512, 0, (hipStream_t)stream>>>(
            A, B, sa, sb, out, M, N, K);
    else if (big && g3_fits(M, N, K))
        k_int8_gemm_dma<true><<<dim3((N + G2_BN - 1) / G2_BN, (M + G2_BM - 1) / G2_BM), G3_THREADS, 0,
                                            (hipStream_t)stream>>>(
            A, B, sa, sb, out, M, N, K);
    else if (big)
        k_int8_gemm_256<true><<<dim3((N + G2_BN - 1) / G2_BN, (M + G2_BM - 1) / G2_BM), 512, 0, (hipStream_t)stream>>>(
            A, B, sa, sb, out, M, N, K);
    else
        k_int8_gemm<true><<<dim3((N + G_BN - 1) / G_BN, (M + G_BM - 1) / G_BM), 256, 0, (hipStream_t)stream>>>(
            A, B, sa, sb, out, M, N, K);
    return (int)hipGetLastError();
}
