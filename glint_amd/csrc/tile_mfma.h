/* Double-buffered BF16 MFMA tile GEMM whose weight operand is dequantized into LDS
 * (gfx950). Shared by the GLINT prefill GEMM and the INT8-pin W8A16 GEMM.
 *
 * y[M, N] = x[M, K] W^T, x BF16 [M, K] row-major with 16-B aligned rows and K % 64 == 0.
 * W is made 16 weights at a time by a Producer, which owns the weight format:
 *   struct Regs;                                  registers of one thread's step
 *   load(Regs &, int row, int quarter, int kb)    global loads of W[row, 64 kb + 16 quarter, +16),
 *                                                 row < N and kb < K / 64 (the kernel clamps)
 *   produce(const Regs &, uint32_t (&)[8], lane)  the 16 weights as BF16 pairs (lo = even k)
 *   LDS_WORDS, setup(float *lds)                  LDS the producer needs (filled before step 0)
 *
 * Block tile BM x BN x 64 (K) over WM x WN waves; each wave owns a (BM / WM) x (BN / WN)
 * tile of v_mfma_f32_16x16x32_bf16 accumulators (f32). Thread t produces W row t / 4,
 * K quarter t % 4 (so BN * 4 == threads), and stages BM * 8 / threads 16-B chunks of x.
 * Each operand has two LDS buffers: step kb runs its MFMAs from buffer kb & 1, then the
 * threads write step kb + 1 into the other (its global loads went out two steps earlier),
 * so a K step needs one barrier. LDS rows are 64 BF16 with an XOR swizzle of their 16-byte
 * chunks (tile_ofs).
 *
 * MFMA operand layout (16x16x32 bf16): lane l supplies row l % 16, k [(l / 16) * 8, +8)
 * of each operand; accumulator i of lane l is D[(l / 16) * 4 + i][l % 16].
 */
#ifndef GLINT_TILE_MFMA_H_
#define GLINT_TILE_MFMA_H_

#include "glint_common.h"

typedef __bf16 glint_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 glint_bf16x2 __attribute__((ext_vector_type(2)));
typedef float glint_f32x2 __attribute__((ext_vector_type(2)));

/* Two f32 to BF16 (round to nearest even; v_cvt_pk_bf16_f32), lo in the low half. */
__device__ __forceinline__ uint32_t glint_cvt_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(glint_f32x2{lo, hi}, glint_bf16x2));
}

/* 128-byte LDS rows (64 BF16), 16-byte chunk c of row r stored at chunk c ^ f(r) with
 * f(r) = ((r >> 1) ^ ((r & 1) << 2)) & 7: the 16 rows of a fragment read (one chunk) then
 * hit distinct banks in every group of 8 lanes and in every group of 16. (Measured no
 * faster than 160-byte padded rows, with 20% less LDS.) */
#define TILE_LDW 64
__device__ __forceinline__ int tile_ofs(int r, int c) {
    return r * TILE_LDW + ((c ^ (((r >> 1) ^ ((r & 1) << 2)) & 7)) << 3);
}

struct TileOutBF16 {
    typedef uint16_t T;
    static __device__ __forceinline__ void store(T *y, int64_t i, float v) { y[i] = glint_f32_to_bf16(v); }
};
struct TileOutF32 {
    typedef float T;
    static __device__ __forceinline__ void store(T *y, int64_t i, float v) { y[i] = v; }
};

/* GLINT planes, bs = 64: weight = CELLS[h][p] * absmax, through the 32-copy LDS table. */
struct GlintTileProducer {
    const glint_u32x2 *hole, *plug; /* 8 B = 16 elements of each plane */
    const float *absmax;
    int N, K;
    float *ltab;
    static constexpr int LDS_WORDS = GLINT_LDS_CELLS_WORDS + 256;
    struct Regs {
        glint_u32x2 h, p;
        float a;
    };
    __device__ __forceinline__ void setup(float *lds) {
        ltab = lds;
        glint_fill_cells_lds(lds, lds + GLINT_LDS_CELLS_WORDS);
    }
    __device__ __forceinline__ void load(Regs &r, int row, int quarter, int kb) const {
        const int64_t q = (int64_t)row * (K >> 4) + kb * 4 + quarter;
        r.h = __builtin_nontemporal_load(&hole[q]);
        r.p = __builtin_nontemporal_load(&plug[q]);
        r.a = absmax[(int64_t)row * (K >> 6) + kb];
    }
    __device__ __forceinline__ void produce(const Regs &r, uint32_t (&packed)[8], int lane) const {
        const uint32_t lb = lane & 31;
        const uint32_t H[2] = {r.h.x, r.h.y}, P[2] = {r.p.x, r.p.y};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t E = glint_codes_even(H[q], P[q]);
            const uint32_t O = glint_codes_odd(H[q], P[q]);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float ve = ltab[(((E >> (8 * b)) & 0xFFu) << 5) | lb] * r.a;
                const float vo = ltab[(((O >> (8 * b)) & 0xFFu) << 5) | lb] * r.a;
                packed[4 * q + b] = glint_cvt_bf16x2(ve, vo);
            }
        }
    }
};

/* INT8 pin (bf16_to_int8_pin_v1), k_in % 64 == 0: weight = BF16 RNE((float)q * scale),
 * scale one f32 per 64 consecutive weights of a row. */
struct Int8PinTileProducer {
    const glint_u32x4 *q; /* 16 weights */
    const float *scale;
    int N, K;
    static constexpr int LDS_WORDS = 0;
    struct Regs {
        glint_u32x4 w;
        float s;
    };
    __device__ __forceinline__ void setup(float *) {}
    __device__ __forceinline__ void load(Regs &r, int row, int quarter, int kb) const {
        r.w = __builtin_nontemporal_load(&q[(int64_t)row * (K >> 4) + kb * 4 + quarter]);
        r.s = scale[(int64_t)row * (K >> 6) + kb];
    }
    __device__ __forceinline__ void produce(const Regs &r, uint32_t (&packed)[8], int) const {
        const uint32_t W[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const float lo = (float)(int8_t)(W[i] >> (16 * b)) * r.s;
                const float hi = (float)(int8_t)(W[i] >> (16 * b + 8)) * r.s;
                packed[2 * i + b] = glint_cvt_bf16x2(lo, hi);
            }
    }
};

template <int BM, int BN, int WM, int WN, class P, class Out>
__global__ __launch_bounds__(64 * WM * WN) void k_tile_mfma(P p, const uint16_t *__restrict__ x,
                                                             typename Out::T *__restrict__ y, int M, int N, int K) {
    constexpr int T = 64 * WM * WN;
    constexpr int TM = BM / WM / 16, TN = BN / WN / 16; /* MFMA tiles per wave */
    constexpr int XV = BM * 8 / T;                      /* x chunks per thread */
    static_assert(BN * 4 == T, "each thread produces a quarter of one W row");
    static_assert(XV * T == BM * 8 && TM * WM * 16 == BM && TN * WN * 16 == BN, "tile shape");
    __shared__ float ptab[P::LDS_WORDS > 0 ? P::LDS_WORDS : 1];
    __shared__ __attribute__((aligned(16))) uint16_t sX[2][BM * TILE_LDW];
    __shared__ __attribute__((aligned(16))) uint16_t sW[2][BN * TILE_LDW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int nK = K >> 6;
    const int wr = tid >> 2, wq = tid & 3;
    const int xr = tid >> 3, xc = tid & 7; /* x chunk i: row xr + (T / 8) i, columns 8 xc */
    glint_f32x4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
            acc[a][b] = glint_f32x4{0.f, 0.f, 0.f, 0.f};

    /* Two register stages alternate over even and odd steps: the loads of step kb + 3 are
     * issued at the end of step kb and written to LDS at the end of step kb + 2. Rows past M
     * or N are clamped into the matrix (their outputs are not stored) and steps past the end
     * reload the last one, so every load is unconditional. */
    struct Stage {
        typename P::Regs w;
        glint_u32x4 x[XV];
    };
    Stage s0, s1;
    const int wrow = min(n0 + wr, N - 1);
    auto gload = [&](int kb, Stage &st) {
        kb = min(kb, nK - 1);
        p.load(st.w, wrow, wq, kb);
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int m = min(m0 + xr + (T / 8) * i, M - 1);
            st.x[i] = *(const glint_u32x4 *)(x + (int64_t)m * K + (int64_t)kb * 64 + xc * 8);
        }
    };
    auto produce = [&](int buf, const Stage &st) {
        uint32_t packed[8];
        p.produce(st.w, packed, lane);
        *(glint_u32x4 *)(sW[buf] + tile_ofs(wr, 2 * wq)) = glint_u32x4{packed[0], packed[1], packed[2], packed[3]};
        *(glint_u32x4 *)(sW[buf] + tile_ofs(wr, 2 * wq + 1)) = glint_u32x4{packed[4], packed[5], packed[6], packed[7]};
#pragma unroll
        for (int i = 0; i < XV; ++i)
            *(glint_u32x4 *)(sX[buf] + tile_ofs(xr + (T / 8) * i, xc)) = st.x[i];
    };
    /* step kb: MFMAs from buffer kb & 1, step kb + 1 (in `next`) into the other buffer, then
     * `next` is refilled with step kb + 3 */
    auto step = [&](int kb, Stage &next) {
        const int cur = kb & 1;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            /* rows (16-row tile base) + lane % 16, chunk 4 ks + lane / 16; the swizzle does not
             * change when a row moves by a multiple of 16 */
            const int fofs = tile_ofs(lane & 15, 4 * ks + (lane >> 4));
            glint_bf16x8 af[TM], bfr[TN];
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[a] = __builtin_bit_cast(glint_bf16x8,
                                           *(const glint_u32x4 *)(sX[cur] + (wm * TM * 16 + a * 16) * TILE_LDW + fofs));
#pragma unroll
            for (int b = 0; b < TN; ++b)
                bfr[b] = __builtin_bit_cast(glint_bf16x8,
                                            *(const glint_u32x4 *)(sW[cur] + (wn * TN * 16 + b * 16) * TILE_LDW + fofs));
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[a], bfr[b], acc[a][b], 0, 0, 0);
        }
        produce(cur ^ 1, next); /* past the end: a clamped copy nobody reads */
        gload(kb + 3, next);
        __syncthreads();
    };

    p.setup(ptab);
    gload(0, s0);
    produce(0, s0);
    gload(1, s1);
    gload(2, s0);
    __syncthreads();
    int kb = 0;
    for (; kb + 2 <= nK; kb += 2) {
        step(kb, s1);
        step(kb + 1, s0);
    }
    if (kb < nK)
        step(kb, s1);
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + wm * TM * 16 + a * 16 + (lane >> 4) * 4 + i;
                const int n = n0 + wn * TN * 16 + b * 16 + (lane & 15);
                if (m < M && n < N)
                    Out::store(y, (int64_t)m * N + n, acc[a][b][i]);
            }
}

#endif
