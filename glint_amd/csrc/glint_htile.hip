/* GLINT H-TILE GEMV / GEMM for gfx950.
 *
 * y[m, n] = sum_k CELLS[h][p] * absmax[(n*K + k) / bs] * x[m, k]
 * (reference cuda/glint_htile.cu:124-164 and glint_htile_sim.py:22-50; f32 arithmetic).
 *
 * k_htile_gemv_xreg — decode (M = 1), bs = 64, K <= 32768: HBM-bound.
 *   Each wave keeps a 2048-wide slice of x in registers (the last slice of a K that is not
 *   a multiple of 2048 partly idle) and streams weight rows past it:
 *   per row, lane l reads 16 B of each nibble plane (32 consecutive k inside one absmax
 *   block), so a wave load is 1 KiB contiguous; rows are multi-buffered in registers. The
 *   cell table sits in LDS as 64 lane-private copies, so lookups never conflict and each
 *   lookup address is one v_perm_b32. Per element: 0.5 op to form code bytes, 1 perm, 1 LDS
 *   read, 1 f32 FMA; per row one FMA by the block absmax and 4 DPP adds.
 * Prefill (M > 1, bf16 out, bs = 64; tile_mfma.h): BF16 MFMA on double-buffered
 *   LDS-dequantized weight tiles, f32 accumulation, K split across workgroups when the
 *   tiles alone would leave CUs idle (fixed-order reduction). k_tile_mfma: 256 x 128 tiles
 *   over 8 waves for M >= 256; k_tile_ss: 64 x 64 / 128 x 64 over 4 waves below, with the
 *   weights loaded a whole 128-B line per 8 lanes. Both are shared with the INT8-pin
 *   W8A16 GEMM.
 * k_htile_generic — every other shape (any M, K, bs, alignment): 64x32 output tiles,
 *   weights decoded to f32 in LDS per 32-wide K step, f32 FMAs in k order.
 */
#include <algorithm>
#include <type_traits>

#include "glint_common.h"
#include "glint_htile.h"
#include "tile_mfma.h"

/* ------------------------------------------------ GEMV with x in registers */
/* For K a multiple of EL (EL = 32 elements per lane; every K with bs = 64): a row is cut
 * into chunks of EL elements (EL/2 bytes of each plane, inside one absmax block) and
 * S = ceil(K / (64 EL)) slices of 64 chunks, the last one partial where 64 EL does not
 * divide K. Wave (s, g) of a workgroup holds slice s
 * of x in registers (lane l: the EL f32 of chunk 64 s + l) and runs rows r0 + g,
 * r0 + g + G, ... of the workgroup's row range; LDS then serves only the cell lookups. Per
 * row a wave loads 32 EL bytes of each plane plus its block scales, rows multi-buffered in
 * registers; its partial sum is folded to 4 row-of-16 sums by DPP and parked in LDS, and
 * after one barrier the workgroup adds the 4 S partials of each row in a fixed order. */
#ifndef GEMV_X_THREADS
#define GEMV_X_THREADS 512 /* most threads per workgroup at S <= 2 (whole waves of S slices are used) */
#endif
#ifndef GEMV_X_THREADS_WIDE
#define GEMV_X_THREADS_WIDE 1024 /* most threads per workgroup at S > 2 */
#endif
#ifndef GEMV_X_WIDE_TARGET
#define GEMV_X_WIDE_TARGET 768 /* S > 2: G = max(2, TARGET / (64 S)) row groups share x through LDS */
#endif
#ifndef GEMV_X_EL
#define GEMV_X_EL 32 /* elements per lane per row: 32 (16-B plane loads) or 16 (8-B) */
#endif
#ifndef GEMV_G1_DIV
#define GEMV_G1_DIV 2 /* one row group per workgroup (G == 1: S > 8): resident grid / this where >= the CUs */
#endif
#ifndef GEMV_X_DEPTH_S2
#define GEMV_X_DEPTH_S2 1 /* rows of loads in flight per wave at S <= 2 slices (K <= 4096) */
#endif
#ifndef GEMV_X_DEPTH
#define GEMV_X_DEPTH 1 /* rows of loads in flight per wave at S > 2 */
#endif
#ifndef GEMV_X_DEPTH_G1
#define GEMV_X_DEPTH_G1 1 /* rows of loads in flight per wave at G == 1 (S > 8: K > 16384; 8192 x 28672: 41.5 us, two rows 44.3, three 45.4) */
#endif
#ifndef GEMV_X_PRE
#define GEMV_X_PRE 8 /* most rows issued before the table fill's barrier */
#endif
#define GEMV_X_PRE_OF(D) ((GEMV_X_PRE) < (D) ? (GEMV_X_PRE) : (D))
#ifndef GEMV_X_NO_RELOAD
#define GEMV_X_NO_RELOAD 1 /* the ring loads no row past the wave's last */
#endif
#ifndef GEMV_X_BATCH
#define GEMV_X_BATCH 4 /* groups of 8 cell lookups a wave may have in flight */
#endif
#ifndef GEMV_X_WPE
#define GEMV_X_WPE 1 /* minimum waves per SIMD the register allocation must allow */
#endif
#define GEMV_X_RED_MAX 4096 /* floats of per-row partials a workgroup may park in LDS */
#define GEMV_X_S_MAX (GEMV_X_THREADS_WIDE / 64) /* most K slices: K <= 32768 at EL = 32 */
/* dynamic LDS of k_htile_gemv_xreg: the row partials, or x as BF16 while it is staged */
#define GEMV_X_STAGE_MAX_K 16384 /* x is staged in LDS at G >= 2, i.e. S <= 8 */
#define GEMV_X_LDS_MAX (GEMV_X_RED_MAX * 4 > GEMV_X_STAGE_MAX_K * 2 ? GEMV_X_RED_MAX * 4 : GEMV_X_STAGE_MAX_K * 2)

template <int EL> struct GemvVec;
template <> struct GemvVec<32> { typedef glint_u32x4 T; };
template <> struct GemvVec<16> { typedef glint_u32x2 T; };

template <int EL>
struct GemvRow {
    typename GemvVec<EL>::T h, p; /* EL packed elements of each plane */
    float a;
};

template <int EL>
__device__ __forceinline__ void gemv_x_load(const void *__restrict__ hole, const void *__restrict__ plug,
                                            const float *__restrict__ absmax, int64_t n, int nch, uint32_t j,
                                            GemvRow<EL> &row) {
    typedef typename GemvVec<EL>::T V;
    row.h = __builtin_nontemporal_load((const V *)hole + n * nch + j);
    row.p = __builtin_nontemporal_load((const V *)plug + n * nch + j);
    row.a = absmax[n * (nch / (64 / EL)) + (j / (64 / EL))];
}

template <int EL>
__device__ __forceinline__ uint32_t gemv_word(const typename GemvVec<EL>::T &v, int q) {
    return v[q];
}

/* The 64-copy cell table through the scalar path: run r (16 B, 4 copies of cell r >> 4) of
 * thread t is t + k blockDim.x, so a wave's 64 runs of step k hold the 4 cells starting at
 * (wave base + k blockDim.x) / 16, one s_load_dwordx4 per step (blockDim.x % 16 == 0).
 * Scalar loads do not queue behind the wave's vector loads of weight rows. 13 steps cover
 * the 4096 runs for blockDim.x >= 316; a loop covers smaller blocks. */
#define GLINT_FILL_STEPS 13
struct GlintCellFillS {
    glint_f32x4 c[GLINT_FILL_STEPS]; /* wave-uniform: lands in scalar registers */
};
__device__ __forceinline__ void glint_cells_fill_sload(GlintCellFillS &f) {
    const int wbase = __builtin_amdgcn_readfirstlane((int)threadIdx.x & ~63);
#pragma unroll
    for (int k = 0; k < GLINT_FILL_STEPS; ++k) {
        const int c0 = min((wbase + k * (int)blockDim.x) >> 4, 252);
        f.c[k] = *(const glint_f32x4 *)(&kCells[0][0] + c0);
    }
}
__device__ __forceinline__ void glint_cells_fill_sstore(float *ltab, const GlintCellFillS &f) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const bool odd = (threadIdx.x >> 4) & 1, high = (threadIdx.x >> 5) & 1; /* cell c0 + (lane >> 4) */
#pragma unroll
    for (int k = 0; k < GLINT_FILL_STEPS; ++k) {
        const int r = (int)threadIdx.x + k * (int)blockDim.x;
        const float lo = odd ? f.c[k].y : f.c[k].x, hi = odd ? f.c[k].w : f.c[k].z;
        const float v = high ? hi : lo;
        if (r < GLINT_LDS_CELLS64_WORDS / 4)
            ((f32x4 *)ltab)[r] = f32x4{v, v, v, v};
    }
    for (int r = threadIdx.x + GLINT_FILL_STEPS * blockDim.x; r < GLINT_LDS_CELLS64_WORDS / 4; r += blockDim.x) {
        const float v = (&kCells[0][0])[r >> 4];
        ((f32x4 *)ltab)[r] = f32x4{v, v, v, v};
    }
}

#ifndef GEMV_HALF_TABLE
#define GEMV_HALF_TABLE 1
#endif
#if GEMV_HALF_TABLE
typedef GlintCellFillH GemvFill;
#define gemv_fill_sload glint_cells_fillh_sload
#define gemv_fill_sstore glint_cells_fillh_sstore
#define GEMV_LANE4(lane) ((uint32_t)((lane) & 31) * 4u)
#else
typedef GlintCellFillS GemvFill;
#define gemv_fill_sload glint_cells_fill_sload
#define gemv_fill_sstore glint_cells_fill_sstore
#define GEMV_LANE4(lane) ((uint32_t)(lane) * 4u)
#endif

/* A lane's partial the way the reference forms it, w = cell * absmax per weight and then
 * the FMA with x, for a block whose absmax is infinite, NaN or at least 2^126: there the
 * factored form (sum of cell * x, times absmax) can give +-inf where products of mixed sign
 * give NaN, or a finite value where a product overflows. Only the f32-out GEMVs take it;
 * `xr` is the lane's 32 elements of x as f32. */
template <int EL>
__device__ __forceinline__ float gemv_exact_part(const float *ltab, const GemvRow<EL> &row, uint32_t lane4,
                                                 const float (&xr)[EL]) {
    float pe = 0.0f;
#pragma unroll
    for (int q = 0; q < EL / 8; ++q) {
        const uint32_t H = gemv_word<EL>(row.h, q), P = gemv_word<EL>(row.p, q);
        const uint32_t E = glint_codes_even(H, P);
        const uint32_t O = glint_codes_odd(H, P);
        pe = fmaf(glint_lds_f32(ltab, glint_cell_addr<0>(E, lane4)) * row.a, xr[8 * q + 0], pe);
        pe = fmaf(glint_lds_f32(ltab, glint_cell_addr<0>(O, lane4)) * row.a, xr[8 * q + 1], pe);
        pe = fmaf(glint_lds_f32(ltab, glint_cell_addr<1>(E, lane4)) * row.a, xr[8 * q + 2], pe);
        pe = fmaf(glint_lds_f32(ltab, glint_cell_addr<1>(O, lane4)) * row.a, xr[8 * q + 3], pe);
        pe = fmaf(glint_lds_f32(ltab, glint_cell_addr<2>(E, lane4)) * row.a, xr[8 * q + 4], pe);
        pe = fmaf(glint_lds_f32(ltab, glint_cell_addr<2>(O, lane4)) * row.a, xr[8 * q + 5], pe);
        pe = fmaf(glint_lds_f32(ltab, glint_cell_addr<3>(E, lane4)) * row.a, xr[8 * q + 6], pe);
        pe = fmaf(glint_lds_f32(ltab, glint_cell_addr<3>(O, lane4)) * row.a, xr[8 * q + 7], pe);
    }
    return pe;
}

/* XC > 0: x goes through LDS. Thread t loads 16-B chunks t + c blockDim.x (c < XC, with
 * XC blockDim.x >= K / 8; threads past the last chunk load it again and store nothing), the
 * G waves of a slice then read it from LDS instead of each loading it from L2. XC == 0:
 * each wave loads its slice itself (G == 1, no repeats). PART: K % (64 EL) != 0, so the
 * last slice holds fewer than 64 chunks; its idle lanes load the row's last chunk again
 * and add nothing. */
template <int EL, bool OUT_BF16, int XC, int DEPTH, int MAXT, bool PART>
__global__ __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(GEMV_X_WPE))) void k_htile_gemv_xreg(
    const void *__restrict__ hole, const void *__restrict__ plug, const float *__restrict__ absmax,
    const glint_u32x4 *__restrict__ x, void *__restrict__ y, int N, int K, int G, int rows_per_wg) {
    __shared__ __attribute__((aligned(16))) float ltab[GLINT_LDS_CELLS64_WORDS]; /* 64 KiB at LDS offset 0 */
    extern __shared__ __attribute__((aligned(16))) float red[]; /* [rows_per_wg][S][4]; first x when XC > 0 */
    constexpr int Q = EL / 8; /* 8-element groups per chunk = packed words per plane */

    const int lane = threadIdx.x & 63;
    const uint32_t lane4 = GEMV_LANE4(lane);
    const int nch = K / EL, S = PART ? (nch + 63) >> 6 : nch >> 6;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int s = w % S, g = w / S;
    const int r0 = blockIdx.x * rows_per_wg;
    const int nrows = max(min(rows_per_wg, N - r0), 0);
    const int my = g < nrows ? (nrows - g + G - 1) / G : 0; /* rows r0 + g + i G, i < my */
    /* row of item i, clamped into the matrix (a clamped reload is never used) */
    auto row_of = [&](int i) -> int64_t { return (int64_t)min(r0 + g + min(i, max(my - 1, 0)) * G, N - 1); };
    const uint32_t j = (uint32_t)(s * 64 + lane);
    const bool act = !PART || j < (uint32_t)nch; /* lane holds a chunk of the row */
    const uint32_t jl = act ? j : (uint32_t)nch - 1u;

    /* Loads go out in the order they are consumed (the wait counter is in order): the
     * cell table, x, then the first rows; the table's LDS writes follow. */
    GemvFill fill;
    gemv_fill_sload(fill);
    glint_u32x4 xv[XC > Q ? XC : Q];
    if (XC > 0) {
#pragma unroll
        for (int c = 0; c < XC; ++c)
            xv[c] = x[min((int)threadIdx.x + c * (int)blockDim.x, (K >> 3) - 1)]; /* clamped: blockDim may exceed K / 8 */
    } else {
#pragma unroll
        for (int q = 0; q < Q; ++q)
            xv[q] = x[jl * Q + q];
    }
    __builtin_amdgcn_sched_barrier(0);
    GemvRow<EL> buf[DEPTH];
#pragma unroll
    for (int d = 0; d < GEMV_X_PRE_OF(DEPTH); ++d)
        gemv_x_load<EL>(hole, plug, absmax, row_of(d), nch, jl, buf[d]);
    __builtin_amdgcn_sched_barrier(0);
    gemv_fill_sstore(ltab, fill);
    if (XC > 0) {
#pragma unroll
        for (int c = 0; c < XC; ++c)
            if ((int)threadIdx.x + c * (int)blockDim.x < (K >> 3))
                ((glint_u32x4 *)red)[threadIdx.x + c * blockDim.x] = xv[c];
    }
    __syncthreads();
    if (XC > 0) {
#pragma unroll
        for (int q = 0; q < Q; ++q)
            xv[q] = ((const glint_u32x4 *)red)[jl * Q + q];
    }
    float xr[EL];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const glint_u32x4 v = xv[q];
        xr[8 * q + 0] = glint_bf16lo(v.x); xr[8 * q + 1] = glint_bf16hi(v.x);
        xr[8 * q + 2] = glint_bf16lo(v.y); xr[8 * q + 3] = glint_bf16hi(v.y);
        xr[8 * q + 4] = glint_bf16lo(v.z); xr[8 * q + 5] = glint_bf16hi(v.z);
        xr[8 * q + 6] = glint_bf16lo(v.w); xr[8 * q + 7] = glint_bf16hi(v.w);
    }
    if (XC > 0)
        __syncthreads(); /* x is read out before the row partials reuse its LDS */
#pragma unroll
    for (int d = GEMV_X_PRE_OF(DEPTH); d < DEPTH; ++d)
        gemv_x_load<EL>(hole, plug, absmax, row_of(d), nch, jl, buf[d]);

    auto compute_row = [&](int i, const GemvRow<EL> &row) {
        float part = 0.0f;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const uint32_t H = gemv_word<EL>(row.h, q), P = gemv_word<EL>(row.p, q);
            const uint32_t E = glint_codes_even(H, P);
            const uint32_t O = glint_codes_odd(H, P);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<0>(E, lane4)), xr[8 * q + 0], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<0>(O, lane4)), xr[8 * q + 1], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<1>(E, lane4)), xr[8 * q + 2], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<1>(O, lane4)), xr[8 * q + 3], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<2>(E, lane4)), xr[8 * q + 4], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<2>(O, lane4)), xr[8 * q + 5], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<3>(E, lane4)), xr[8 * q + 6], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<3>(O, lane4)), xr[8 * q + 7], part);
            /* at most 8 GEMV_X_BATCH lookups in flight per wave: bounds live registers */
            if ((q + 1) % GEMV_X_BATCH == 0)
                __builtin_amdgcn_sched_barrier(0);
        }
        float sc = row.a * part;
        if constexpr (!OUT_BF16)
            if (!(__builtin_fabsf(row.a) < 0x1p126f)) /* rare: the f32 ABI's per-weight products */
                sc = gemv_exact_part<EL>(ltab, row, lane4, xr);
        if (PART && !act)
            sc = 0.0f;
        const float v = glint_row16_sum(sc);
        if ((lane & 15) == 0)
            red[((g + i * G) * S + s) * 4 + (lane >> 4)] = v;
    };

    /* rows i .. i + DEPTH - 1 are in flight at the top of each round; full rounds keep
     * every compute unconditional, so the wait counter can count the loads in flight.
     * Rounds run while every load is of a real row (GEMV_X_NO_RELOAD), then the at most
     * 2 DEPTH - 1 rows left load only what exists: a clamped re-load of the last row would be
     * a request for nothing. */
    int i = 0;
#if GEMV_X_NO_RELOAD
    for (; i + 2 * DEPTH <= my; i += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            compute_row(i + d, buf[d]);
            gemv_x_load<EL>(hole, plug, absmax, row_of(i + d + DEPTH), nch, jl, buf[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
        if (i + d < my) {
            compute_row(i + d, buf[d]);
            if (i + d + DEPTH < my)
                gemv_x_load<EL>(hole, plug, absmax, row_of(i + d + DEPTH), nch, jl, buf[d]);
        }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
        if (i + DEPTH + d < my)
            compute_row(i + DEPTH + d, buf[d]);
#else
    for (; i + DEPTH <= my; i += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            compute_row(i + d, buf[d]);
            gemv_x_load<EL>(hole, plug, absmax, row_of(i + d + DEPTH), nch, jl, buf[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d)
        if (i + d < my)
            compute_row(i + d, buf[d]);
#endif
    __syncthreads();

    for (int t = threadIdx.x; t < nrows; t += blockDim.x) {
        const int row = r0 + t;
        float sum = 0.0f;
        for (int k = 0; k < S * 4; ++k)
            sum += red[t * S * 4 + k];
        if (OUT_BF16)
            ((uint16_t *)y)[row] = glint_f32_to_bf16(sum);
        else
            ((float *)y)[row] = sum;
    }
}

/* ------------------------------------- decode GEMV, claimed items, one item in flight */
/* k_htile_gemv_cu: M = 1, bs = 64, K % 2048 == 0, K <= 32768, aligned. The per-element
 * work of k_htile_gemv_xreg (x slice in registers, 64-copy cell table, 16 B per lane per
 * plane per item), with a different split and schedule:
 *   - an item is (row, K slice of 2048). A workgroup holds G waves per slice (64 S G
 *     threads) and a contiguous band of rows. Wave (s, g) takes items g and g + G of slice
 *     s, then claims the slice's next items from an LDS counter. The SIMD arbiter issues for
 *     the oldest waves first, so waves with equal static shares end far apart; claimed items
 *     let the favoured waves take more of the band.
 *   - one item in flight per wave: wait for the item, issue the next item's loads, then
 *     look up and multiply. A plain read of these bytes streams faster with one 1 KiB piece
 *     per wave in flight than with two. The next item's byte offsets are formed before the
 *     wait, so once an item lands the wave's next instructions are its loads, not VALU work
 *     queued behind older waves' lookups.
 *   - loads are raw buffer loads over the band: an item past the band's end reads beyond the
 *     buffer's range, which the hardware drops (no memory request, zeros back), so no load
 *     sits under a branch and the wait counter tracks exactly one item in flight.
 *   - each (row, slice) partial has its own LDS slot and the workgroup adds a row's slots in
 *     a fixed order, so results do not depend on which wave took which item (bit-identical
 *     to k_htile_gemv_xreg).
 * Two shapes of launch (template NT):
 *   - S <= 2 (K <= 4096, the gate/up shape): 512-thread workgroups, two per CU; x and the
 *     first two items go out together.
 *   - S > 2 (the down shape): one workgroup of 64 S G <= 1024 threads per CU (the 64 KiB x
 *     stage keeps a second one off the CU); each wave's x chunk lands before its weight
 *     loads go out (then its first two items), since x issued together with them is served
 *     behind the weights of every wave that started earlier (x 1.6 us median into a launch,
 *     2.6 us at worst).
 * Measured against k_htile_gemv_xreg in one process (rotated pins): 14336 x 4096 11.68
 * against 11.94 us, 4096 x 14336 12.00 against 12.75 us. */
#define GEMV_CU_SMAX 16 /* K <= 32768 */
#define GEMV_CU_DYN_MAX (28 * 1024) /* bytes of dynamic LDS: the partials, 16 S per row */

/* Per-wave timeline of k_htile_gemv_cu, compiled only into the measurement library
 * libglint_encode_tl.so (-DGLINT_TIMELINE). A wave keeps its stamps in registers and
 * lane 0 stores them when the wave ends, so each launch overwrites the slots of the one
 * before it and the last launch's stamps remain. Slots of wave blockIdx.x * waves + w:
 *   0 s_memrealtime (100 MHz) at entry      1 XCC_ID << 32 | HW_ID
 *   2 s_memtime (shader clock) at entry     3 s_memrealtime after the first item
 *   4 s_memrealtime after the item loop     5 s_memrealtime after the row stores
 *   6 items computed by the wave            7 s_memtime after the row stores */
#ifdef GLINT_TIMELINE
#define GLINT_TL_SLOTS 8
#define GLINT_TL_WAVES 16384
__device__ unsigned long long g_glint_tl[GLINT_TL_WAVES * GLINT_TL_SLOTS];
extern "C" __attribute__((visibility("default"))) int glint_timeline_fetch(void *dst, size_t bytes) {
    if (!dst || bytes > sizeof(g_glint_tl))
        return (int)hipErrorInvalidValue;
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_glint_tl), bytes, 0, hipMemcpyDeviceToHost);
}
#define GEMV_TL(stmt) stmt
#else
#define GEMV_TL(stmt)
#endif

template <bool OUT_BF16, int XC, int NT, int XS, bool XFIRST>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_htile_gemv_cu(
    const uint8_t *__restrict__ hole, const uint8_t *__restrict__ plug, const float *__restrict__ absmax,
    const glint_u32x4 *__restrict__ x, void *__restrict__ y, int N, int K, int G, int rows_per_wg) {
    /* One block, so the table sits at LDS offset 0 (a lookup address is then one v_perm). */
    __shared__ struct __attribute__((aligned(16))) {
        float ltab[GLINT_LDS_CELLS64_WORDS];
        glint_u32x4 xs[XS]; /* x as BF16, XS >= K / 8 chunks of 16 B */
        int claim[GEMV_CU_SMAX];
    } sh;
    float *const ltab = sh.ltab;
    glint_u32x4 *const xs = sh.xs;
    int *const claim = sh.claim;
    extern __shared__ __attribute__((aligned(16))) float red[]; /* [rows_per_wg][S][4] */
    constexpr int EL = 32, Q = EL / 8;
    const int lane = threadIdx.x & 63;
    const uint32_t lane4 = GEMV_LANE4(lane);
    const int S = K >> 11;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int s = w % S, g = w / S;
    const int r0 = blockIdx.x * rows_per_wg;
    const int nrows = max(min(rows_per_wg, N - r0), 0);
    GEMV_TL(const unsigned long long tl_t0 = __builtin_amdgcn_s_memrealtime();
            const unsigned long long tl_m0 = __builtin_amdgcn_s_memtime();
            const unsigned long long tl_hw = ((unsigned long long)__builtin_amdgcn_s_getreg(63508) << 32) |
                                             (unsigned)__builtin_amdgcn_s_getreg(63492);
            unsigned long long tl_t1 = 0; int tl_items = 0;)

    /* the band's rows of each plane and of absmax; offsets at or past num_records load zeros */
    const uint32_t rowb = (uint32_t)K >> 1; /* bytes of a row in each plane */
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(hole + (int64_t)r0 * rowb), (short)0, (int)((uint32_t)nrows * rowb), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(plug + (int64_t)r0 * rowb), (short)0, (int)((uint32_t)nrows * rowb), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(absmax + (int64_t)r0 * (K >> 6)), (short)0, (int)((uint32_t)nrows * (rowb >> 3)), GLINT_BUF_DWORD3);
    const uint32_t lofs = (uint32_t)(s * 1024 + lane * 16), aofs = (uint32_t)(s * 128 + (lane >> 1) * 4);
    /* an item's two byte offsets, formed ahead of the wait that precedes its loads */
    struct Ofs {
        uint32_t w, a;
    };
    auto ofs = [&](int i) -> Ofs { return {(uint32_t)i * rowb + lofs, (uint32_t)i * (rowb >> 3) + aofs}; };
    auto load_at = [&](Ofs o, GemvRow<EL> &row) {
        row.h = __builtin_amdgcn_raw_buffer_load_b128(rh, o.w, 0, 2 /* nt */);
        row.p = __builtin_amdgcn_raw_buffer_load_b128(rp, o.w, 0, 2);
        row.a = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ra, o.a, 0, 0));
    };
    auto load = [&](int i, GemvRow<EL> &row) { load_at(ofs(i), row); };

    /* loads in the order they are consumed: the cell table (scalar), x, the first items */
    GemvFill fill;
    gemv_fill_sload(fill);
    glint_u32x4 xv[XC];
#pragma unroll
    for (int c = 0; c < XC; ++c)
        xv[c] = x[min((int)threadIdx.x + c * (int)blockDim.x, (K >> 3) - 1)];
    __builtin_amdgcn_sched_barrier(0);
    if (XFIRST) /* x lands before this wave's weight loads go out */
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0);
    __builtin_amdgcn_sched_barrier(0);
    /* items g and g + G of slice s are static and both go out before the barrier that waits
     * for the table and x, so the stream does not pause while the prologue finishes (the
     * steady state then keeps one item in flight) */
    int cur = g, nxt = g + G;
    GemvRow<EL> bufA, bufB;
    load(cur, bufA);
    __builtin_amdgcn_sched_barrier(0);
    load(nxt, bufB);
    __builtin_amdgcn_sched_barrier(0);
    gemv_fill_sstore(ltab, fill);
#pragma unroll
    for (int c = 0; c < XC; ++c)
        if ((int)threadIdx.x + c * (int)blockDim.x < (K >> 3))
            xs[threadIdx.x + c * blockDim.x] = xv[c];
    if ((int)threadIdx.x < S)
        claim[threadIdx.x] = 2 * G;
    __syncthreads();
    float xr[EL];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const glint_u32x4 v = xs[(s * 64 + lane) * Q + q];
        xr[8 * q + 0] = glint_bf16lo(v.x); xr[8 * q + 1] = glint_bf16hi(v.x);
        xr[8 * q + 2] = glint_bf16lo(v.y); xr[8 * q + 3] = glint_bf16hi(v.y);
        xr[8 * q + 4] = glint_bf16lo(v.z); xr[8 * q + 5] = glint_bf16hi(v.z);
        xr[8 * q + 6] = glint_bf16lo(v.w); xr[8 * q + 7] = glint_bf16hi(v.w);
    }
    /* The counter's address goes through an empty asm, so the compiler does not see it as
     * wave-uniform: its atomic optimizer would otherwise rewrite the add into a form that
     * waits for the result right away. Only lane 0 adds; the result is read one item later,
     * so its LDS round trip is hidden and no atomic sits among the lookups. */
    typedef __attribute__((address_space(3))) int lds_int;
    lds_int *claim_s = (lds_int *)&claim[s];
    asm volatile("" : "+v"(claim_s));
    auto claim_one = [&]() -> int {
        int v = 0;
        if (lane == 0)
            v = __hip_atomic_fetch_add(claim_s, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return v;
    };
    int pend = claim_one();

    auto compute = [&](const GemvRow<EL> &row, int item) {
        float part = 0.0f;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const uint32_t H = gemv_word<EL>(row.h, q), P = gemv_word<EL>(row.p, q);
            const uint32_t E = glint_codes_even(H, P);
            const uint32_t O = glint_codes_odd(H, P);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<0>(E, lane4)), xr[8 * q + 0], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<0>(O, lane4)), xr[8 * q + 1], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<1>(E, lane4)), xr[8 * q + 2], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<1>(O, lane4)), xr[8 * q + 3], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<2>(E, lane4)), xr[8 * q + 4], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<2>(O, lane4)), xr[8 * q + 5], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<3>(E, lane4)), xr[8 * q + 6], part);
            part = fmaf(glint_lds_f32(ltab, glint_cell_addr<3>(O, lane4)), xr[8 * q + 7], part);
            if ((q + 1) % GEMV_X_BATCH == 0)
                __builtin_amdgcn_sched_barrier(0);
        }
        float sc = row.a * part;
        if constexpr (!OUT_BF16)
            if (!(__builtin_fabsf(row.a) < 0x1p126f)) /* rare: the f32 ABI's per-weight products */
                sc = gemv_exact_part<EL>(ltab, row, lane4, xr);
        const float v = glint_row16_sum(sc);
        if ((lane & 15) == 0)
            red[(item * S + s) * 4 + (lane >> 4)] = v;
        GEMV_TL(++tl_items;)
    };
    /* first item (landed before the barrier) */
    if (cur < nrows)
        compute(bufA, cur);
    GEMV_TL(tl_t1 = __builtin_amdgcn_s_memrealtime();)
    /* steady state: wait for the item in `row` (the only one in flight), send the next
     * claimed item's loads into `other` (past the band they are dropped by the buffer range
     * check), compute. Items are claimed in increasing order, so once `nxt` is past the band
     * every later one is. The loads sit outside any branch and the loop runs in pairs, so the
     * wait counter tracks exactly one item in flight. */
    auto step = [&](GemvRow<EL> &row, GemvRow<EL> &other) {
        cur = nxt;
        nxt = __builtin_amdgcn_readfirstlane(pend);
        pend = claim_one();
        /* the next item's offsets go ahead of the wait, so once `row` lands the wave's next
         * instructions are the loads themselves, not VALU work queued behind older waves'
         * lookups */
        const Ofs o = ofs(nxt);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0);
        __builtin_amdgcn_sched_barrier(0);
        load_at(o, other);
        __builtin_amdgcn_sched_barrier(0);
        if (cur < nrows)
            compute(row, cur);
    };
    while (nxt < nrows) {
        step(bufB, bufA);
        step(bufA, bufB);
    }
    GEMV_TL(const unsigned long long tl_t2 = __builtin_amdgcn_s_memrealtime();)
    __syncthreads();

    for (int t = threadIdx.x; t < nrows; t += blockDim.x) {
        const int row = r0 + t;
        float sum = 0.0f;
        for (int k = 0; k < S * 4; ++k)
            sum += red[t * S * 4 + k];
        if (OUT_BF16)
            ((uint16_t *)y)[row] = glint_f32_to_bf16(sum);
        else
            ((float *)y)[row] = sum;
    }
#ifdef GLINT_TIMELINE
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0); /* the row stores have left the wave */
    const unsigned long long tl_t3 = __builtin_amdgcn_s_memrealtime(), tl_m1 = __builtin_amdgcn_s_memtime();
    const int tl_w = (int)blockIdx.x * (int)(blockDim.x >> 6) + w;
    if (lane == 0 && tl_w < GLINT_TL_WAVES) {
        unsigned long long *o = g_glint_tl + (size_t)tl_w * GLINT_TL_SLOTS;
        o[0] = tl_t0; o[1] = tl_hw; o[2] = tl_m0; o[3] = tl_t1;
        o[4] = tl_t2; o[5] = tl_t3; o[6] = (unsigned long long)tl_items; o[7] = tl_m1;
    }
#endif
}

/* ------------------------------------------------- small-M decode GEMV (BF16 out) */
/* k_htile_gemv_mr: M = 2 .. MR rows of x at once (batched decode), bs = 64, K % 2048 == 0,
 * aligned. The layout and row walk of k_htile_gemv_xreg: wave (s, g) streams rows
 * r0 + g, r0 + g + G, ... over K slice s, 32 elements per lane per row. Each weight is
 * looked up once for all MR rows of x: the cells of a pair of elements are rounded to one
 * BF16 pair, which v_dot2_f32_bf16 multiplies into the f32 partial of each row against the
 * row's BF16 pair of x (x stays in registers as loaded, MR x 16 words per lane); the block
 * absmax scales each partial once per row. So the weights are read once whatever M is,
 * where the MFMA tiles cost the same at M = 2 as at M = 64. Numerics: the weights enter as
 * BF16(cell) x absmax, the tiles' BF16(cell x absmax) up to one rounding of the scale;
 * both within the BF16 API's 1e-2 relative Frobenius bound. Rows of x past M repeat row
 * M - 1 and are not stored. */
typedef __bf16 glint_bf16x2_t __attribute__((ext_vector_type(2)));
/* F32: the f32-out form (the reference ABI's launch_glint_htile_s3_f32_stream at M = 2 .. 4):
 * x held as f32 (MR x 32 registers) and one f32 FMA per weight and row in k order, the
 * weights the exact f32 cells; the same arithmetic per row as the M = 1 f32 GEMV, so the
 * same (K + 2) 2^-23 sum |w x| bound. */
template <int MR, bool F32, bool PART, int MAXT, int DEPTH>
__global__ __launch_bounds__(MAXT) void k_htile_gemv_mr(const void *__restrict__ hole,
                                                                  const void *__restrict__ plug,
                                                                  const float *__restrict__ absmax,
                                                                  const uint16_t *__restrict__ x,
                                                                  void *__restrict__ y, int M, int N, int K,
                                                                  int G, int rows_per_wg) {
    __shared__ __attribute__((aligned(16))) float ltab[GLINT_LDS_CELLS64_WORDS]; /* 64 KiB at LDS offset 0 */
    extern __shared__ __attribute__((aligned(16))) float red[]; /* [rows_per_wg][S][4][MR] */
    constexpr int EL = 32, Q = EL / 8;
    const int lane = threadIdx.x & 63;
    const uint32_t lane4 = GEMV_LANE4(lane);
    const int nch = K / EL, S = PART ? (nch + 63) >> 6 : nch >> 6;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int s = w % S, g = w / S;
    const int r0 = blockIdx.x * rows_per_wg;
    const int nrows = max(min(rows_per_wg, N - r0), 0);
    const int my = g < nrows ? (nrows - g + G - 1) / G : 0;
    auto row_of = [&](int i) -> int64_t { return (int64_t)min(r0 + g + min(i, max(my - 1, 0)) * G, N - 1); };
    const uint32_t j = (uint32_t)(s * 64 + lane);
    const bool act = !PART || j < (uint32_t)nch; /* PART: idle lanes of the last slice */
    const uint32_t jl = act ? j : (uint32_t)nch - 1u;

    GemvFill fill;
    gemv_fill_sload(fill);
    /* x: row m's 32 elements [32 j, 32 j + 32) as 16 words of BF16 pairs */
    glint_u32x4 xv[MR][4];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const glint_u32x4 *xr = (const glint_u32x4 *)(x + (int64_t)min(m, M - 1) * K) + (size_t)jl * 4;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            xv[m][c] = xr[c];
    }
    __builtin_amdgcn_sched_barrier(0);
    GemvRow<EL> buf[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
        gemv_x_load<EL>(hole, plug, absmax, row_of(d), nch, jl, buf[d]);
    __builtin_amdgcn_sched_barrier(0);
    gemv_fill_sstore(ltab, fill);
    __syncthreads();
    float xf[F32 ? MR : 1][F32 ? 32 : 1];
    if constexpr (F32) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t xw = xv[m][e >> 2][e & 3];
                xf[m][2 * e] = glint_bf16lo(xw);
                xf[m][2 * e + 1] = glint_bf16hi(xw);
            }
    }

    auto compute_row = [&](int i, const GemvRow<EL> &row) {
        float part[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m)
            part[m] = 0.0f;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const uint32_t H = gemv_word<EL>(row.h, q), P = gemv_word<EL>(row.p, q);
            const uint32_t E = glint_codes_even(H, P);
            const uint32_t O = glint_codes_odd(H, P);
            float c[8];
            c[0] = glint_lds_f32(ltab, glint_cell_addr<0>(E, lane4));
            c[1] = glint_lds_f32(ltab, glint_cell_addr<0>(O, lane4));
            c[2] = glint_lds_f32(ltab, glint_cell_addr<1>(E, lane4));
            c[3] = glint_lds_f32(ltab, glint_cell_addr<1>(O, lane4));
            c[4] = glint_lds_f32(ltab, glint_cell_addr<2>(E, lane4));
            c[5] = glint_lds_f32(ltab, glint_cell_addr<2>(O, lane4));
            c[6] = glint_lds_f32(ltab, glint_cell_addr<3>(E, lane4));
            c[7] = glint_lds_f32(ltab, glint_cell_addr<3>(O, lane4));
            if constexpr (F32) {
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        part[m] = fmaf(c[e], xf[m][8 * q + e], part[m]);
            } else {
                uint32_t wp[4];
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    wp[b] = glint_cvt_bf16x2(c[2 * b], c[2 * b + 1]);
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        /* the word as a value: this compiler bit-casts a vector element in
                         * place as element 0 */
                        const uint32_t xw = xv[m][q][b];
                        part[m] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(glint_bf16x2_t, wp[b]),
                                                                  __builtin_bit_cast(glint_bf16x2_t, xw), part[m],
                                                                  false);
                    }
            }
        }
        const int t = g + i * G;
        float sc[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m)
            sc[m] = row.a * part[m];
        if constexpr (F32)
            if (!(__builtin_fabsf(row.a) < 0x1p126f)) /* rare: the f32 ABI's per-weight products */
#pragma unroll
                for (int m = 0; m < MR; ++m)
                    sc[m] = gemv_exact_part<EL>(ltab, row, lane4, xf[m]);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (PART && !act)
                sc[m] = 0.0f;
            const float v = glint_row16_sum(sc[m]);
            if ((lane & 15) == 0)
                red[((t * S + s) * 4 + (lane >> 4)) * MR + m] = v;
        }
    };
    /* DEPTH rows in flight, full rounds while every load is of a real row (as in
     * k_htile_gemv_xreg) */
    int i = 0;
    for (; i + 2 * DEPTH <= my; i += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            compute_row(i + d, buf[d]);
            gemv_x_load<EL>(hole, plug, absmax, row_of(i + d + DEPTH), nch, jl, buf[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
        if (i + d < my) {
            compute_row(i + d, buf[d]);
            if (i + d + DEPTH < my)
                gemv_x_load<EL>(hole, plug, absmax, row_of(i + d + DEPTH), nch, jl, buf[d]);
        }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
        if (i + DEPTH + d < my)
            compute_row(i + DEPTH + d, buf[d]);
    __syncthreads();

    for (int e = threadIdx.x; e < nrows * MR; e += blockDim.x) {
        const int t = e / MR, m = e % MR;
        if (m >= M)
            continue;
        float sum = 0.0f;
        for (int k = 0; k < S * 4; ++k)
            sum += red[(t * S * 4 + k) * MR + m];
        if (F32)
            ((float *)y)[(int64_t)m * N + r0 + t] = sum;
        else
            ((uint16_t *)y)[(int64_t)m * N + r0 + t] = glint_f32_to_bf16(sum);
    }
}

#ifndef GEMV_MR_ON
#define GEMV_MR_ON 1
#endif
#ifndef GEMV_MR_MAX
#define GEMV_MR_MAX 8 /* largest M the small-M GEMV takes (templates for 2, 4 and 8 rows) */
#endif
/* k_htile_gemv_mr over 2 <= M <= GEMV_MR_MAX (bs 64, K % 64 == 0, aligned; K <= 16384, and
 * up to 32768 where x fits the wide workgroups), the f32-out form up to GEMV_MR_MAX_F32 rows.
 * Measured against the 64-row MFMA tile (k_tile_ss) on 14336 x 4096: M = 2 14.2-15.6 us
 * against 35.0, M = 4 17.8-18.2 against 35.3, M = 5..8 24.7-24.9 against 34.3-34.6 (the
 * 8-row template holds 128 VGPRs of x and runs at 2 waves per SIMD). */
#ifndef GEMV_MR_RL
#define GEMV_MR_RL 4 /* BF16 out: above this many rows k_htile_rl goes first where it takes the shape */
#endif
#ifndef GEMV_MR_RL_F32
#define GEMV_MR_RL_F32 6 /* f32 out: above this many rows k_htile_rl goes first where it takes the shape */
#endif
#ifndef GEMV_MR_MAX_F32
#define GEMV_MR_MAX_F32 4 /* largest M of the f32-out small-M GEMV (x as f32: MR x 32 registers) */
#endif
/* Rows in flight per wave: one for BF16 out (against two: 14336 x 4096 M = 2 14.1 -> 13.4 us,
 * M = 4 17.1 -> 16.4, M = 8 24.4 -> 23.7; 4096 x 14336 M = 2 14.4 -> 13.9; three slower), two
 * for f32 out (one: 14336 x 4096 M = 4 16.4 -> 22.0 us) */
#ifndef GEMV_MR_DEPTH_BF16
#define GEMV_MR_DEPTH_BF16 1
#endif
#ifndef GEMV_MR_DEPTH_F32
#define GEMV_MR_DEPTH_F32 2
#endif
#ifndef GEMV_MR_F32_TWICE
#define GEMV_MR_F32_TWICE 1 /* f32 out at M = 5 .. 8 as two small-M launches */
#endif
#define GEMV_MR_RED_ONE 22528 /* floats of row partials a small-M workgroup alone on its CU may park in LDS (88 KiB) */
#ifndef GEMV_MR_WIDE
#define GEMV_MR_WIDE 1 /* S > 2: the M = 1 kernel's wider workgroups where x fits (see gemv_mr_wide_ok) */
#endif
/* rows of x per template for M rows */
static inline int gemv_mr_rows(int M, bool f32) { return M <= 2 ? 2 : (M <= 4 || f32 ? 4 : 8); }
/* Wider workgroups (up to 1024 threads: at most 128 VGPRs) only for BF16 out with up to
 * 4 rows (x as 64 registers of BF16 words, 114 VGPRs); the f32 form of even 2 rows
 * (x as 64 f32, 140 VGPRs) would spill. */
static inline bool gemv_mr_wide_ok(int MR, bool f32) { return GEMV_MR_WIDE && !f32 && MR <= 4; }
/* Workgroups over S slices: up to GEMV_X_THREADS threads (G = 8 / S row groups, S <= 8),
 * or the M = 1 kernel's wider ones where those hold fewer than 7 waves (S = 3, 5, 6) or
 * cannot hold S (S > 8). Measured (wide against narrow, M = 2 / 4): 4096 x 6144 8.3 / 11.0
 * against 9.2 / 11.6 us, 4096 x 12288 12.6 / 15.7 against 13.5 / 17.6; narrow better at
 * S = 4 (8192 x 8192 14.9 / 18.5 against 15.8 / 19.3) and S = 7 (4096 x 14336). */
static inline bool gemv_mr_is_wide(int S, int MR, bool f32) {
    return gemv_mr_wide_ok(MR, f32) && S > 2 && (S > 8 || S * ((GEMV_X_THREADS / 64) / S) < 7);
}
/* row groups per workgroup, 0 where the template cannot take S */
static inline int gemv_mr_groups(int S, int MR, bool f32) {
    if (!gemv_mr_is_wide(S, MR, f32))
        return S <= 8 ? (GEMV_X_THREADS / 64) / S : 0;
    return std::min(std::max(2, (GEMV_X_WIDE_TARGET / 64) / S), (GEMV_X_THREADS_WIDE / 64) / S);
}
/* whether k_htile_gemv_mr takes M rows at this K (bs 64, K % 64 == 0). The 8-row template is
 * VALU-bound at 2 waves per SIMD; with a partial last slice it was slower than the tiles
 * (13824 x 5120: 63.9 against 42.3 us), so it takes only K % 2048 == 0. */
static inline bool gemv_mr_takes(int M, int K, bool f32) {
    const int S = (K / 2048) + (K % 2048 != 0), MR = gemv_mr_rows(M, f32);
    if (M < 2 || M > (f32 ? GEMV_MR_MAX_F32 : GEMV_MR_MAX) || S > GEMV_X_S_MAX)
        return false;
    if (MR == 8 && (K % 2048) != 0)
        return false;
    return gemv_mr_groups(S, MR, f32) >= 1;
}
template <bool F32>
static int htile_launch_gemv_mr(const uint8_t *hole, const uint8_t *plug, const float *absmax, const void *x, void *y,
                                int M, int N, int K, hipStream_t st) {
    if (!gemv_mr_takes(M, K, F32))
        return -3;
    const int S = (K / 2048) + (K % 2048 != 0), MR = gemv_mr_rows(M, F32), G = gemv_mr_groups(S, MR, F32);
    const int threads = 64 * S * G;
    const bool part = (K % 2048) != 0, wide = gemv_mr_is_wide(S, MR, F32);
    auto pick = [&](auto mr_c) {
        constexpr int R = decltype(mr_c)::value;
        constexpr bool W = !F32 && R <= 4; /* wide templates only where x fits (gemv_mr_wide_ok) */
        constexpr int TW = W ? GEMV_X_THREADS_WIDE : GEMV_X_THREADS;
        constexpr int D = F32 ? GEMV_MR_DEPTH_F32 : GEMV_MR_DEPTH_BF16;
        return part ? (wide ? k_htile_gemv_mr<R, F32, true, TW, D> : k_htile_gemv_mr<R, F32, true, GEMV_X_THREADS, D>)
                    : (wide ? k_htile_gemv_mr<R, F32, false, TW, D> : k_htile_gemv_mr<R, F32, false, GEMV_X_THREADS, D>);
    };
    decltype(&k_htile_gemv_mr<2, F32, false, GEMV_X_THREADS, 2>) kern;
    if (MR == 2)
        kern = pick(std::integral_constant<int, 2>{});
    else if (MR == 4)
        kern = pick(std::integral_constant<int, 4>{});
    else if constexpr (!F32) /* no 8-row f32 form: 256 registers of x */
        kern = pick(std::integral_constant<int, 8>{});
    else
        return -3;
    /* the whole resident grid: halving it where a workgroup holds one row group, as the M = 1
     * kernel does, was slower here (4096 x 14336 f32 out at M = 4: 30.1 against 18.6 us).
     * Where only one workgroup fits a CU anyway (the wide ones, and the narrow ones whose
     * registers allow 2 or 3 waves per SIMD), its row partials may take GEMV_MR_RED_ONE
     * floats of LDS beside the 64 KiB table: with 16 KiB, 8192 x 28672 at M = 4 held 18 rows
     * per workgroup (two generations of workgroups) */
    int red_max = GEMV_X_RED_MAX;
    int64_t resident = std::max<int64_t>(glint_resident_grid((const void *)kern, threads, (size_t)red_max * 4), 1);
    if (resident <= glint_cu_count()) {
        red_max = GEMV_MR_RED_ONE;
        resident = std::max<int64_t>(glint_resident_grid((const void *)kern, threads, (size_t)red_max * 4), 1);
    }
    const int64_t per_wave = ((int64_t)N + G * resident - 1) / (G * resident);
    int64_t rows_per_wg = G * per_wave;
    const int64_t cap = (red_max / (S * 4 * MR)) / G * G;
    if (rows_per_wg > cap)
        rows_per_wg = cap;
    if (rows_per_wg < 1)
        return -3;
    const unsigned grid = (unsigned)((N + rows_per_wg - 1) / rows_per_wg);
    const size_t lds = (size_t)rows_per_wg * S * 4 * MR * sizeof(float);
    if (glint_set_lds_limit((const void *)kern, (size_t)red_max * 4) != 0)
        return -3;
    kern<<<grid, threads, lds, st>>>(hole, plug, absmax, (const uint16_t *)x, y, M, N, K, G, (int)rows_per_wg);
    return hipGetLastError() == hipSuccess ? 0 : -3;
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
/* Prefill GEMM, large M: the shared double-buffered tile kernel with 256 (M) x 128 (N)
 * blocks over 8 waves in 4 x 2 (wave tile 64 x 64); each thread dequantizes 16 weights
 * (8 B of each plane) per K step through the 32-copy cell table. */
#ifndef TILE_SS_BN32
#define TILE_SS_BN32 1 /* M <= 64: 64 x 32 tiles, two workgroups per CU */
#endif
#ifndef TILE_RX
#define TILE_RX 4 /* x register stages of k_tile_ss (M < 256) */
#endif
#ifndef TILE_R_BIG
#define TILE_R_BIG 2 /* register stages (K steps of loads in flight) of the 256 x 128 tiles */
#endif
#define MF2_BM 256
#define MF2_BN 128
#ifndef MF2_MIN_M
#define MF2_MIN_M 256 /* smallest M that takes the 256 x 128 tiles */
#endif

/* ------------------------------------------------------------------ dispatch */
/* k_htile_gemv_xreg over an M = 1 GEMV (bs 64, K % 64 == 0, K <= 64 EL GEMV_X_S_MAX, aligned).
 * A partial last slice (K % 2048 != 0) replaced an x-in-LDS GEMV that ran those shapes at
 * 45-49% of HBM: 13824 x 5120 19.5 -> 15.4 us, 5120 x 13824 20.7 -> 15.0, 5120 x 5120
 * 11.6 -> 8.5, 8192 x 3072 9.8 -> 8.0. EL = 16 (8-B plane loads) was slower than both
 * (13824 x 5120: 24.8 us).
 * Workgroups: up to GEMV_X_THREADS threads at S <= 2 (two per CU); at S > 2 about
 * GEMV_X_WIDE_TARGET threads and at least G = 2 row groups sharing one staged x, one
 * row in flight per wave. Against at most 512 threads (G = 1 at S >= 5, on half the
 * resident grid) with two rows in flight: 4096 x 6144 8.2 -> 7.8 us, 4096 x 10240
 * 12.3 -> 10.5, 4096 x 12288 12.3 -> 11.3, 4096 x 14336 13.1 -> 12.8, 28672 x 8192
 * 40.6 -> 39.4; 4096 x 16384 equal. */
template <bool OUT_BF16, int EL = GEMV_X_EL>
static int htile_launch_gemv_xreg(const uint8_t *hole, const uint8_t *plug, const float *absmax, const void *x,
                                  void *y, int N, int K, hipStream_t st) {
    const int S = (K / EL + 63) / 64;
    const bool part = (K % (64 * EL)) != 0;
    const int G = S <= 2 ? (GEMV_X_THREADS / 64) / S
                         : std::min(std::max(2, (GEMV_X_WIDE_TARGET / 64) / S), (GEMV_X_THREADS_WIDE / 64) / S);
    const int threads = 64 * S * G;
    if (G < 1 || (G >= 2 && (size_t)K * 2 > GEMV_X_LDS_MAX))
        return -3;
    /* x staging (G >= 2): K / 8 chunks of 16 B over 64 S G threads, XC chunks per thread;
     * S <= 2 (G >= 4): one chunk, one row in flight per wave; more slices: GEMV_X_DEPTH */
    auto pick = [&](auto part_c) {
        constexpr bool P = decltype(part_c)::value;
        return S <= 2 ? k_htile_gemv_xreg<EL, OUT_BF16, 1, GEMV_X_DEPTH_S2, GEMV_X_THREADS, P>
                      : (G >= 2 ? k_htile_gemv_xreg<EL, OUT_BF16, 2, GEMV_X_DEPTH, GEMV_X_THREADS_WIDE, P>
                                : k_htile_gemv_xreg<EL, OUT_BF16, 0, GEMV_X_DEPTH_G1, GEMV_X_THREADS_WIDE, P>);
    };
    auto kern = part ? pick(std::true_type{}) : pick(std::false_type{});
    const size_t lds_max = G >= 2 ? std::max<size_t>(GEMV_X_RED_MAX * 4, (size_t)K * 2) : GEMV_X_RED_MAX * 4;
    int64_t resident = std::max<int64_t>(glint_resident_grid((const void *)kern, threads, lds_max), 1);
    if (G == 1 && resident / GEMV_G1_DIV >= glint_cu_count())
        resident /= GEMV_G1_DIV; /* only where two or more workgroups would share a CU */
    const int64_t per_wave = ((int64_t)N + G * resident - 1) / (G * resident);
    int64_t rows_per_wg = G * per_wave;
    const int64_t cap = (GEMV_X_RED_MAX / (S * 4)) / G * G;
    if (rows_per_wg > cap)
        rows_per_wg = cap;
    const unsigned grid = (unsigned)((N + rows_per_wg - 1) / rows_per_wg);
    size_t lds = (size_t)rows_per_wg * S * 4 * sizeof(float);
    if (G >= 2 && lds < (size_t)K * 2)
        lds = (size_t)K * 2; /* x staging: K <= GEMV_X_STAGE_MAX_K, within GEMV_X_LDS_MAX bytes */
    if (glint_set_lds_limit((const void *)kern, GEMV_X_LDS_MAX) != 0)
        return -3;
    kern<<<grid, threads, lds, st>>>(hole, plug, absmax, (const glint_u32x4 *)x, y, N, K, G, (int)rows_per_wg);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* k_htile_gemv_cu over an M = 1 GEMV (bs 64, K % 2048 == 0, aligned): at S <= 2 slices two
 * 512-thread workgroups per CU, at S > 2 one of up to 1024 threads; a band of
 * ceil(N / workgroups) rows each. Returns 1 where the shape does not fit its plan (the caller
 * then takes k_htile_gemv_xreg), else 0 or -3. */
#ifndef GEMV_CU_ON
#define GEMV_CU_ON 1
#endif
#define GEMV_CU_NARROW_DYN_MAX (7 * 1024) /* two 512-thread workgroups (72 KiB static each) per CU */
template <bool OUT_BF16>
static int htile_launch_gemv_cu(const uint8_t *hole, const uint8_t *plug, const float *absmax, const void *x,
                                void *y, int N, int K, hipStream_t st) {
    if (!GEMV_CU_ON || K % 2048 != 0)
        return 1;
    const int S = K / 2048;
    if (S > GEMV_CU_SMAX)
        return 1;
    const bool narrow = S <= 2;
    const int G = (narrow ? 8 : 16) / S; /* waves per slice */
    const int wgs = glint_cu_count() * (narrow ? 2 : 1);
    const int64_t rows = ((int64_t)N + wgs - 1) / wgs;
    const size_t lds = (size_t)rows * S * 16; /* the row partials */
    if (lds > (narrow ? GEMV_CU_NARROW_DYN_MAX : GEMV_CU_DYN_MAX) || rows * (K / 2) >= ((int64_t)1 << 31))
        return 1;
    const unsigned grid = (unsigned)(((int64_t)N + rows - 1) / rows);
    const int threads = 64 * S * G;
    /* x staging: K / 8 chunks of 16 B over `threads` threads, XC chunks each */
    auto kern = narrow ? k_htile_gemv_cu<OUT_BF16, 1, 512, 512, false>
                       : (G >= 4 ? k_htile_gemv_cu<OUT_BF16, 1, 1024, GEMV_CU_SMAX * 256, true>
                                 : (G >= 2 ? k_htile_gemv_cu<OUT_BF16, 2, 1024, GEMV_CU_SMAX * 256, true>
                                           : k_htile_gemv_cu<OUT_BF16, 4, 1024, GEMV_CU_SMAX * 256, true>));
    if (glint_set_lds_limit((const void *)kern, GEMV_CU_DYN_MAX) != 0)
        return -3;
    kern<<<grid, threads, lds, st>>>(hole, plug, absmax, (const glint_u32x4 *)x, y, N, K, G, (int)rows);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* ------------------------------------ small-M prefill, weights dequantized into registers */
/* k_htile_rd: M <= 64 rows of x (MB = 1, 2 or 4 MFMA row blocks of 16), bs = 64,
 * K % 128 == 0, aligned, BF16 out. The MFMA tiles stage W through LDS and meet at a barrier
 * every 64-wide K step; at small M a step holds too little work to hide that chain. Here
 * each wave owns a strip of 16 W rows and turns its own loads straight into MFMA B operands:
 *   - K runs in W chunks of 128. Lane l loads 16 B of each plane of row l % 16 at chunk
 *     elements [32 (l / 16), +32) and one absmax. Word s of those 16 B is elements [8 s, +8)
 *     of its quarter, which is what v_mfma_f32_16x16x32_bf16 step s wants from the lane when
 *     the K order inside a chunk is permuted so that step s takes elements 32 g + 8 s .. +8
 *     of lane group g. x is read in the same order, so each product is the one the GEMM
 *     defines; only the order of the f32 sums changes.
 *   - KW waves share a strip: x moves in chunks of KW W chunks, and wave kw of the strip
 *     takes W chunk kw of each (its partial sums are added to the others' in kw order at
 *     the end, through LDS). Two waves per SIMD (KW = 2) overlap one wave's dequantization
 *     with the other's MFMAs and loads; with one, the phases of a chunk ran back to back.
 *   - W loads go out in bursts of RD_BURST chunks per wave, two bursts in registers: a load
 *     instruction covers 16 rows x 64 B, and a burst of the KW waves of a strip puts
 *     KW RD_BURST x 64 B of each row in flight together. Read one chunk at a time (all waves
 *     walking K together, 64 B of each 2-KiB row per chunk) these planes streamed at 40% of
 *     HBM; in bursts of 4 chunks per row at 54% (a read-only probe over 14336 x 4096).
 *   - dequantization per element: half a VALU op forms the code byte, one v_perm the lookup
 *     address in the 64-copy cell table, one LDS read, one multiply by the block absmax,
 *     half a v_cvt_pk_bf16_f32 (BF16(cell * absmax), the rounding the other BF16 kernels
 *     apply).
 *   - x chunks (16 MB rows x 256 KW bytes) are loaded three chunks ahead into registers and
 *     written one chunk ahead into an LDS double buffer whose 16-B pieces are XOR-swizzled by
 *     row within each W chunk's 256 bytes (an A fragment read, 16 rows x one piece, hits
 *     distinct banks). One barrier per x chunk, which waits for LDS accesses only.
 *   - a workgroup holds R <= 64 rows, R about N ks / CUs, so one workgroup per CU covers
 *     N (14336 x 4096: 56 rows each, 256 workgroups); K is split ks ways through the split-K
 *     workspace where N alone leaves too few rows per CU (4096 x 14336: 4 ways of 64 rows).
 * Loads past the workgroup's rows, x rows past M and chunk loads past the K range are out of
 * their buffer's range: the hardware drops them and returns zeros. */
#ifndef RD_ON
#define RD_ON 1
#endif
#define RD_STRIPS 4 /* 16-row W strips per workgroup */
#ifndef RD_KW
#define RD_KW 2 /* waves per strip (1: 4-20% slower) */
#endif
#ifndef RD_BURST
#define RD_BURST 2 /* W chunks per load burst of one wave; two bursts in registers (4: 3-8% slower) */
#endif
#define RD_OOR 0x7FFFFF00u /* a buffer offset past every range */
#ifndef RD_W_AUX
#define RD_W_AUX 0 /* cache policy of the weight loads */
#endif

template <int MB, int KW>
__global__ __launch_bounds__(64 * RD_STRIPS * KW, 1) void k_htile_rd(const uint8_t *__restrict__ hole,
                                                                     const uint8_t *__restrict__ plug,
                                                                     const float *__restrict__ absmax,
                                                                     const uint16_t *__restrict__ x,
                                                                     uint16_t *__restrict__ y, int M, int N, int K,
                                                                     int R, int cps, float *__restrict__ part,
                                                                     unsigned *ctr) {
    constexpr int T = 64 * RD_STRIPS * KW;
    constexpr int XROW = 256 * KW;                /* bytes of one x row of an x chunk */
    constexpr int XCH = 16 * MB * XROW;           /* bytes of one x chunk */
    constexpr int NX = XCH / 16 / T;              /* 16-B pieces of an x chunk per thread */
    constexpr int U = 2 * RD_BURST;               /* x chunks per unrolled round */
    static_assert(NX >= 1 && NX * 16 * T == XCH, "x chunk split over the threads");
    static_assert(U % 2 == 0, "two x register stages per round");
    __shared__ float ltab[GLINT_LDS_CELLS64_WORDS];
    __shared__ __attribute__((aligned(16))) uint8_t xb0[XCH], xb1[XCH];
    const int lane = threadIdx.x & 63, m16 = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int strip = w % RD_STRIPS, kw = w / RD_STRIPS;
    const uint32_t lane4 = (uint32_t)(lane & 31) * 4u; /* the half-filled table: copy lane % 32 */
    const int n0 = blockIdx.x * R;
    const int nrows = min(R, N - n0); /* >= 1 */
    const int c0 = blockIdx.z * cps;
    const int nj = min(K >> 7, c0 + cps) - c0;  /* W chunks of the split, >= 1 (the host sizes gridDim.z) */
    const int nxc = (nj + KW - 1) / KW;         /* x chunks */
    const uint32_t rowb = (uint32_t)K >> 1;

    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(hole + (int64_t)n0 * rowb), (short)0, (int)((uint32_t)nrows * rowb), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(plug + (int64_t)n0 * rowb), (short)0, (int)((uint32_t)nrows * rowb), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(absmax + (int64_t)n0 * (K >> 6)), (short)0, (int)((uint32_t)nrows * (rowb >> 3)), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        (void *)x, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), GLINT_BUF_DWORD3);
    const uint32_t wrow = (uint32_t)(16 * strip + m16);
    const uint32_t wofs = wrow * rowb + 16u * (uint32_t)g;
    const uint32_t aofs = (wrow * (uint32_t)(K >> 6) + (uint32_t)(g >> 1)) * 4u;
    /* x piece i of thread t: slot s = t + T i of the chunk (row s / (16 KW), piece
     * s % (16 KW); consecutive threads read one row's contiguous bytes), stored at piece
     * (s % (16 KW)) ^ (row % 16) of its LDS row (the XOR keeps a piece in its W chunk's
     * 256 bytes) */
    uint32_t xgo[NX], xlo[NX];
#pragma unroll
    for (int i = 0; i < NX; ++i) {
        const int sl = (int)threadIdx.x + T * i, r = sl / (16 * KW), pc = sl % (16 * KW);
        xgo[i] = (uint32_t)r * (uint32_t)K * 2u + (uint32_t)(pc << 4);
        xlo[i] = (uint32_t)(r * XROW + ((pc ^ (r & 15)) << 4));
    }

    struct WReg {
        glint_u32x4 h, p;
        float a;
    };
    WReg wr[U];
    glint_u32x4 xr[2][NX];
    /* this wave's W chunk of x chunk X: KW X + kw of the split */
    auto wload = [&](int X, WReg &s) {
        const int j = KW * X + kw;
        const uint32_t c = (uint32_t)(c0 + j);
        const bool in = j < nj;
        const uint32_t o = in ? wofs + c * 64u : RD_OOR, oa = in ? aofs + c * 8u : RD_OOR;
        s.h = __builtin_amdgcn_raw_buffer_load_b128(rh, o, 0, RD_W_AUX);
        s.p = __builtin_amdgcn_raw_buffer_load_b128(rp, o, 0, RD_W_AUX);
        s.a = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ra, oa, 0, RD_W_AUX));
    };
    auto wburst = [&](int X0, int st) {
#pragma unroll
        for (int c = 0; c < RD_BURST; ++c)
            wload(X0 + c, wr[st + c]);
    };
    auto xload = [&](int X, glint_u32x4 (&xs)[NX]) {
        const uint32_t c = (uint32_t)(c0 + KW * X);
        const bool in = X < nxc;
#pragma unroll
        for (int i = 0; i < NX; ++i)
            xs[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, in ? xgo[i] + c * 256u : RD_OOR, 0, 0);
    };
    auto xstore = [&](uint8_t *buf, const glint_u32x4 (&xs)[NX]) {
#pragma unroll
        for (int i = 0; i < NX; ++i)
            *(glint_u32x4 *)(buf + xlo[i]) = xs[i];
    };
    auto dequant = [&](const WReg &s, glint_bf16x8 (&bq)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t E = glint_codes_even(s.h[q], s.p[q]), O = glint_codes_odd(s.h[q], s.p[q]);
            const float f0 = glint_lds_f32(ltab, glint_cell_addr<0>(E, lane4));
            const float f1 = glint_lds_f32(ltab, glint_cell_addr<0>(O, lane4));
            const float f2 = glint_lds_f32(ltab, glint_cell_addr<1>(E, lane4));
            const float f3 = glint_lds_f32(ltab, glint_cell_addr<1>(O, lane4));
            const float f4 = glint_lds_f32(ltab, glint_cell_addr<2>(E, lane4));
            const float f5 = glint_lds_f32(ltab, glint_cell_addr<2>(O, lane4));
            const float f6 = glint_lds_f32(ltab, glint_cell_addr<3>(E, lane4));
            const float f7 = glint_lds_f32(ltab, glint_cell_addr<3>(O, lane4));
            bq[q] = __builtin_bit_cast(glint_bf16x8,
                                       glint_u32x4{glint_cvt_bf16x2(f0 * s.a, f1 * s.a), glint_cvt_bf16x2(f2 * s.a, f3 * s.a),
                                                   glint_cvt_bf16x2(f4 * s.a, f5 * s.a), glint_cvt_bf16x2(f6 * s.a, f7 * s.a)});
        }
    };
    glint_f32x4 acc[MB][1];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
        acc[mb][0] = glint_f32x4{0.f, 0.f, 0.f, 0.f};
    /* A fragments of MFMA step s of this wave's W chunk in an x chunk */
    auto aread = [&](const uint8_t *xs, int s, glint_bf16x8 (&af)[MB]) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
            af[mb] = __builtin_bit_cast(glint_bf16x8, *(const glint_u32x4 *)(xs + (16 * mb + m16) * XROW +
                                                                             (((16 * kw + 4 * g + s) ^ m16) << 4)));
    };
    /* the chunk's 4 MFMA steps, step s + 1's fragments read while step s multiplies */
    auto mma = [&](const uint8_t *xs, const glint_bf16x8 (&bq)[4]) {
        glint_bf16x8 af[2][MB];
        aread(xs, 0, af[0]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s + 1 < 4)
                aread(xs, s + 1, af[(s + 1) & 1]);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                acc[mb][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[s & 1][mb], bq[s], acc[mb][0], 0, 0, 0);
        }
    };
    /* x chunk X (u = X % U) is in LDS buffer u % 2 (written one chunk earlier, published by
     * this barrier, which also ends every read of the other buffer); x chunk X + 1 goes into
     * that buffer from register stage (u + 1) % 2, which then takes x chunk X + 3. The last
     * chunk of a burst refills the burst's stages with the burst after next. */
    /* (Pinning these phases in order with sched_barrier measured 5-13% slower: the compiler's
     * interleaving of one step's MFMAs with the next step's loads and lookups pays.) */
    auto step = [&](int X, int u) {
        __syncthreads();
        xstore((u & 1) ? xb0 : xb1, xr[(u + 1) & 1]);
        xload(X + 3, xr[(u + 1) & 1]);
        glint_bf16x8 bq[4];
        dequant(wr[u], bq);
        if (u % RD_BURST == RD_BURST - 1)
            wburst(X + 1 + RD_BURST, u + 1 - RD_BURST);
        mma((u & 1) ? xb1 : xb0, bq);
    };

    /* the steady state's order of loads from the start (a reordered prologue would leave the
     * first chunks' wait counts short): table (scalar), x chunks 0 and 1, two W bursts, then
     * x chunk 2 into the stage x chunk 0 leaves */
    GlintCellFillHN<(2048 + T - 1) / T> fill;
    glint_cells_fillh_sload(fill);
    __builtin_amdgcn_sched_barrier(0);
    xload(0, xr[0]);
    __builtin_amdgcn_sched_barrier(0);
    xload(1, xr[1]);
    __builtin_amdgcn_sched_barrier(0);
    wburst(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    wburst(RD_BURST, RD_BURST);
    __builtin_amdgcn_sched_barrier(0);
    glint_cells_fillh_sstore(ltab, fill);
    xstore(xb0, xr[0]); /* the first step's barrier publishes the table and x chunk 0 */
    xload(2, xr[0]);
    int X = 0;
    for (; X + U <= nxc; X += U) {
#pragma unroll
        for (int u = 0; u < U; ++u)
            step(X + u, u);
    }
#pragma unroll
    for (int u = 0; u + 1 < U; ++u)
        if (X + u < nxc)
            step(X + u, u);
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0); /* the trailing dropped loads */

    /* the strip's KW partials, added in kw order by wave kw = 0 (the x buffers are free) */
    if constexpr (KW > 1) {
        float *red = (float *)xb0;
        static_assert((KW - 1) * RD_STRIPS * 64 * MB * 4 * 4 <= XCH, "partials fit an x buffer");
        __syncthreads();
        if (kw > 0)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    red[((((kw - 1) * RD_STRIPS + strip) * MB + mb) * 4 + i) * 64 + lane] = acc[mb][0][i];
        __syncthreads();
        if (kw == 0)
#pragma unroll
            for (int k = 1; k < KW; ++k)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[mb][0][i] += red[((((k - 1) * RD_STRIPS + strip) * MB + mb) * 4 + i) * 64 + lane];
        __syncthreads(); /* the split-K epilogue's flag word lives in xb0 */
    }
    if (gridDim.z > 1 && !tile_splitk_epilogue<MB, 1, 64 * RD_STRIPS>(acc, part, ctr, *(unsigned *)xb1,
                                                                       (int)threadIdx.x, kw == 0))
        return;
    const int nl = 16 * strip + m16;
    if (kw == 0 && nl < nrows)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * mb + 4 * g + i;
                if (m < M)
                    y[(int64_t)m * N + n0 + nl] = glint_f32_to_bf16(acc[mb][0][i]);
            }
}

/* k_htile_rl: k_htile_rd (KW = 2) with the weights read as whole 128-B lines. In k_htile_rd
 * a load instruction covers 16 rows x 64 B, half of a 128-B line per row, because lane l must
 * hold row l % 16 for the MFMA; the two waves of a strip each take one half of every line.
 * Here a wave's load instruction covers 8 rows x 128 B (lane l: row 8 kw + l / 8 of the strip,
 * 16-B piece l % 8 of the line that holds both waves' chunks of an x chunk), so the memory
 * requests are whole lines: with the same bytes and the same work, a timing probe of that load
 * form ran the 14336 x 4096 M = 64 launch 12% faster, M = 16 18%.
 *   - The lines go register -> LDS -> register into the MFMA layout, through the upper 128 B
 *     of each 256-B row of the cell table, which the half fill leaves unused (256 rows: 4
 *     strips x 2 buffers x 2 planes x 16 W rows). 16-B pieces are XOR-swizzled by row.
 *   - Line X is loaded 2-3 steps before it is written to LDS (step X - 2, after that step's
 *     barrier) and read back into registers at step X - 1 (after the next barrier); step X
 *     dequantizes it. The absmax of a lane's 64-block comes by its own load, 3 steps ahead.
 *   - x as in k_htile_rd; halves of an x chunk past the split's chunks are not loaded (zeros),
 *     so a non-finite x value there cannot reach another row's sum through a zero weight. */
#ifndef RD_FL
#define RD_FL 1 /* M <= 64: k_htile_rl (0: k_htile_rd) */
#endif
#ifndef RL_STAGES
#define RL_STAGES 4 /* k_htile_rl: W line register stages (6: M = 64 gate 29.5 -> 30.2 us, 8: 31.1; the
                     * prologue's longer first load burst costs more than the deeper lead gains) */
#endif
#ifndef RD_FL_F32
#define RD_FL_F32 1 /* f32 out at M <= 64: k_htile_rl's three-plane form (0: the f32 tiles) */
#endif
/* F32: f32 out (the reference ABI) with the weights w = CELLS * absmax split into three exact
 * BF16 planes (GlintTileProducer::finish_split's rule), each multiplied by x in the MFMA: the
 * products are exact and only the f32 sums differ from a scalar loop's. A step dequantizes
 * and multiplies one MFMA step at a time (3 B operands, 3 MB MFMAs). */
template <int MB, bool F32 = false>
__global__ __launch_bounds__(512, 1) void k_htile_rl(const uint8_t *__restrict__ hole, const uint8_t *__restrict__ plug,
                                                     const float *__restrict__ absmax, const uint16_t *__restrict__ x,
                                                     typename std::conditional<F32, float, uint16_t>::type *__restrict__ y,
                                                     int M, int N, int K, int R, int cps, float *__restrict__ part,
                                                     unsigned *ctr) {
    constexpr int KW = 2, T = 512, STRIPS = 4;
    constexpr int XROW = 256 * KW;      /* bytes of one x row of an x chunk (one W line) */
    constexpr int XCH = 16 * MB * XROW; /* bytes of one x chunk */
    constexpr int NX = XCH / 16 / T;    /* 16-B pieces of an x chunk per thread */
    constexpr int U = RL_STAGES;        /* W line register stages (x chunks per unrolled round) */
    static_assert(U % 2 == 0 && U >= 4, "stages in pairs, lines loaded U - 2 steps ahead of their LDS write");
    static_assert(NX >= 1 && NX * 16 * T == XCH, "x chunk split over the threads");
    __shared__ float ltab[GLINT_LDS_CELLS64_WORDS];
    __shared__ __attribute__((aligned(16))) uint8_t xb0[XCH], xb1[XCH];
    uint8_t *const lt = (uint8_t *)ltab;
    const int lane = threadIdx.x & 63, m16 = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int strip = w % STRIPS, kw = w / STRIPS;
    const uint32_t lane4 = (uint32_t)(lane & 31) * 4u; /* the half-filled table: copy lane % 32 */
    const int n0 = blockIdx.x * R;
    const int nrows = min(R, N - n0); /* >= 1 */
    const int c0 = blockIdx.z * cps;  /* even: the host keeps cps even */
    const int nj = min(K >> 7, c0 + cps) - c0;
    const int nxc = (nj + 1) >> 1; /* x chunks = W lines */
    const uint32_t rowb = (uint32_t)K >> 1;

    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(hole + (int64_t)n0 * rowb), (short)0, (int)((uint32_t)nrows * rowb), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(plug + (int64_t)n0 * rowb), (short)0, (int)((uint32_t)nrows * rowb), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(absmax + (int64_t)n0 * (K >> 6)), (short)0, (int)((uint32_t)nrows * (rowb >> 3)), GLINT_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        (void *)x, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), GLINT_BUF_DWORD3);
    /* the lane's line piece: row lr of the strip, 16-B piece lane % 8 */
    const int lr = 8 * kw + (lane >> 3);
    const uint32_t lofs = (uint32_t)(16 * strip + lr) * rowb + (uint32_t)(lane & 7) * 16u;
    /* the lane's absmax: MFMA row 16 strip + m16, block g / 2 of the wave's chunk */
    const uint32_t aofs = ((uint32_t)(16 * strip + m16) * (uint32_t)(K >> 6) + (uint32_t)(g >> 1)) * 4u;
    /* LDS slots: W row r of plane pl in buffer b of this strip is table row
     * ((strip * 2 + b) * 2 + pl) * 16 + r, bytes 128 .. 255; piece c sits at c ^ (r % 8) */
    const uint32_t put0 = ((uint32_t)((strip * 2) * 2 * 16 + lr) << 8) + 128u +
                          ((uint32_t)((lane & 7) ^ (lr & 7)) << 4);
    const uint32_t get0 = ((uint32_t)((strip * 2) * 2 * 16 + m16) << 8) + 128u +
                          ((uint32_t)((4 * kw + g) ^ (m16 & 7)) << 4);
    constexpr uint32_t BUF = 2 * 16 * 256, PLANE = 16 * 256; /* byte steps of b and pl */
    uint32_t xgo[NX], xlo[NX];
    int xhalf[NX];
#pragma unroll
    for (int i = 0; i < NX; ++i) {
        const int sl = (int)threadIdx.x + T * i, r = sl / (16 * KW), pc = sl % (16 * KW);
        xgo[i] = (uint32_t)r * (uint32_t)K * 2u + (uint32_t)(pc << 4);
        xlo[i] = (uint32_t)(r * XROW + ((pc ^ (r & 15)) << 4));
        xhalf[i] = pc >> 4; /* the W chunk of the line the piece belongs to */
    }

    struct WLine {
        glint_u32x4 h, p;
    };
    WLine wl[U];      /* lines in the load layout */
    WLine wb[2];      /* lines in the MFMA layout (this wave's chunk), from LDS */
    float am[U];      /* absmax of the wave's chunk of x chunk X, stage X % U */
    glint_u32x4 xr[2][NX];
    auto wline = [&](int X, WLine &s) {
        const uint32_t o = 2 * X < nj ? lofs + (uint32_t)(c0 + 2 * X) * 64u : RD_OOR;
        s.h = __builtin_amdgcn_raw_buffer_load_b128(rh, o, 0, 0);
        s.p = __builtin_amdgcn_raw_buffer_load_b128(rp, o, 0, 0);
    };
    auto aload = [&](int X, float &a) {
        const int j = 2 * X + kw;
        a = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(ra, j < nj ? aofs + (uint32_t)(c0 + j) * 8u : RD_OOR, 0, 0));
    };
    auto xload = [&](int X, glint_u32x4 (&xs)[NX]) {
        const uint32_t c = (uint32_t)(c0 + KW * X);
#pragma unroll
        for (int i = 0; i < NX; ++i)
            xs[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, 2 * X + xhalf[i] < nj ? xgo[i] + c * 256u : RD_OOR, 0, 0);
    };
    auto xstore = [&](uint8_t *buf, const glint_u32x4 (&xs)[NX]) {
#pragma unroll
        for (int i = 0; i < NX; ++i)
            *(glint_u32x4 *)(buf + xlo[i]) = xs[i];
    };
    auto wput = [&](int X, const WLine &s) {
        const uint32_t a = put0 + (uint32_t)(X & 1) * BUF;
        *(glint_u32x4 *)(lt + a) = s.h;
        *(glint_u32x4 *)(lt + a + PLANE) = s.p;
    };
    auto wget = [&](int X, WLine &s) {
        const uint32_t a = get0 + (uint32_t)(X & 1) * BUF;
        s.h = *(const glint_u32x4 *)(lt + a);
        s.p = *(const glint_u32x4 *)(lt + a + PLANE);
    };
    auto dequant = [&](const WLine &s, float a, glint_bf16x8 (&bq)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t E = glint_codes_even(s.h[q], s.p[q]), O = glint_codes_odd(s.h[q], s.p[q]);
            const float f0 = glint_lds_f32(ltab, glint_cell_addr<0>(E, lane4));
            const float f1 = glint_lds_f32(ltab, glint_cell_addr<0>(O, lane4));
            const float f2 = glint_lds_f32(ltab, glint_cell_addr<1>(E, lane4));
            const float f3 = glint_lds_f32(ltab, glint_cell_addr<1>(O, lane4));
            const float f4 = glint_lds_f32(ltab, glint_cell_addr<2>(E, lane4));
            const float f5 = glint_lds_f32(ltab, glint_cell_addr<2>(O, lane4));
            const float f6 = glint_lds_f32(ltab, glint_cell_addr<3>(E, lane4));
            const float f7 = glint_lds_f32(ltab, glint_cell_addr<3>(O, lane4));
            bq[q] = __builtin_bit_cast(glint_bf16x8,
                                       glint_u32x4{glint_cvt_bf16x2(f0 * a, f1 * a), glint_cvt_bf16x2(f2 * a, f3 * a),
                                                   glint_cvt_bf16x2(f4 * a, f5 * a), glint_cvt_bf16x2(f6 * a, f7 * a)});
        }
    };
    glint_f32x4 acc[MB][1];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
        acc[mb][0] = glint_f32x4{0.f, 0.f, 0.f, 0.f};
    auto aread = [&](const uint8_t *xs, int s, glint_bf16x8 (&af)[MB]) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
            af[mb] = __builtin_bit_cast(glint_bf16x8, *(const glint_u32x4 *)(xs + (16 * mb + m16) * XROW +
                                                                             (((16 * kw + 4 * g + s) ^ m16) << 4)));
    };
    auto mma = [&](const uint8_t *xs, const glint_bf16x8 (&bq)[4]) {
        glint_bf16x8 af[2][MB];
        aread(xs, 0, af[0]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s + 1 < 4)
                aread(xs, s + 1, af[(s + 1) & 1]);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                acc[mb][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[s & 1][mb], bq[s], acc[mb][0], 0, 0, 0);
        }
    };
    /* F32: MFMA step s's 8 weights of this lane as three BF16 planes (hi, mid, lo: w == hi + mid
     * + lo exactly; an infinite w keeps mid = lo = 0, a NaN w stays NaN in hi) */
    auto split3 = [&](const WLine &s, float a, int q, glint_bf16x8 (&bp)[3]) {
        const uint32_t E = glint_codes_even(s.h[q], s.p[q]), O = glint_codes_odd(s.h[q], s.p[q]);
        float v[8];
        v[0] = glint_lds_f32(ltab, glint_cell_addr<0>(E, lane4));
        v[1] = glint_lds_f32(ltab, glint_cell_addr<0>(O, lane4));
        v[2] = glint_lds_f32(ltab, glint_cell_addr<1>(E, lane4));
        v[3] = glint_lds_f32(ltab, glint_cell_addr<1>(O, lane4));
        v[4] = glint_lds_f32(ltab, glint_cell_addr<2>(E, lane4));
        v[5] = glint_lds_f32(ltab, glint_cell_addr<2>(O, lane4));
        v[6] = glint_lds_f32(ltab, glint_cell_addr<3>(E, lane4));
        v[7] = glint_lds_f32(ltab, glint_cell_addr<3>(O, lane4));
        const bool big = !(__builtin_fabsf(a) < 0x1p126f); /* only there can w be infinite */
        uint32_t hi[8], mid[8], lo[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float w = v[i] * a;
            const float h = __uint_as_float(__float_as_uint(w) & 0xFFFF0000u);
            float r1 = w - h;
            if (big)
                r1 = __builtin_isinf(w) ? 0.0f : r1;
            const float md = __uint_as_float(__float_as_uint(r1) & 0xFFFF0000u);
            hi[i] = __float_as_uint(h);
            mid[i] = __float_as_uint(md);
            lo[i] = __float_as_uint(r1 - md);
        }
        uint32_t ph[4], pm[4], pl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ph[j] = __builtin_amdgcn_perm(hi[2 * j + 1], hi[2 * j], 0x07060302u);
            pm[j] = __builtin_amdgcn_perm(mid[2 * j + 1], mid[2 * j], 0x07060302u);
            pl[j] = __builtin_amdgcn_perm(lo[2 * j + 1], lo[2 * j], 0x07060302u);
        }
        bp[0] = __builtin_bit_cast(glint_bf16x8, glint_u32x4{ph[0], ph[1], ph[2], ph[3]});
        bp[1] = __builtin_bit_cast(glint_bf16x8, glint_u32x4{pm[0], pm[1], pm[2], pm[3]});
        bp[2] = __builtin_bit_cast(glint_bf16x8, glint_u32x4{pl[0], pl[1], pl[2], pl[3]});
    };
    auto mma3 = [&](const uint8_t *xs, const WLine &s, float a) {
        glint_bf16x8 af[2][MB];
        aread(xs, 0, af[0]);
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            glint_bf16x8 bp[3];
            split3(s, a, st, bp);
            if (st + 1 < 4)
                aread(xs, st + 1, af[(st + 1) & 1]);
#pragma unroll
            for (int pl = 0; pl < 3; ++pl)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[mb][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[st & 1][mb], bp[pl], acc[mb][0], 0, 0, 0);
        }
    };
    /* step X (u = X % U): x chunk X + 1 into LDS, x chunk X + 3 and the absmax of X + 3
     * issued, line X + 2 into LDS, line X + 1 out of LDS, line X dequantized and multiplied;
     * on even steps lines X + 4 and X + 5 go out into the stages lines X and X + 1 left */
    auto step = [&](int X, int u) {
        __syncthreads();
        xstore((u & 1) ? xb0 : xb1, xr[(u + 1) & 1]);
        xload(X + 3, xr[(u + 1) & 1]);
        aload(X + 3, am[(u + 3) % U]);
        wput(X + 2, wl[(u + 2) % U]);
        wget(X + 1, wb[(u + 1) & 1]);
        if constexpr (F32) {
            if ((u & 1) == 0) {
                wline(X + U, wl[u]);
                wline(X + U + 1, wl[u + 1]);
            }
            mma3((u & 1) ? xb1 : xb0, wb[u & 1], am[u]);
        } else {
            glint_bf16x8 bq[4];
            dequant(wb[u & 1], am[u], bq);
            if ((u & 1) == 0) {
                wline(X + U, wl[u]);
                wline(X + U + 1, wl[u + 1]);
            }
            mma((u & 1) ? xb1 : xb0, bq);
        }
    };

    GlintCellFillHN<(2048 + T - 1) / T> fill;
    glint_cells_fillh_sload(fill);
    __builtin_amdgcn_sched_barrier(0);
    xload(0, xr[0]);
    __builtin_amdgcn_sched_barrier(0);
    xload(1, xr[1]);
    aload(0, am[0]);
    aload(1, am[1]);
    aload(2, am[2]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < U; ++s)
        wline(s, wl[s]);
    __builtin_amdgcn_sched_barrier(0);
    glint_cells_fillh_sstore(ltab, fill);
    xstore(xb0, xr[0]);
    xload(2, xr[0]);
    wput(0, wl[0]);
    wput(1, wl[1]);
    __syncthreads();
    wget(0, wb[0]);
    int X = 0;
    for (; X + U <= nxc; X += U) {
#pragma unroll
        for (int u = 0; u < U; ++u)
            step(X + u, u);
    }
#pragma unroll
    for (int u = 0; u + 1 < U; ++u)
        if (X + u < nxc)
            step(X + u, u);
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0); /* the trailing dropped loads */

    /* the strip's two partials, added in kw order by wave kw = 0 (the x buffers are free) */
    float *red = (float *)xb0;
    static_assert(STRIPS * 64 * MB * 4 * 4 <= XCH, "partials fit an x buffer");
    __syncthreads();
    if (kw > 0)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                red[((strip * MB + mb) * 4 + i) * 64 + lane] = acc[mb][0][i];
    __syncthreads();
    if (kw == 0)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[mb][0][i] += red[((strip * MB + mb) * 4 + i) * 64 + lane];
    __syncthreads(); /* the split-K epilogue's flag word lives in xb0 */
    if (gridDim.z > 1 && !tile_splitk_epilogue<MB, 1, 64 * STRIPS>(acc, part, ctr, *(unsigned *)xb1,
                                                                    (int)threadIdx.x, kw == 0))
        return;
    const int nl = 16 * strip + m16;
    if (kw == 0 && nl < nrows)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * mb + 4 * g + i;
                if (m < M) {
                    if constexpr (F32)
                        y[(int64_t)m * N + n0 + nl] = acc[mb][0][i];
                    else
                        y[(int64_t)m * N + n0 + nl] = glint_f32_to_bf16(acc[mb][0][i]);
                }
            }
}

/* k_htile_rl (k_htile_rd) over an M <= 64 prefill, BF16 out, or f32 out (F32: k_htile_rl
 * only). Returns 1 where the shape does not fit (K % 128 != 0, offsets beyond 31 bits; the
 * caller takes the LDS tiles), -5 where a `fixed` workspace is too small for the split plan,
 * else 0 or -3. */
template <int MB, bool F32>
static int htile_launch_rd_mb(const uint8_t *hole, const uint8_t *plug, const float *absmax, const uint16_t *x,
                              void *y, int M, int N, int K, hipStream_t st, const GlintSplitWs *fixed) {
    const int cus = glint_cu_count(), nc = K >> 7;
    constexpr int RMAX = 16 * RD_STRIPS, TILE_FLOATS = MB * 4 * 64 * RD_STRIPS;
    auto plan = [&](int ks, int &cps, int &R, unsigned &gx) {
        cps = (nc + ks - 1) / ks;
        if (RD_FL)
            cps = (cps + 1) & ~1; /* k_htile_rl: splits start on a W line */
        ks = (nc + cps - 1) / cps;
        R = (int)std::min<int64_t>(RMAX, (((int64_t)N * ks + cus - 1) / cus + 7) / 8 * 8);
        gx = (unsigned)((N + R - 1) / R);
        return ks;
    };
    int cps, R;
    unsigned gx;
    int ks = plan(std::max(1, std::min(std::min(TILE_SPLIT_MAX, nc), (int)((int64_t)cus * RMAX / N))), cps, R, gx);
    GlintSplitWs ws{nullptr, nullptr, 0, 0};
    if (ks > 1) {
        const bool got = fixed ? (ws = *fixed, true) : glint_split_ws_stream(st, ws);
        const bool fits = got && (size_t)ks * gx * TILE_FLOATS <= ws.part_floats && (size_t)gx <= ws.nctr;
        if (!fits) {
            if (fixed)
                return -5;
            ks = plan(1, cps, R, gx); /* no workspace (a capture without one): unsplit */
            ws = GlintSplitWs{nullptr, nullptr, 0, 0};
        }
    }
    if (F32)
        k_htile_rl<MB, true><<<dim3(gx, 1, (unsigned)ks), 512, 0, st>>>(hole, plug, absmax, x, (float *)y, M, N, K, R,
                                                                      cps, ws.part, ws.ctr);
    else if (RD_FL)
        k_htile_rl<MB><<<dim3(gx, 1, (unsigned)ks), 512, 0, st>>>(hole, plug, absmax, x, (uint16_t *)y, M, N, K, R, cps,
                                                                ws.part, ws.ctr);
    else
        k_htile_rd<MB, RD_KW><<<dim3(gx, 1, (unsigned)ks), 64 * RD_STRIPS * RD_KW, 0, st>>>(
            hole, plug, absmax, x, (uint16_t *)y, M, N, K, R, cps, ws.part, ws.ctr);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
template <bool F32 = false>
static int htile_launch_rd(const uint8_t *hole, const uint8_t *plug, const float *absmax, const void *x, void *y,
                           int M, int N, int K, hipStream_t st, const GlintSplitWs *fixed) {
    if (!RD_ON || (F32 && !RD_FL_F32) || M < 1 || M > 64 || K % 128 != 0 || (int64_t)M * K * 2 >= (int64_t)RD_OOR ||
        (int64_t)16 * RD_STRIPS * (K / 2) >= (int64_t)RD_OOR)
        return 1;
    const uint16_t *xb = (const uint16_t *)x;
    if (M <= 16)
        return htile_launch_rd_mb<1, F32>(hole, plug, absmax, xb, y, M, N, K, st, fixed);
    if (M <= 32)
        return htile_launch_rd_mb<2, F32>(hole, plug, absmax, xb, y, M, N, K, st, fixed);
    return htile_launch_rd_mb<4, F32>(hole, plug, absmax, xb, y, M, N, K, st, fixed);
}

/* f32 output at M > 1 (the reference ABI's prefill use): 3-plane k_tile_mfma, whose
 * products are exact and whose sums are f32. 128 x 128 tiles over 8 waves (2 x 4, wave tile
 * 64 x 32) fill the 160 KiB of LDS: x 32 KiB, three W planes 96 KiB, cell table 32 KiB;
 * below 128 rows 64 x 128 tiles (8 waves in a row, wave tile 64 x 16), or 64 x 64 over 4
 * waves where those would leave CUs idle (4096 x 14336 at M = 64: 78.5 -> 61.6 us). */
#define F32_TILE_MIN_M 128
#ifndef F32_BN64
#define F32_BN64 1
#endif

/* `fixed`: the caller's split-K workspace (the no-allocation entry point); null for the
 * stream's own. Returns 0, -1 null pointer, -2 bs <= 0, -3 launch error, -5 the split plan
 * needs more than the fixed workspace holds. K < 1 writes zeros (the empty sum). */
/* y[0 .. n) = 0 (words of 16 or 32 bits): the K <= 0 result. A kernel, not a memset, so
 * it can be recorded into a graph. */
template <typename T>
__global__ __launch_bounds__(256) void k_htile_zero(T *__restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        y[i] = (T)0;
}

template <bool OUT_BF16>
static int htile_launch(const uint8_t *hole, const uint8_t *plug, const float *absmax, const void *x, void *y, int M,
                        int N, int K, int bs, hipStream_t st, const GlintSplitWs *fixed = nullptr) {
    if (!hole || !plug || !absmax || !x || !y)
        return -1;
    if (bs <= 0)
        return -2;
    if (M <= 0 || N <= 0)
        return 0;
    if (K < 1) {
        /* no k term: every output is the empty sum, 0, as the reference's k loop runs no
         * iteration and stores its zero accumulators (cuda/glint_htile.cu:141-163) */
        const int64_t n = (int64_t)M * N;
        const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 4096);
        if (OUT_BF16)
            k_htile_zero<uint16_t><<<grid, 256, 0, st>>>((uint16_t *)y, n);
        else
            k_htile_zero<float><<<grid, 256, 0, st>>>((float *)y, n);
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    const bool fast_ok = bs == 64 && (K % 64) == 0 && glint_aligned(hole, 16) && glint_aligned(plug, 16) &&
                         glint_aligned(absmax, 4) && glint_aligned(x, 16);
    /* M = 1: the x-register GEMV (K <= 32768), else the tiles; M > 1: the small-M GEMV or
     * the tiles */
    const bool gemv_x_ok = M == 1 && fast_ok && (K / GEMV_X_EL + 63) / 64 <= GEMV_X_S_MAX;
    const bool mfma_ok = fast_ok && !gemv_x_ok;
    /* BF16 out above GEMV_MR_RL rows: k_htile_rl first (14336 x 4096 M = 5 .. 8: 18.0-19.2 us
     * against 22.5-23.8 for the 8-row small-M GEMV; 4096 x 14336 18.3-18.4 against 24.8-25.0),
     * the small-M GEMV where that does not take the shape */
    const bool rl_first = M > (OUT_BF16 ? GEMV_MR_RL : GEMV_MR_RL_F32);
    if (mfma_ok && GEMV_MR_ON && !rl_first && gemv_mr_takes(M, K, !OUT_BF16))
        return htile_launch_gemv_mr<!OUT_BF16>(hole, plug, absmax, x, y, M, N, K, st);
    /* f32 out from GEMV_MR_RL_F32 + 1 rows: k_htile_rl's three-plane form (14336 x 4096 M = 8
     * 31.3 -> 30.1 us, 16 49.7 -> 30.2, 32 49.9 -> 33.9, 64 50.3 -> 41.4; 4096 x 14336 M = 8
     * 33.6 -> 29.2, 64 61.8 -> 39.8, against the two small-M launches and the f32 tiles; at
     * M = 5 the two launches were faster, 30.6 against 31.5) */
    if (!OUT_BF16 && mfma_ok && M > GEMV_MR_RL_F32 && M <= 64) {
        const int rc = htile_launch_rd<true>(hole, plug, absmax, x, y, M, N, K, st, fixed);
        if (rc != 1)
            return rc;
    }
    if (!OUT_BF16 && mfma_ok && GEMV_MR_ON && GEMV_MR_F32_TWICE && M > GEMV_MR_MAX_F32 && M <= 2 * GEMV_MR_MAX_F32 &&
        gemv_mr_takes(GEMV_MR_MAX_F32, K, true)) {
        /* f32 out at M = 5 .. 8: the 4-row form twice (the weights are read twice), rows 4 ..
         * M - 1 by the small-M form or, for one row, the M = 1 GEMV; the same f32 arithmetic
         * per row as one launch would have */
        const int rc = htile_launch_gemv_mr<true>(hole, plug, absmax, x, y, GEMV_MR_MAX_F32, N, K, st);
        if (rc != 0)
            return rc;
        const int M2 = M - GEMV_MR_MAX_F32;
        const uint16_t *x2 = (const uint16_t *)x + (int64_t)GEMV_MR_MAX_F32 * K;
        float *y2 = (float *)y + (int64_t)GEMV_MR_MAX_F32 * N;
        return M2 >= 2 ? htile_launch_gemv_mr<true>(hole, plug, absmax, x2, y2, M2, N, K, st)
                       : htile_launch_gemv_xreg<false>(hole, plug, absmax, x2, y2, N, K, st);
    }
    if (gemv_x_ok) {
        const int rc = htile_launch_gemv_cu<OUT_BF16>(hole, plug, absmax, x, y, N, K, st);
        return rc != 1 ? rc : htile_launch_gemv_xreg<OUT_BF16>(hole, plug, absmax, x, y, N, K, st);
    }
    if (mfma_ok && OUT_BF16) {
        const GlintTileProducer p{(const glint_u32x2 *)hole, (const glint_u32x2 *)plug, absmax, N, K, nullptr};
        const uint16_t *xb = (const uint16_t *)x;
        uint16_t *yb = (uint16_t *)y;
        bool planned;
        if (M <= 64) {
            const int rc = htile_launch_rd(hole, plug, absmax, x, y, M, N, K, st, fixed);
            if (rc != 1)
                return rc;
        }
        if (rl_first && GEMV_MR_ON && gemv_mr_takes(M, K, false))
            return htile_launch_gemv_mr<false>(hole, plug, absmax, x, y, M, N, K, st);
        if (M <= 64)
            planned = TILE_SS_BN32
                          ? tile_ss_launch<64, 32, TILE_RX, GlintTileProducer, TileOutBF16>(p, xb, yb, M, N, K, st, 2, fixed)
                          : tile_ss_launch<64, 64, TILE_RX, GlintTileProducer, TileOutBF16>(p, xb, yb, M, N, K, st, 1, fixed);
        else if (M < MF2_MIN_M)
            planned = tile_ss_launch<128, 64, TILE_RX, GlintTileProducer, TileOutBF16>(p, xb, yb, M, N, K, st, 1, fixed);
        else if (TILE_BIG && TILE_SK && tile_big_fits(M, N, K) && tile_sk_pays(M, N, K) &&
                 tile_big_sk_launch<TILE_R_BIG, GlintTileProducer, TileOutBF16>(p, xb, yb, M, N, K, st, fixed))
            planned = true;
        else if (TILE_BIG && tile_big_fits(M, N, K) && tile_big_pays(M, N))
            planned = tile_big_launch<TILE_R_BIG, GlintTileProducer, TileOutBF16>(p, xb, yb, M, N, K, st, fixed);
        else if (TILE_BIG && tile_big_fits(M, N, K) && tile_big_split_fills(M, N, K) &&
                 tile_big_split_launch<TILE_R_BIG, GlintTileProducer, TileOutBF16>(p, xb, yb, M, N, K, st, fixed))
            planned = true;
        else
            planned = tile_mfma_launch<MF2_BM, MF2_BN, 4, 2, TILE_R_BIG, GlintTileProducer, TileOutBF16>(p, xb, yb, M, N,
                                                                                                       K, st, fixed);
        if (!planned)
            return -5;
    } else if (mfma_ok) {
        const GlintTileProducer p{(const glint_u32x2 *)hole, (const glint_u32x2 *)plug, absmax, N, K, nullptr};
        const uint16_t *xb = (const uint16_t *)x;
        float *yf = (float *)y;
        /* below 128 rows, 64 x 64 tiles (4 waves) where the 64 x 128 ones, split K ways at most
         * TILE_SPLIT_MAX, would leave CUs idle (the 4096-row down projection) */
        const int64_t tiles128 = (int64_t)((N + 127) / 128) * ((M + 63) / 64);
        const bool narrow = F32_BN64 && tiles128 * TILE_SPLIT_MAX < glint_cu_count();
        const bool planned =
            M < F32_TILE_MIN_M
                ? (narrow ? tile_mfma_launch<64, 64, 1, 4, 2, GlintTileProducer, TileOutF32, 3>(p, xb, yf, M, N, K, st, fixed)
                          : tile_mfma_launch<64, 128, 1, 8, 2, GlintTileProducer, TileOutF32, 3>(p, xb, yf, M, N, K, st,
                                                                                                  fixed))
                : tile_mfma_launch<128, 128, 2, 4, 2, GlintTileProducer, TileOutF32, 3>(p, xb, yf, M, N, K, st, fixed);
        if (!planned)
            return -5;
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

GLINT_API int glint_htile_workspace_reserve(struct ihipStream_t *stream) {
    GlintSplitWs ws;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
        return -1;
    return glint_split_ws_stream((hipStream_t)stream, ws) ? 0 : -1;
}

GLINT_API int glint_htile_workspace_release(struct ihipStream_t *stream) {
    return glint_split_ws_release((hipStream_t)stream);
}

/* Library-internal (not exported): the stream's split-K workspace if it already has one,
 * for the K-major kernels' slice reductions; never allocates (one workspace cache per
 * library). */
bool glint_stream_workspace(hipStream_t st, GlintSplitWs *ws) { return glint_split_ws_stream(st, *ws, false); }

/* Library-internal (not exported): the BF16-out launch with the caller's split-K
 * workspace in place of the stream's own. Used by the no-allocation entry point. */
int glint_htile_bf16_launch_ws(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax, const void *d_x,
                               uint16_t *d_y, int M, int N, int K, int bs, hipStream_t st, const GlintSplitWs *ws) {
    return htile_launch<true>(d_hole, d_plug, d_absmax, d_x, d_y, M, N, K, bs, st, ws);
}
