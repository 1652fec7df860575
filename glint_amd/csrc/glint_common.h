/* Shared device and host helpers for the GLINT HIP kernels (gfx950 / CDNA4). */
#ifndef GLINT_COMMON_H_
#define GLINT_COMMON_H_

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#define GLINT_API extern "C" __attribute__((visibility("default")))

/* ------------------------------------------------------------------ tables */

/* Encode bucket table (see glint_codebook.h): code = base + (v > thr). */
struct GlintCodeEntry {
    uint32_t thr; /* f32 bits; +inf when no threshold falls inside the bucket */
    uint32_t base;
};

/* LDS layout of the 256-entry f32 cell table: 32 copies, copy j entirely in LDS
 * bank j, so the lookup of lane l (copy l % 32) never conflicts with another lane's
 * in the same 32-lane half of a ds_read_b32. Index of code c for lane l:
 * (c << 5) | (l & 31). 32 KiB. */
#define GLINT_LDS_CELLS_WORDS (256 * 32)

#include "glint_cells.h"
/* Device copy of GLINT_CELLS (one per translation unit). */
static __constant__ float kCells[16][16] = GLINT_CELLS_INIT;

/* Fill the bank-private table. `stage` is 256 floats of LDS scratch. Must be called by
 * every thread of the block (contains barriers); blockDim.x must divide 8192. */
__device__ __forceinline__ void glint_fill_cells_lds(float *ltab, float *stage) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x)
        stage[i] = (&kCells[0][0])[i];
    __syncthreads();
    /* word i holds cell i >> 5: consecutive threads write consecutive words (no
     * conflicts) and read one broadcast value per 32 threads */
    for (int i = threadIdx.x; i < GLINT_LDS_CELLS_WORDS; i += blockDim.x)
        ltab[i] = stage[i >> 5];
    __syncthreads();
}

/* ------------------------------------------------------------- device helpers */
typedef uint32_t glint_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t glint_u32x2 __attribute__((ext_vector_type(2)));
typedef float glint_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float glint_bf16lo(uint32_t d) { return __uint_as_float(d << 16); }
__device__ __forceinline__ float glint_bf16hi(uint32_t d) { return __uint_as_float(d & 0xFFFF0000u); }

/* BF16 bits of f, round to nearest even, before the NaN rule: the upper half of the
 * returned word is the BF16 pattern (glint_np.py:25-31 without its NaN branch). */
__device__ __forceinline__ uint32_t glint_rne_hi(float f) {
    const uint32_t u = __float_as_uint(f);
    return u + 0x7FFFu + ((u >> 16) & 1u);
}
/* Full reference rule, NaN -> (u >> 16) | 0x40. */
__device__ __forceinline__ uint16_t glint_f32_to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    if (f != f)
        return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)(glint_rne_hi(f) >> 16);
}
/* Two BF16 (RNE, non-NaN inputs) packed lo | hi << 16. */
__device__ __forceinline__ uint32_t glint_pack_bf16x2(float lo, float hi) {
    return __builtin_amdgcn_perm(glint_rne_hi(hi), glint_rne_hi(lo), 0x07060302u);
}

/* DPP lane moves (gfx9 encodings). */
#define GLINT_DPP_QUAD_1032 0xB1  /* quad_perm [1,0,3,2] */
#define GLINT_DPP_QUAD_2301 0x4E  /* quad_perm [2,3,0,1] */
#define GLINT_DPP_ROW_HALF_MIRROR 0x141
#define GLINT_DPP_ROW_MIRROR 0x140

template <int CTRL>
__device__ __forceinline__ int glint_dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

/* Max over each aligned group of 8 lanes (non-negative ints). */
__device__ __forceinline__ int glint_max8(int v) {
    v = max(v, glint_dpp<GLINT_DPP_QUAD_1032>(v));
    v = max(v, glint_dpp<GLINT_DPP_QUAD_2301>(v));
    v = max(v, glint_dpp<GLINT_DPP_ROW_HALF_MIRROR>(v));
    return v;
}

/* Sum over the 64 lanes of a wave; every lane gets the total. */
__device__ __forceinline__ float glint_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float glint_wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

/* ------------------------------------------------------------- host helpers */
static inline bool glint_aligned(const void *p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

#endif
