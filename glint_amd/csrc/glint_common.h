/* Shared device and host helpers for the GLINT HIP kernels (gfx950 / CDNA4). */
#ifndef GLINT_COMMON_H_
#define GLINT_COMMON_H_

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

/* s_waitcnt immediate for vmcnt(0) alone (gfx9 encoding: vmcnt [3:0] and [15:14] = 0,
 * expcnt [6:4] and lgkmcnt [11:8] at their maxima). On gfx9 stores count in vmcnt too. */
#define GLINT_WAIT_VMCNT0 0x0F70
/* s_waitcnt immediate for vmcnt(n) alone, n < 64 */
#define GLINT_WAIT_VMCNT(n) (0x0F70 | ((n) & 15) | ((((n) >> 4) & 3) << 14))
/* s_waitcnt immediate for vmcnt(n) and lgkmcnt(0), n < 64 */
#define GLINT_WAIT_VMCNT_LGKM0(n) (0x0070 | ((n) & 15) | ((((n) >> 4) & 3) << 14))
/* dword 3 of a raw buffer resource on gfx9-family parts: 32-bit data format, no swizzle */
#define GLINT_BUF_DWORD3 0x00020000

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

typedef float glint_f32x4 __attribute__((ext_vector_type(4)));
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

/* The same 32-copy table, filled straight from the constant table with 16-B stores:
 * thread t writes runs r = t, t + blockDim.x, ... of 4 words; run r holds 4 copies of cell
 * r / 8. A thread's loads all go out before its stores. Ends with a barrier. */
__device__ __forceinline__ void glint_fill_cells_lds_direct(float *ltab) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    constexpr int RUNS = GLINT_LDS_CELLS_WORDS / 4;
    if (blockDim.x == 256) {
        float v[RUNS / 256];
#pragma unroll
        for (int k = 0; k < RUNS / 256; ++k)
            v[k] = (&kCells[0][0])[((int)threadIdx.x + 256 * k) >> 3];
#pragma unroll
        for (int k = 0; k < RUNS / 256; ++k)
            ((f32x4 *)ltab)[threadIdx.x + 256 * k] = f32x4{v[k], v[k], v[k], v[k]};
    } else {
        for (int r = threadIdx.x; r < RUNS; r += blockDim.x) {
            const float v = (&kCells[0][0])[r >> 3];
            ((f32x4 *)ltab)[r] = f32x4{v, v, v, v};
        }
    }
    __syncthreads();
}

/* 64-copy layout for the streaming kernels: word (c << 6) | lane, i.e. byte address
 * c * 256 + lane * 4 (64 KiB). Every lane reads its own copy, each copy lives in one
 * bank, and the byte address of code byte k of a word E is one v_perm_b32 that drops
 * E's byte k into address byte 1 next to the lane's byte lane*4. */
#define GLINT_LDS_CELLS64_WORDS (256 * 64)

__device__ __forceinline__ void glint_fill_cells_lds64(float *ltab, float *stage) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x)
        stage[i] = (&kCells[0][0])[i];
    __syncthreads();
    for (int i = threadIdx.x; i < GLINT_LDS_CELLS64_WORDS; i += blockDim.x)
        ltab[i] = stage[i >> 6];
    __syncthreads();
}

/* Same table, filled straight from the constant table: thread t writes the 16-B runs
 * [16 w4, 16 w4 + 16) for w4 = t, t + blockDim.x, ...; a run holds 4 copies of cell
 * w4 / 16. Ends with a barrier. */
__device__ __forceinline__ void glint_fill_cells_lds64_direct(float *ltab) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    for (int w4 = threadIdx.x; w4 < GLINT_LDS_CELLS64_WORDS / 4; w4 += blockDim.x) {
        const float v = (&kCells[0][0])[w4 >> 4];
        ((f32x4 *)ltab)[w4] = f32x4{v, v, v, v};
    }
    __syncthreads();
}

/* The same fill split in two so it can be overlapped with a kernel's first loads: the
 * cell values go out first (issue order is wait order for vector loads), the LDS writes
 * come after the kernel has issued its own loads. 8 runs per thread cover the table for
 * blockDim >= 512; a loop covers smaller blocks. The caller issues the barrier. */
struct GlintCellFill {
    float v[8];
    int run[8];
};
__device__ __forceinline__ void glint_cells_fill_load(GlintCellFill &f) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        f.run[k] = min((int)threadIdx.x + k * (int)blockDim.x, GLINT_LDS_CELLS64_WORDS / 4 - 1);
        f.v[k] = (&kCells[0][0])[f.run[k] >> 4];
    }
}
__device__ __forceinline__ void glint_cells_fill_store(float *ltab, const GlintCellFill &f) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int k = 0; k < 8; ++k) /* clamped runs rewrite the last run with its own value */
        ((f32x4 *)ltab)[f.run[k]] = f32x4{f.v[k], f.v[k], f.v[k], f.v[k]};
    for (int r = threadIdx.x + 8 * blockDim.x; r < GLINT_LDS_CELLS64_WORDS / 4; r += blockDim.x) {
        const float v = (&kCells[0][0])[r >> 4];
        ((f32x4 *)ltab)[r] = f32x4{v, v, v, v};
    }
}

/* Half fill: lanes l and l + 32 share copy l % 32, so only copies 0 .. 31
 * of each cell are written: 2048 runs of 16 B instead of 4096 (the fill's LDS writes were
 * 0.5-0.8 us of the 14336 x 4096 launch). A lookup address stays one v_perm (lane4 =
 * (lane % 32) * 4); two lanes of a ds_read then share a bank. Run u (0 .. 2047) is run
 * (u / 8) * 16 + u % 8 of the 64-copy layout; thread t takes u = t + k blockDim.x, so a
 * wave's 64 runs of step k hold 8 consecutive cells: two s_load_dwordx4 per step.
 * 14336 x 4096: 12.30-12.59 -> 11.87-11.95 us. A 16-copy form was slower (12.8 us), and so
 * was a generic form of this fill (12.3 us): keep the prologue's code as it is. */
#define GLINT_FILLH_STEPS 5 /* covers 2048 runs for blockDim.x >= 410 */
/* STEPS scalar steps cover the table for blockDim.x >= 2048 / STEPS (8 for 256 threads, so no
 * vector load of the table and no wait for the kernel's own first loads is needed) */
template <int STEPS>
struct GlintCellFillHN {
    glint_f32x4 c[STEPS][2];
};
typedef GlintCellFillHN<GLINT_FILLH_STEPS> GlintCellFillH;
template <int STEPS>
__device__ __forceinline__ void glint_cells_fillh_sload(GlintCellFillHN<STEPS> &f) {
    const int wbase = __builtin_amdgcn_readfirstlane((int)threadIdx.x & ~63);
#pragma unroll
    for (int k = 0; k < STEPS; ++k) {
        const int c0 = min((wbase + k * (int)blockDim.x) >> 3, 248);
        f.c[k][0] = *(const glint_f32x4 *)(&kCells[0][0] + c0);
        f.c[k][1] = *(const glint_f32x4 *)(&kCells[0][0] + c0 + 4);
    }
}
template <int STEPS>
__device__ __forceinline__ void glint_cells_fillh_sstore(float *ltab, const GlintCellFillHN<STEPS> &f) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63, ci = lane >> 3; /* cell c0 + ci (blockDim.x % 64 == 0) */
#pragma unroll
    for (int k = 0; k < STEPS; ++k) {
        const int u = (int)threadIdx.x + k * (int)blockDim.x;
        const glint_f32x4 lo = f.c[k][0], hi = f.c[k][1];
        const float vl = (ci & 2) ? ((ci & 1) ? lo.w : lo.z) : ((ci & 1) ? lo.y : lo.x);
        const float vh = (ci & 2) ? ((ci & 1) ? hi.w : hi.z) : ((ci & 1) ? hi.y : hi.x);
        const float v = (ci & 4) ? vh : vl;
        if (u < 2048)
            ((f32x4 *)ltab)[(u >> 3) * 16 + (u & 7)] = f32x4{v, v, v, v};
    }
    for (int u = threadIdx.x + STEPS * blockDim.x; u < 2048; u += blockDim.x) {
        const float v = (&kCells[0][0])[u >> 3];
        ((f32x4 *)ltab)[(u >> 3) * 16 + (u & 7)] = f32x4{v, v, v, v};
    }
}
/* Byte address of code byte K of E for the lane whose lane*4 is `lane4` (in byte 0). */
template <int K>
__device__ __forceinline__ uint32_t glint_cell_addr(uint32_t E, uint32_t lane4) {
    return __builtin_amdgcn_perm(E, lane4, 0x0C0C0000u | ((4u + K) << 8));
}
__device__ __forceinline__ float glint_lds_f32(const float *base, uint32_t byte_addr) {
    return *(const float *)((const char *)base + byte_addr);
}

/* Code bytes of 4 consecutive element pairs: byte j of the even word is element 2j's
 * code (hole << 4 | plug), byte j of the odd word element 2j+1's. */
__device__ __forceinline__ uint32_t glint_codes_even(uint32_t H, uint32_t P) {
    return ((H << 4) & 0xF0F0F0F0u) | (P & 0x0F0F0F0Fu);
}
__device__ __forceinline__ uint32_t glint_codes_odd(uint32_t H, uint32_t P) {
    return (H & 0xF0F0F0F0u) | ((P >> 4) & 0x0F0F0F0Fu);
}

/* A split-K workspace (tile_mfma.h): f32 partials plus one arrival counter per output
 * tile, counters zero between launches. */
struct GlintSplitWs {
    float *part;
    unsigned *ctr;
    size_t part_floats, nctr; /* capacities */
};

/* ------------------------------------------------------------- device helpers */
typedef uint32_t glint_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t glint_u32x2 __attribute__((ext_vector_type(2)));

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

/* v + (v of the lane CTRL names), as one v_add_f32 with a DPP source: every lane these
 * controls name is inside the row, so the old value 0 is never used */
template <int CTRL>
__device__ __forceinline__ float glint_add_dpp(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

/* Sum over each row of 16 lanes, left in every lane of the row (DPP only, no LDS). */
__device__ __forceinline__ float glint_row16_sum(float v) {
    v = glint_add_dpp<GLINT_DPP_QUAD_1032>(v);
    v = glint_add_dpp<GLINT_DPP_QUAD_2301>(v);
    v = glint_add_dpp<GLINT_DPP_ROW_HALF_MIRROR>(v);
    v = glint_add_dpp<GLINT_DPP_ROW_MIRROR>(v);
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
#include <mutex>

static inline bool glint_aligned(const void *p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

/* Workgroups of `kernel` (block size `threads`, `dyn_lds` bytes of dynamic LDS) that fit
 * on one CU at once; 1 if the runtime cannot say. Sizes persistent grids. */
static inline int glint_resident_blocks(const void *kernel, int threads, size_t dyn_lds = 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, dyn_lds) != hipSuccess || n < 1)
        n = 1;
    return n;
}

/* Workgroups of `kernel` resident on the whole current device (CUs x occupancy), computed
 * once per (kernel, device, block size, dynamic LDS): the occupancy query costs
 * microseconds, which a microsecond-scale decode launch cannot pay on every call. */
static inline int64_t glint_resident_grid(const void *kernel, int threads, size_t dyn_lds) {
    static std::mutex mu;
    static struct { const void *k; int dev, threads; size_t lds; int64_t blocks; } seen[128];
    static int nseen = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return 256;
    {
        std::lock_guard<std::mutex> lock(mu);
        for (int i = 0; i < nseen; ++i)
            if (seen[i].k == kernel && seen[i].dev == dev && seen[i].threads == threads && seen[i].lds == dyn_lds)
                return seen[i].blocks;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        cus = 256;
    const int64_t blocks = (int64_t)cus * glint_resident_blocks(kernel, threads, dyn_lds);
    std::lock_guard<std::mutex> lock(mu);
    if (nseen < 128)
        seen[nseen++] = {kernel, dev, threads, dyn_lds, blocks};
    return blocks;
}

/* CUs of the current device (256 if the runtime cannot say), cached per device. */
static inline int glint_cu_count() {
    static std::mutex mu;
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

/* Raise a kernel's dynamic-LDS limit to `bytes` on the current device (needed above
 * 64 KiB); remembered per (kernel, device). Returns 0 or -1. */
static inline int glint_set_lds_limit(const void *kernel, size_t bytes) {
    static std::mutex mu;
    /* (kernel, device) pairs already raised; past the last slot the attribute is set on every
     * call, which is correct but costs a runtime call per launch */
    static struct { const void *k; int dev; size_t bytes; } seen[256];
    static int nseen = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return -1;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < nseen; ++i)
        if (seen[i].k == kernel && seen[i].dev == dev && seen[i].bytes >= bytes)
            return 0;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess)
        return -1;
    if (nseen < 256)
        seen[nseen++] = {kernel, dev, bytes};
    return 0;
}

#endif
