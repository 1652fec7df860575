/* Double-buffered BF16 MFMA tile GEMM whose weight operand is dequantized into LDS
 * (gfx950). Shared by the GLINT prefill GEMM and the INT8-pin W8A16 GEMM.
 *
 * y[M, N] = x[M, K] W^T, x BF16 [M, K] row-major with 16-B aligned rows and K % 64 == 0.
 * W is made 16 weights at a time by a Producer, which owns the weight format:
 *   struct Regs;                                  registers of one thread's step
 *   load(Regs &, int row, int quarter, int kb)    global loads of W[row, 64 kb + 16 quarter, +16),
 *                                                 row < N and kb < K / 64 (the kernel clamps)
 *   lookup(const Regs &, float (&v)[16], lane)    first phase (table reads are issued here, so
 *                                                 their latency overlaps the step's MFMAs)
 *   finish(const Regs &, const float (&v)[16], uint32_t (&)[8])
 *                                                 the 16 weights as BF16 pairs (lo = even k)
 *   LDS_WORDS, setup(float *lds, float *stage)    LDS the producer needs, filled before step 0
 *                                                 (stage: 256 words of scratch LDS, free again
 *                                                 after setup returns)
 *
 * Block tile BM x BN x 64 (K) over WM x WN waves; each wave owns a (BM / WM) x (BN / WN)
 * tile of v_mfma_f32_16x16x32_bf16 accumulators (f32). Thread t produces W row t / 4,
 * K quarter t % 4 (so BN * 4 == threads), and stages BM * 8 / threads 16-B chunks of x.
 * Each operand has two LDS buffers: step kb runs its MFMAs from buffer kb & 1, then the
 * threads write step kb + 1 into the other, so a K step needs one barrier. Global loads run
 * R steps ahead through a ring of R register stages. LDS rows are 64 BF16 with an XOR
 * swizzle of their 16-byte chunks (tile_ofs).
 *
 * Split K: gridDim.z workgroups share an output tile, workgroup z walking K steps
 * [z kps, (z + 1) kps). Each writes its f32 partial tile to `part` and counts itself in
 * ctr[tile]; the last to arrive adds the partials in z order (whichever workgroup that is,
 * the sum is the same), stores the tile and clears its counter, so counters are zero
 * between launches. With gridDim.z == 1, part and ctr are unused.
 *
 * MFMA operand layout (16x16x32 bf16): lane l supplies row l % 16, k [(l / 16) * 8, +8)
 * of each operand; accumulator i of lane l is D[(l / 16) * 4 + i][l % 16].
 */
#ifndef GLINT_TILE_MFMA_H_
#define GLINT_TILE_MFMA_H_

#include "glint_common.h"

#include <algorithm>

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
#ifndef TILE_SPLIT_MAX
#define TILE_SPLIT_MAX 4 /* most K splits per output tile */
#endif

#ifndef TILE_INTERLEAVE
#define TILE_INTERLEAVE 1 /* k_tile_mfma: second K slice's fragment reads between the first's MFMAs */
#endif
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

/* GLINT planes, bs = 64: weight = CELLS[h][p] * absmax, through the 32-copy LDS cell
 * table (lane l reads copy l % 32). A 64-copy table, whose lookup address is one
 * v_perm_b32, measured 3% slower here: its fill doubles and the LDS budget tightens. */
/* Weight loads of the tile producers. A tile GEMM reads every weight once per block of x
 * rows, so the loads keep the default cache policy and the blocks after the first find the
 * weights in L2. With the nontemporal hint (right for the M = 1 GEMV, which reads each weight
 * once) every block fetched them again from beyond L2: on the 14336 x 4096 gate shape M = 512
 * went 91.9 -> 82.5 us, M = 2048 325.5 -> 264.4 us with plain loads; M <= 128 moved by 1-3%.
 * TILE_W_NT_STEP / TILE_W_NT_SS = 1 restore the hint for the per-step (k_tile_mfma,
 * k_tile_big) and the super-step (k_tile_ss) loads. */
#ifndef TILE_W_NT_STEP
#define TILE_W_NT_STEP 0
#endif
#ifndef TILE_W_NT_SS
#define TILE_W_NT_SS 0
#endif
template <int NT, class V> __device__ __forceinline__ V tile_wload(const V *p) {
    if constexpr (NT != 0)
        return __builtin_nontemporal_load(p);
    else
        return *p;
}

struct GlintTileProducer {
    const glint_u32x2 *hole, *plug; /* 8 B = 16 elements of each plane */
    const float *absmax;
    int N, K;
    float *ltab;
    static constexpr int LDS_WORDS = GLINT_LDS_CELLS_WORDS;
    static constexpr int LOADS = 3; /* global load instructions per load() */
    struct Regs {
        glint_u32x2 h, p;
        float a;
    };
    __device__ __forceinline__ void setup(float *lds, float *) {
        ltab = lds;
        glint_fill_cells_lds_direct(lds);
    }
    __device__ __forceinline__ void load(Regs &r, int row, int quarter, int kb) const {
        const int64_t q = (int64_t)row * (K >> 4) + kb * 4 + quarter;
        r.h = tile_wload<TILE_W_NT_STEP>(&hole[q]);
        r.p = tile_wload<TILE_W_NT_STEP>(&plug[q]);
        r.a = absmax[(int64_t)row * (K >> 6) + kb];
    }
    /* load() with the row given as base = row * K / 16 (8-B units), for N * K < 2^36: one
     * 32-bit register per row instead of two 64-bit offsets */
    static constexpr int REG_WORDS = 5; /* h, p, a: the leading words of Regs */
    __device__ __forceinline__ uint32_t row_base(int row) const { return (uint32_t)row * (uint32_t)(K >> 4); }
    __device__ __forceinline__ void load_at(Regs &r, uint32_t base, int quarter, int kb) const {
        const uint32_t q = base + (uint32_t)(kb * 4 + quarter);
        r.h = tile_wload<TILE_W_NT_STEP>(&hole[q]);
        r.p = tile_wload<TILE_W_NT_STEP>(&plug[q]);
        r.a = absmax[(base >> 2) + (uint32_t)kb];
    }
    /* v[8 q + 2 b] / v[8 q + 2 b + 1]: cells of the even / odd element of byte b of word q */
    __device__ __forceinline__ void lookup(const Regs &r, float (&v)[16], int lane) const {
        const uint32_t H[2] = {r.h.x, r.h.y}, P[2] = {r.p.x, r.p.y};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t E = glint_codes_even(H[q], P[q]);
            const uint32_t O = glint_codes_odd(H[q], P[q]);
            const uint32_t lb = lane & 31;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                v[8 * q + 2 * b] = ltab[(((E >> (8 * b)) & 0xFFu) << 5) | lb];
                v[8 * q + 2 * b + 1] = ltab[(((O >> (8 * b)) & 0xFFu) << 5) | lb];
            }
        }
    }
    __device__ __forceinline__ void finish(const Regs &r, const float (&v)[16], uint32_t (&packed)[8]) const {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            packed[i] = glint_cvt_bf16x2(v[2 * i] * r.a, v[2 * i + 1] * r.a);
    }
    /* The f32 weights w = CELLS * absmax (the reference's f32 product) as three BF16 planes
     * with w == hi + mid + lo exactly: hi keeps w's top 16 bits, mid the top 16 bits of the
     * exact remainder w - hi, and lo = w - hi - mid, which has at most 8 significant bits
     * (w has 24), so it is a BF16 value as it stands. A product x * plane is then exact in
     * the MFMA and y differs from the f32 sum of w * x only by the accumulation. An infinite
     * w (absmax inf, or an f32 overflow of CELLS * absmax) keeps mid = lo = 0, where w - hi
     * would be NaN; a NaN w stays NaN in hi (its quiet bit is in the top half). */
    __device__ __forceinline__ void finish_split(const Regs &r, const float (&v)[16], uint32_t (&packed)[3][8]) const {
        const bool big = !(__builtin_fabsf(r.a) < 0x1p126f); /* only there can w be infinite */
        float hi[16], mid[16], lo[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float w = v[i] * r.a;
            hi[i] = __uint_as_float(__float_as_uint(w) & 0xFFFF0000u);
            float r1 = w - hi[i];
            if (big)
                r1 = __builtin_isinf(w) ? 0.0f : r1;
            mid[i] = __uint_as_float(__float_as_uint(r1) & 0xFFFF0000u);
            lo[i] = r1 - mid[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            packed[0][i] = __builtin_amdgcn_perm(__float_as_uint(hi[2 * i + 1]), __float_as_uint(hi[2 * i]), 0x07060302u);
            packed[1][i] = __builtin_amdgcn_perm(__float_as_uint(mid[2 * i + 1]), __float_as_uint(mid[2 * i]), 0x07060302u);
            packed[2][i] = __builtin_amdgcn_perm(__float_as_uint(lo[2 * i + 1]), __float_as_uint(lo[2 * i]), 0x07060302u);
        }
    }

    /* Super-step interface (k_tile_ss): piece c (0..7) of a row's super-step (4 K steps, 256
     * elements) is elements [32 c, +32): 16 B of each plane and one absmax. Its groups h = 0, 1
     * (16 elements each) lie in K step c / 2, quarters 2 (c & 1) + h. `step` is the piece's
     * K step, already clamped into the matrix by the caller. */
    struct SRegs {
        glint_u32x4 h, p;
        float a;
    };
    static __device__ __forceinline__ int sstep(int c, int) { return c >> 1; }
    static __device__ __forceinline__ int squarter(int c, int h) { return ((c & 1) << 1) | h; }
    __device__ __forceinline__ void sload(SRegs &r, int row, int step0, int c, int last) const {
        const int kb = min(step0 + (c >> 1), last);
        const int64_t i = (int64_t)row * (K >> 5) + kb * 2 + (c & 1);
        r.h = tile_wload<TILE_W_NT_SS>((const glint_u32x4 *)hole + i);
        r.p = tile_wload<TILE_W_NT_SS>((const glint_u32x4 *)plug + i);
        r.a = absmax[(int64_t)row * (K >> 6) + kb];
    }
    __device__ __forceinline__ void slookup(const SRegs &r, int h, float (&v)[16], int lane) const {
        Regs g;
        g.h = h ? glint_u32x2{r.h.z, r.h.w} : glint_u32x2{r.h.x, r.h.y};
        g.p = h ? glint_u32x2{r.p.z, r.p.w} : glint_u32x2{r.p.x, r.p.y};
        lookup(g, v, lane);
    }
    __device__ __forceinline__ void sfinish(const SRegs &r, int, const float (&v)[16], uint32_t (&packed)[8]) const {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            packed[i] = glint_cvt_bf16x2(v[2 * i] * r.a, v[2 * i + 1] * r.a);
    }
};

/* INT8 pin (bf16_to_int8_pin_v1), k_in % 64 == 0: weight = BF16 RNE((float)q * scale),
 * scale one f32 per 64 consecutive weights of a row. */
struct Int8PinTileProducer {
    const glint_u32x4 *q; /* 16 weights */
    const float *scale;
    int N, K;
    static constexpr int LDS_WORDS = 0;
    static constexpr int LOADS = 2; /* global load instructions per load() */
    struct Regs {
        glint_u32x4 w;
        float s;
    };
    __device__ __forceinline__ void setup(float *, float *) {}
    __device__ __forceinline__ void load(Regs &r, int row, int quarter, int kb) const {
        r.w = tile_wload<TILE_W_NT_STEP>(&q[(int64_t)row * (K >> 4) + kb * 4 + quarter]);
        r.s = scale[(int64_t)row * (K >> 6) + kb];
    }
    /* load() with the row given as base = row * K / 16 (16-B units), for N * K < 2^36 */
    static constexpr int REG_WORDS = 5; /* w, s: the leading words of Regs */
    __device__ __forceinline__ uint32_t row_base(int row) const { return (uint32_t)row * (uint32_t)(K >> 4); }
    __device__ __forceinline__ void load_at(Regs &r, uint32_t base, int quarter, int kb) const {
        r.w = tile_wload<TILE_W_NT_STEP>(&q[base + (uint32_t)(kb * 4 + quarter)]);
        r.s = scale[(base >> 2) + (uint32_t)kb];
    }
    __device__ __forceinline__ void lookup(const Regs &r, float (&v)[16], int) const {
        const uint32_t W[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = (float)(int8_t)(W[i >> 2] >> (8 * (i & 3)));
    }
    __device__ __forceinline__ void finish(const Regs &r, const float (&v)[16], uint32_t (&packed)[8]) const {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            packed[i] = glint_cvt_bf16x2(v[2 * i] * r.s, v[2 * i + 1] * r.s);
    }

    /* Super-step interface (k_tile_ss): piece c (0..7) of a row's 256-byte super-step is the
     * 16 bytes at 16 c and at 128 + 16 c (each load instruction then covers whole 128-B
     * lines); group h lies in K step c / 4 + 2 h, quarter c & 3. */
    struct SRegs {
        glint_u32x4 w[2];
        float s[2];
    };
    static __device__ __forceinline__ int sstep(int c, int h) { return (c >> 2) + 2 * h; }
    static __device__ __forceinline__ int squarter(int c, int) { return c & 3; }
    __device__ __forceinline__ void sload(SRegs &r, int row, int step0, int c, int last) const {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int kb = min(step0 + sstep(c, h), last);
            r.w[h] = tile_wload<TILE_W_NT_SS>(&q[(int64_t)row * (K >> 4) + kb * 4 + (c & 3)]);
            r.s[h] = scale[(int64_t)row * (K >> 6) + kb];
        }
    }
    __device__ __forceinline__ void slookup(const SRegs &r, int h, float (&v)[16], int) const {
        const uint32_t W[4] = {r.w[h].x, r.w[h].y, r.w[h].z, r.w[h].w};
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = (float)(int8_t)(W[i >> 2] >> (8 * (i & 3)));
    }
    __device__ __forceinline__ void sfinish(const SRegs &r, int h, const float (&v)[16], uint32_t (&packed)[8]) const {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            packed[i] = glint_cvt_bf16x2(v[2 * i] * r.s[h], v[2 * i + 1] * r.s[h]);
    }
};

/* Split-K epilogue (gridDim.z > 1). Partials and counters are accessed with device-scope
 * relaxed atomics, which are coherent across the XCDs' separate L2 caches without the L2
 * write-back and invalidate that device-scope fences cost. Ordering: a workgroup's partial
 * stores have completed (vmcnt 0) before the barrier that precedes its counter increment,
 * and the reducer issues its partial loads after it has seen the final count. Partial
 * element e of thread t sits at e T + t. Returns true in the last workgroup of the tile,
 * whose acc then holds the z-ordered sum; the others return false and store nothing.
 * s_last: one word of LDS that nothing else uses any more. */
/* tid: the thread's index among the T that hold the tile (threadIdx.x unless the block has
 * more threads than that); threads with active false hold no part of it, store and load
 * nothing and only join the barriers. */
template <int NA, int NB, int T>
__device__ __forceinline__ bool tile_splitk_epilogue(glint_f32x4 (&acc)[NA][NB], float *__restrict__ part,
                                                     unsigned *ctr, unsigned &s_last, int tid, bool active) {
    constexpr int NV = NA * NB * 4;
    const unsigned tile = blockIdx.y * gridDim.x + blockIdx.x;
    const size_t tsz = (size_t)NV * T, zstride = (size_t)gridDim.x * gridDim.y * tsz;
    float *mine = part + blockIdx.z * zstride + tile * tsz;
    if (active)
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    __hip_atomic_store(mine + ((a * NB + b) * 4 + i) * T + tid, acc[a][b][i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0);
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(&ctr[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.z - 1;
    __syncthreads();
    if (!s_last)
        return false;
    if (!active)
        return true;
    /* The partials are read in rounds of CH accumulators, all TILE_SPLIT_MAX splits of a
     * round in flight at once (z clamped; a split past gridDim.z is loaded and ignored). */
    constexpr int CH = NV < 16 ? NV : 16;
    const unsigned zl = gridDim.z - 1;
    const float *base = part + tile * tsz;
#pragma unroll
    for (int c0 = 0; c0 < NV; c0 += CH) {
        float v[TILE_SPLIT_MAX][CH];
#pragma unroll
        for (int z = 0; z < TILE_SPLIT_MAX; ++z)
#pragma unroll
            for (int c = 0; c < CH; ++c)
                v[z][c] = __hip_atomic_load(base + min((unsigned)z, zl) * zstride + (size_t)(c0 + c) * T + tid,
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int e = c0 + c, a = e / (NB * 4), b = (e / 4) % NB, i = e % 4;
            float sum = blockIdx.z == 0 ? acc[a][b][i] : v[0][c];
#pragma unroll
            for (int z = 1; z < TILE_SPLIT_MAX; ++z)
                if ((unsigned)z <= zl)
                    sum += (unsigned)z == blockIdx.z ? acc[a][b][i] : v[z][c];
            acc[a][b][i] = sum;
        }
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(&ctr[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}
template <int NA, int NB, int T>
__device__ __forceinline__ bool tile_splitk_epilogue(glint_f32x4 (&acc)[NA][NB], float *__restrict__ part,
                                                     unsigned *ctr, unsigned &s_last) {
    return tile_splitk_epilogue<NA, NB, T>(acc, part, ctr, s_last, (int)threadIdx.x, true);
}

/* Stream-K partition of a tile GEMM: the flattened units (tile, K step), tile-major, tiles
 * numbered row-major over the gx-wide tile grid, are cut into `wgs` contiguous ranges of
 * equal length (to one unit), workgroup g owning [start(g), start(g + 1)) with start(g) =
 * floor(g units / wgs). A workgroup walks its range as segments, one per tile it touches:
 * the tail of one tile, whole tiles, the head of another. Whole tiles are stored directly;
 * the contributors of a split tile meet through the split-K workspace (tile_sk_fixup).
 * With one workgroup per CU and units spread evenly, no CU idles while another still has a
 * tile to finish, whatever the tile count. */
struct TileSK {
    int units; /* tiles * nk < 2^31 (the host checks) */
    int wgs, nk, gx;
};
#define TILE_SK_SEGS 3 /* most segments (tiles touched) per workgroup */
__device__ __forceinline__ int tile_sk_start(const TileSK &sk, int g) {
    return (int)((int64_t)g * sk.units / sk.wgs);
}
/* the workgroup whose range holds unit v: the largest g with start(g) <= v */
__device__ __forceinline__ int tile_sk_owner(const TileSK &sk, int v) {
    return (int)(((int64_t)(v + 1) * sk.wgs + sk.units - 1) / sk.units) - 1;
}

/* Stream-K epilogue of a segment that covers part of tile t (workgroup g). The tile's
 * contributors are workgroups glo .. ghi (at most CMAX, which the host checks); each that
 * is not the last to arrive writes its f32 partial to its slot (2 h + e: e = 0 where tile t
 * holds the start of h's range, else 1, so a workgroup's first and last segments never
 * share a slot) and counts itself in ctr[glo] (glo's range ends inside t, so no other split
 * tile uses that counter). A workgroup that finds all others counted skips its own write.
 * The last adds the partials in contributor order, whichever workgroup it is, so the sum
 * and the result are deterministic, clears the counter and returns true with the sum in
 * acc. Ordering and atomics as in tile_splitk_epilogue. s_flag: one word of LDS that
 * nothing else uses any more; tid: threadIdx.x. */
template <int NA, int NB, int T, int CMAX>
__device__ __forceinline__ bool tile_sk_fixup(glint_f32x4 (&acc)[NA][NB], const TileSK &sk, int g, int t,
                                              float *__restrict__ part, unsigned *ctr, unsigned &s_flag, int tid) {
    constexpr int NV = NA * NB * 4;
    const int t0 = t * sk.nk;
    const int glo = tile_sk_owner(sk, t0), ghi = tile_sk_owner(sk, t0 + sk.nk - 1);
    const unsigned c = (unsigned)(ghi - glo + 1);
    unsigned *cnt = ctr + glo;
    auto slot = [&](int h) -> float * {
        const int e = tile_sk_start(sk, h) >= t0 ? 0 : 1;
        return part + (size_t)(2 * h + e) * ((size_t)NV * T);
    };
    if (tid == 0)
        s_flag = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == c - 1;
    __syncthreads();
    bool last = s_flag != 0;
    __syncthreads(); /* every thread has read s_flag before it is written again */
    if (!last) {
        float *mine = slot(g);
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    __hip_atomic_store(mine + ((a * NB + b) * 4 + i) * T + tid, acc[a][b][i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0);
        __syncthreads();
        if (tid == 0)
            s_flag = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == c - 1;
        __syncthreads();
        last = s_flag != 0;
    }
    if (!last)
        return false;
    /* the other contributors' partials in rounds of CH accumulators, all in flight at once
     * (other contributor i is contributor i, or i + 1 from the reducer's own index on;
     * indices past the last contributor are clamped to it, loaded and ignored, so no load
     * sits under a branch) */
    constexpr int CH = NV < 16 ? NV : 16, NO = CMAX - 1;
    const int me = g - glo;
    const float *src[NO];
#pragma unroll
    for (int i = 0; i < NO; ++i)
        src[i] = slot(glo + min(i < me ? i : i + 1, (int)c - 1));
#pragma unroll
    for (int c0 = 0; c0 < NV; c0 += CH) {
        float v[NO][CH];
#pragma unroll
        for (int i = 0; i < NO; ++i)
#pragma unroll
            for (int k = 0; k < CH; ++k)
                v[i][k] = __hip_atomic_load(src[i] + (size_t)(c0 + k) * T + tid, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int e = c0 + k, a = e / (NB * 4), b = (e / 4) % NB, q = e % 4;
            const float mine = acc[a][b][q];
            float sum = me == 0 ? mine : v[0][k];
#pragma unroll
            for (int j = 1; j < CMAX; ++j)
                if ((unsigned)j < c)
                    sum += j == me ? mine : (j < me ? v[j < NO ? j : NO - 1][k] : v[j - 1][k]);
            acc[a][b][q] = sum;
        }
        __builtin_amdgcn_sched_barrier(0); /* one round's loads in flight at a time */
    }
    if (tid == 0)
        __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

/* NP = 1: W is one BF16 plane (the BF16-out GEMMs). NP = 3: the producer's finish_split
 * makes three BF16 planes whose sum is the f32 weight exactly, and every x fragment is
 * multiplied with all three (the f32-out H-TILE: f32 products, f32 accumulation). */
template <int BM, int BN, int WM, int WN, int R, class P, class Out, int NP = 1>
__global__ __launch_bounds__(64 * WM * WN) void k_tile_mfma(P p, const uint16_t *__restrict__ x,
                                                             typename Out::T *__restrict__ y, int M, int N, int K,
                                                             int kps, float *__restrict__ part, unsigned *ctr) {
    constexpr int T = 64 * WM * WN;
    constexpr int TM = BM / WM / 16, TN = BN / WN / 16; /* MFMA tiles per wave */
    constexpr int XV = BM * 8 / T;                      /* x chunks per thread */
    constexpr int U = (R % 2) ? 2 * R : R;              /* steps per unrolled round */
    constexpr int NV = TM * TN * 4;                     /* accumulators per thread */
    static_assert(BN * 4 == T, "each thread produces a quarter of one W row");
    static_assert(XV * T == BM * 8 && TM * WM * 16 == BM && TN * WN * 16 == BN, "tile shape");
    static_assert(R >= 2 && R <= 8, "register stages");
    static_assert(NP == 1 || NP == 3, "W planes");
    __shared__ float ptab[P::LDS_WORDS > 0 ? P::LDS_WORDS : 1];
    __shared__ __attribute__((aligned(16))) uint16_t sX[2][BM * TILE_LDW];
    __shared__ __attribute__((aligned(16))) uint16_t sW[2][NP][BN * TILE_LDW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb0 = blockIdx.z * kps;
    const int ns = min(K >> 6, kb0 + kps) - kb0; /* >= 1: the host sizes gridDim.z */
    const int wr = tid >> 2, wq = tid & 3;
    const int xr = tid >> 3, xc = tid & 7; /* x chunk i: row xr + (T / 8) i, columns 8 xc */
    glint_f32x4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
            acc[a][b] = glint_f32x4{0.f, 0.f, 0.f, 0.f};

    /* Register stage (j + 1) % R holds local step j + 1 while step j runs; step j writes it
     * to LDS and refills the stage with step j + 1 + R. Rows past M or N are clamped into the
     * matrix (their outputs are not stored) and steps past the end reload the last one, so
     * every load is unconditional and the wait counts stay exact. */
    struct Stage {
        typename P::Regs w;
        glint_u32x4 x[XV];
    };
    Stage st[R];
    const int wrow = min(n0 + wr, N - 1);
    auto gload = [&](int j, Stage &sg) {
        const int kb = kb0 + min(j, ns - 1);
        p.load(sg.w, wrow, wq, kb);
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int m = min(m0 + xr + (T / 8) * i, M - 1);
            sg.x[i] = *(const glint_u32x4 *)(x + (int64_t)m * K + (int64_t)kb * 64 + xc * 8);
        }
    };
    auto store = [&](int buf, const Stage &sg, const float (&v)[16]) {
        uint32_t packed[NP][8];
        if constexpr (NP == 1)
            p.finish(sg.w, v, packed[0]);
        else
            p.finish_split(sg.w, v, packed);
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) {
            *(glint_u32x4 *)(sW[buf][pl] + tile_ofs(wr, 2 * wq)) =
                glint_u32x4{packed[pl][0], packed[pl][1], packed[pl][2], packed[pl][3]};
            *(glint_u32x4 *)(sW[buf][pl] + tile_ofs(wr, 2 * wq + 1)) =
                glint_u32x4{packed[pl][4], packed[pl][5], packed[pl][6], packed[pl][7]};
        }
#pragma unroll
        for (int i = 0; i < XV; ++i)
            *(glint_u32x4 *)(sX[buf] + tile_ofs(xr + (T / 8) * i, xc)) = sg.x[i];
    };
    /* local step j (j % U == u): the fragments of buffer u & 1 and the table reads for step
     * j + 1 are issued together, then the MFMAs run while they land; step j + 1 then goes into
     * the other buffer and its register stage is refilled */
    auto step = [&](int j, int u) {
        const int cur = u & 1;
        Stage &nx = st[(u + 1) % R];
        glint_bf16x8 af[2][TM], bfr[2][NP][TN];
        /* rows (16-row tile base) + lane % 16, chunk 4 ks + lane / 16; the swizzle does not
         * change when a row moves by a multiple of 16 */
        auto frags = [&](int ks) {
            const int fofs = tile_ofs(lane & 15, 4 * ks + (lane >> 4));
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[ks][a] = __builtin_bit_cast(
                    glint_bf16x8, *(const glint_u32x4 *)(sX[cur] + (wm * TM * 16 + a * 16) * TILE_LDW + fofs));
#pragma unroll
            for (int pl = 0; pl < NP; ++pl)
#pragma unroll
                for (int b = 0; b < TN; ++b)
                    bfr[ks][pl][b] = __builtin_bit_cast(
                        glint_bf16x8, *(const glint_u32x4 *)(sW[cur][pl] + (wn * TN * 16 + b * 16) * TILE_LDW + fofs));
        };
        /* planes outermost: consecutive MFMAs update different accumulators */
        auto mfmas = [&](int ks) {
#pragma unroll
            for (int pl = 0; pl < NP; ++pl)
#pragma unroll
                for (int a = 0; a < TM; ++a)
#pragma unroll
                    for (int b = 0; b < TN; ++b)
                        acc[a][b] =
                            __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[ks][a], bfr[ks][pl][b], acc[a][b], 0, 0, 0);
        };
        float v[16];
        if (TILE_INTERLEAVE) {
            /* the second K slice's fragment reads go out between the first slice's MFMAs */
            frags(0);
            p.lookup(nx.w, v, lane);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(0);
            frags(1);
#pragma unroll
            for (int i = 0; i < TM + NP * TN; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, (NP * TM * TN) / (TM + NP * TN), 0); /* MFMA */
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                               /* LDS read */
            }
            __builtin_amdgcn_sched_barrier(0);
            mfmas(1);
        } else {
            frags(0);
            frags(1);
            p.lookup(nx.w, v, lane);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(0);
            mfmas(1);
        }
        __builtin_amdgcn_sched_barrier(0);
        store(cur ^ 1, nx, v); /* past the end: a clamped copy nobody reads */
        gload(j + 1 + R, nx);
        __syncthreads();
    };

    p.setup(ptab, (float *)&sX[0][0]); /* sX is free until the first x store */
#pragma unroll
    for (int i = 0; i < R; ++i)
        gload(i, st[i]);
    {
        float v[16];
        p.lookup(st[0].w, v, lane);
        store(0, st[0], v);
    }
    gload(R, st[0]);
    __syncthreads();
    int j = 0;
    for (; j + U <= ns; j += U) {
#pragma unroll
        for (int u = 0; u < U; ++u)
            step(j + u, u);
    }
#pragma unroll
    for (int u = 0; u + 1 < U; ++u)
        if (j + u < ns)
            step(j + u, u);

    if (gridDim.z > 1 && !tile_splitk_epilogue<TM, TN, T>(acc, part, ctr, *(unsigned *)&sX[0][0]))
        return;
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

/* Tile GEMM for BN = 64 or 32 W rows (M up to a few hundred) with the weights streamed in
 * super-steps of 4 K steps (256 elements): per super-step a thread loads 16-B pieces of
 * RR = BN / 32 W rows such that 8 consecutive lanes cover a whole 128-B line of a plane
 * (P::sload). Loads that cover whole lines stream at about twice the rate of the per-step
 * 8-byte pieces k_tile_mfma uses, which bounded it at small M. The 2 RR groups of 16
 * weights a thread holds are dequantized into a double-buffered 4-step W tile in LDS
 * (super-step s + 1 while s is multiplied): at RR = 2 one group per K step, at RR = 1 one
 * every other step (looked up in one step, stored in the next). x keeps the per-step ring
 * (RX stages) and double buffer of k_tile_mfma. Block tile BM x BN over 2 x 2 waves
 * (BM = 64 or 128); W rows 8 w + lane / 8 (+ 32) of wave w, piece lane % 8. Clamping and
 * split K as in k_tile_mfma. */
/* BM = 64 without a producer table, or BN = 32 (80 KiB of LDS with the table): at most 256
 * VGPRs (two waves per SIMD), so two workgroups fit a CU */
template <int BM, int BN, int RX, class P, class Out>
__global__ __launch_bounds__(256, (BN == 32 || (BM == 64 && P::LDS_WORDS == 0)) ? 2 : 1) void k_tile_ss(P p, const uint16_t *__restrict__ x, typename Out::T *__restrict__ y,
                                                 int M, int N, int K, int kps, float *__restrict__ part,
                                                 unsigned *ctr) {
    constexpr int T = 256, WN = 2, TM = BM / 32, TN = BN / 32, RR = BN / 32, XV = BM * 8 / T;
    constexpr int U = 8; /* steps per unrolled round: two super-steps, RX | 8 */
    static_assert((BM == 64 || BM == 128) && (BN == 32 || BN == 64) && (RX == 2 || RX == 4 || RX == 8),
                  "tile shape, x stages");
    __shared__ float ptab[P::LDS_WORDS > 0 ? P::LDS_WORDS : 1];
    __shared__ __attribute__((aligned(16))) uint16_t sX[2][BM * TILE_LDW];
    __shared__ __attribute__((aligned(16))) uint16_t sW[2][4][BN * TILE_LDW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb0 = blockIdx.z * kps;
    const int ns = min(K >> 6, kb0 + kps) - kb0; /* >= 1: the host sizes gridDim.z */
    const int last = kb0 + ns - 1;               /* W loads past the split clamp here */
    const int c = lane & 7;
    int lrow[RR], wrow[RR];
#pragma unroll
    for (int rr = 0; rr < RR; ++rr) {
        lrow[rr] = wave * 8 + (lane >> 3) + 32 * rr;
        wrow[rr] = min(n0 + lrow[rr], N - 1);
    }
    const int xr = tid >> 3, xc = tid & 7; /* x chunk i: row xr + 32 i, columns 8 xc */
    glint_f32x4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
            acc[a][b] = glint_f32x4{0.f, 0.f, 0.f, 0.f};

    typename P::SRegs sw[2][RR]; /* [super-stage][row set] */
    glint_u32x4 xs[RX][XV];
    auto gload_w = [&](int ss, typename P::SRegs (&sg)[RR]) {
#pragma unroll
        for (int rr = 0; rr < RR; ++rr)
            p.sload(sg[rr], wrow[rr], kb0 + 4 * ss, c, last);
    };
    auto gload_x = [&](int j, glint_u32x4 (&xg)[XV]) {
        const int kb = kb0 + min(j, ns - 1);
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int m = min(m0 + xr + 32 * i, M - 1);
            xg[i] = *(const glint_u32x4 *)(x + (int64_t)m * K + (int64_t)kb * 64 + xc * 8);
        }
    };
    auto store_x = [&](int buf, const glint_u32x4 (&xg)[XV]) {
#pragma unroll
        for (int i = 0; i < XV; ++i)
            *(glint_u32x4 *)(sX[buf] + tile_ofs(xr + 32 * i, xc)) = xg[i];
    };
    /* group t of a super-stage: row set t / 2, half t % 2. The 16-B chunks of W step slot s
     * are additionally XORed with s: the 8 lanes of a store instruction (one row, 4 slots)
     * then hit 8 distinct bank groups, and a fragment read (one slot) is unchanged. */
    auto finish_w = [&](int buf, const typename P::SRegs (&sg)[RR], int t, const float (&v)[16]) {
        uint32_t pk[8];
        p.sfinish(sg[t >> 1], t & 1, v, pk);
        const int slot = P::sstep(c, t & 1), qq = P::squarter(c, t & 1);
        uint16_t *w = sW[buf][slot];
        *(glint_u32x4 *)(w + tile_ofs(lrow[t >> 1], (2 * qq) ^ slot)) = glint_u32x4{pk[0], pk[1], pk[2], pk[3]};
        *(glint_u32x4 *)(w + tile_ofs(lrow[t >> 1], (2 * qq + 1) ^ slot)) = glint_u32x4{pk[4], pk[5], pk[6], pk[7]};
    };
    /* local step j, u = j % 8: super-step j / 4 (LDS tile (u / 4) & 1, slot t = u % 4). First
     * the LDS stores for later steps go out (group t of super-step j / 4 + 1, looked up in
     * the previous step, and x of step j + 1), so their latency hides behind this step's
     * reads and MFMAs; then the fragments, the table reads of the next group, the MFMAs.
     * After group 3 the super-stage is refilled two super-steps ahead. */
    float v[16]; /* table reads of the next group to store */
    auto step = [&](int j, int u) {
        const int t = u & 3, sb = (u >> 2) & 1;
        typename P::SRegs(&nw)[RR] = sw[sb ^ 1];
        /* past the end: clamped data nobody reads */
        if constexpr (RR == 2)
            finish_w(sb ^ 1, nw, t, v);
        else if (t & 1)
            finish_w(sb ^ 1, nw, t >> 1, v);
        store_x((u & 1) ^ 1, xs[(u + 1) % RX]);
        glint_bf16x8 af[2][TM], bfr[2][TN];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int fofs = tile_ofs(lane & 15, 4 * ks + (lane >> 4));
            const int wofs = tile_ofs(lane & 15, (4 * ks + (lane >> 4)) ^ t);
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[ks][a] = __builtin_bit_cast(
                    glint_bf16x8, *(const glint_u32x4 *)(sX[u & 1] + (wm * TM * 16 + a * 16) * TILE_LDW + fofs));
#pragma unroll
            for (int b = 0; b < TN; ++b)
                bfr[ks][b] = __builtin_bit_cast(
                    glint_bf16x8, *(const glint_u32x4 *)(sW[sb][t] + (wn * TN * 16 + b * 16) * TILE_LDW + wofs));
        }
        if constexpr (RR == 1) {
            if (!(t & 1))
                p.slookup(nw[0], t >> 1, v, lane);
        } else if (t < 3) {
            p.slookup(nw[(t + 1) >> 1], (t + 1) & 1, v, lane);
        } else {
            p.slookup(sw[sb][0], 0, v, lane); /* group 0 of super-step j / 4 + 2 */
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[ks][a], bfr[ks][b], acc[a][b], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (t == 3)
            gload_w((j >> 2) + 3, nw);
        gload_x(j + 1 + RX, xs[(u + 1) % RX]);
        __syncthreads();
    };

    p.setup(ptab, (float *)&sX[0][0]); /* sX is free until the first x store */
    gload_w(0, sw[0]);
    gload_w(1, sw[1]);
#pragma unroll
    for (int i = 0; i < RX; ++i)
        gload_x(i, xs[i]);
#pragma unroll
    for (int t = 0; t < 2 * RR; ++t) {
        p.slookup(sw[0][t >> 1], t & 1, v, lane);
        finish_w(0, sw[0], t, v);
    }
    if constexpr (RR == 2)
        p.slookup(sw[1][0], 0, v, lane);
    gload_w(2, sw[0]);
    store_x(0, xs[0]);
    gload_x(RX, xs[0]);
    __syncthreads();
    int j = 0;
    for (; j + U <= ns; j += U) {
#pragma unroll
        for (int u = 0; u < U; ++u)
            step(j + u, u);
    }
#pragma unroll
    for (int u = 0; u + 1 < U; ++u)
        if (j + u < ns)
            step(j + u, u);

    if (gridDim.z > 1 && !tile_splitk_epilogue<TM, TN, T>(acc, part, ctr, *(unsigned *)&sX[0][0]))
        return;
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

/* 256 x 256 block tile (M >= 256): 8 waves in 2 (M) x 4 (N), wave tile 128 x 64 (8 x 4 MFMA
 * tiles, 128 accumulator registers per lane), so each MFMA operand byte read from LDS feeds
 * 1.33x the MACs of a 64 x 64 wave tile. The x tile reaches LDS without passing through
 * registers: each wave issues 4 buffer loads with the lds bit per step (8 rows x 128 B
 * each), every lane loading the 16-B chunk that belongs at its LDS slot under the row
 * swizzle. That keeps x out of the register budget the accumulators need. The x load for
 * step j + 1 goes out at the start of step j and is waited for (s_waitcnt) before the
 * step's closing barrier; W goes through R register stages and the producer as in
 * k_tile_mfma (each thread makes 16 weights of two rows, t / 4 and t / 4 + 128). LDS:
 * 2 x 32 KiB of x, 2 x 32 KiB of W, the producer's table (160 KiB in all). The producer
 * must provide row_base / load_at (32-bit row offsets) and REG_WORDS. */
/* SK (CMAX > 0): Stream-K, one workgroup per range of TileSK units (blockIdx.x), the cell
 * table filled once for all of the workgroup's segments; CMAX bounds a split tile's
 * contributors. Otherwise one tile (and K split z) per workgroup. */
template <int R, class P, class Out, int CMAX = 0>
__global__ __launch_bounds__(512) void k_tile_big(P p, const uint16_t *__restrict__ x, typename Out::T *__restrict__ y,
                                                  int M, int N, int K, int kps, float *__restrict__ part,
                                                  unsigned *ctr, TileSK sk) {
    constexpr int T = 512, BM = 256, BN = 256, TM = 8, TN = 4;
    constexpr int U = (R % 2) ? 2 * R : R;
    static_assert(R >= 2 && R <= 4, "register stages");
    __shared__ float ptab[P::LDS_WORDS > 0 ? P::LDS_WORDS : 1];
    /* four separate arrays, not [2][...]: the compiler then knows the x DMA into one buffer
     * does not alias reads of the others, and does not wait for the DMA before them */
    __shared__ __attribute__((aligned(16))) uint16_t sX0[BM * TILE_LDW], sX1[BM * TILE_LDW];
    __shared__ __attribute__((aligned(16))) uint16_t sW0[BN * TILE_LDW], sW1[BN * TILE_LDW];
    auto sX = [&](int b) { return b ? sX1 : sX0; };
    auto sW = [&](int b) { return b ? sW1 : sW0; };
    /* tid, lane, wr and wq are set again at the start of every Stream-K segment from a
     * value the compiler cannot see through, so what it derives from them (LDS and row
     * offsets) is recomputed per segment instead of held live through the segment's epilogue */
    int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    /* the segment: output tile at (m0, n0), K steps [kb0, kb0 + ns), ns >= 1 */
    int m0 = 0, n0 = 0, kb0 = 0, ns = 1;
    int wr = tid >> 2, wq = tid & 3;
    glint_f32x4 acc[TM][TN];

    struct Stage {
        typename P::Regs w[2];
    };
    Stage st[R];
    uint32_t wbase[2];
    auto gload = [&](int j, Stage &sg) {
        const int kb = kb0 + min(j, ns - 1);
        p.load_at(sg.w[0], wbase[0], wq, kb);
        p.load_at(sg.w[1], wbase[1], wq, kb);
    };
    /* x DMA: wave w, instruction q covers rows 8 (4 w + q) .. +7; lane l takes row
     * 8 (4 w + q) + l / 8, LDS slot l % 8, i.e. logical chunk (l % 8) ^ f(row) */
    /* x DMA through a buffer resource (a MUBUF load with the lds bit: the compiler tracks its
     * counter precisely, where the global form makes it wait for every load to finish).
     * Wave w, instruction q covers rows 8 (4 w + q) .. +7; lane l takes row 8 (4 w + q) + l / 8,
     * LDS slot l % 8, i.e. logical chunk (l % 8) ^ f(row). Offsets in bytes: M * K * 2 < 2^32
     * (the host checks), and every row is clamped into the matrix. */
    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc((void *)x, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), GLINT_BUF_DWORD3);
    uint32_t xvo[4];
    auto xdma = [&](int j, int buf) {
        const uint32_t kb = (uint32_t)(kb0 + min(j, ns - 1));
#pragma unroll
        for (int q = 0; q < 4; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xres, (__attribute__((address_space(3))) void *)(sX(buf) + 8 * (4 * wave + q) * TILE_LDW), 16, xvo[q],
                kb * 128u, 0, 0);
    };
    auto store_row = [&](int buf, const typename P::Regs &rg, int row, const float (&v)[16]) {
        uint32_t pk[8];
        p.finish(rg, v, pk);
        *(glint_u32x4 *)(sW(buf) + tile_ofs(row, 2 * wq)) = glint_u32x4{pk[0], pk[1], pk[2], pk[3]};
        *(glint_u32x4 *)(sW(buf) + tile_ofs(row, 2 * wq + 1)) = glint_u32x4{pk[4], pk[5], pk[6], pk[7]};
    };
    /* one K slice: the 4 B fragments, then per A tile one fragment read and its 4 MFMAs, so
     * at most one A fragment is live (the accumulators hold 128 registers) */
    auto kslice = [&](int cur, int ks) {
        const int fofs = tile_ofs(lane & 15, 4 * ks + (lane >> 4));
        glint_bf16x8 bfr[TN];
#pragma unroll
        for (int b = 0; b < TN; ++b)
            bfr[b] = __builtin_bit_cast(glint_bf16x8,
                                        *(const glint_u32x4 *)(sW(cur) + (wn * TN * 16 + b * 16) * TILE_LDW + fofs));
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const glint_bf16x8 af = __builtin_bit_cast(
                glint_bf16x8, *(const glint_u32x4 *)(sX(cur) + (wm * TM * 16 + a * 16) * TILE_LDW + fofs));
#pragma unroll
            for (int b = 0; b < TN; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[b], acc[a][b], 0, 0, 0);
        }
    };
    /* step j (j % U == u): the x DMA of step j + 1 into the other buffer (last read before
     * the previous barrier); each K slice's MFMAs run while one W row of step j + 1 is looked
     * up; then W row stores, the stage refill, the wait for the DMA, the barrier */
    /* an empty asm that "redefines" a stage's registers where the step consumes them: without
     * it the compiler computes a stage's lookup indices a step early, right after its loads
     * were issued, and waits for them there */
    auto pin = [&](typename P::Regs &rg) {
        uint32_t *w = (uint32_t *)&rg;
#pragma unroll
        for (int i = 0; i < P::REG_WORDS; ++i)
            asm volatile("" : "+v"(w[i]));
    };
    auto step = [&](int j, int u) {
        const int cur = u & 1;
        Stage &nx = st[(u + 1) % R];
        xdma(j + 1, cur ^ 1);
        pin(nx.w[0]);
        pin(nx.w[1]);
        float v[16];
        p.lookup(nx.w[0], v, lane);
        kslice(cur, 0);
        store_row(cur ^ 1, nx.w[0], wr, v); /* past the end: clamped data nobody reads */
        __builtin_amdgcn_sched_barrier(0); /* keep the halves apart: registers are at the limit */
        p.lookup(nx.w[1], v, lane);
        kslice(cur, 1);
        store_row(cur ^ 1, nx.w[1], wr + 128, v);
        gload(j + 1 + R, nx);
        /* the x DMA of step j + 1 is older than the W loads just issued (two loads of
         * P::LOADS instructions): wait until only those are outstanding */
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT(2 * P::LOADS));
        __syncthreads();
    };

    /* one segment: accumulators cleared, row offsets, the pipeline filled, the K loop */
    auto run = [&]() {
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b)
                acc[a][b] = glint_f32x4{0.f, 0.f, 0.f, 0.f};
        wbase[0] = p.row_base(min(n0 + wr, N - 1));
        wbase[1] = p.row_base(min(n0 + wr + 128, N - 1));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = 8 * (4 * wave + q) + (lane >> 3);
            const int chunk = ((lane & 7) ^ (((r >> 1) ^ ((r & 1) << 2)) & 7));
            xvo[q] = ((uint32_t)min(m0 + r, M - 1) * (uint32_t)K + (uint32_t)chunk * 8u) * 2u;
        }
        xdma(0, 0);
#pragma unroll
        for (int i = 0; i < R; ++i)
            gload(i, st[i]);
        {
            float v[16];
            p.lookup(st[0].w[0], v, lane);
            store_row(0, st[0].w[0], wr, v);
            p.lookup(st[0].w[1], v, lane);
            store_row(0, st[0].w[1], wr + 128, v);
        }
        gload(R, st[0]);
        /* only the refill just issued stays outstanding: the loop then enters with the
         * counter state of its own back edge, and the compiler adds no full wait inside it */
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT(2 * P::LOADS));
        __syncthreads();
        int j = 0;
        for (; j + U <= ns; j += U) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                step(j + u, u);
        }
#pragma unroll
        for (int u = 0; u + 1 < U; ++u)
            if (j + u < ns)
                step(j + u, u);
    };
    auto store_tile = [&]() {
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
    };

    p.setup(ptab, (float *)sX1); /* sX1 is free until step 0's x DMA */
    if constexpr (CMAX == 0) {
        m0 = blockIdx.y * BM;
        n0 = blockIdx.x * BN;
        kb0 = blockIdx.z * kps;
        ns = min(K >> 6, kb0 + kps) - kb0; /* >= 1: the host sizes gridDim.z */
        run();
        if (gridDim.z > 1 && !tile_splitk_epilogue<TM, TN, T>(acc, part, ctr, *(unsigned *)sX0))
            return;
        store_tile();
    } else {
        const int g = blockIdx.x;
        int u = tile_sk_start(sk, g);
        const int u1 = tile_sk_start(sk, g + 1);
        /* at most TILE_SK_SEGS segments (the host checks), unrolled: as a loop the compiler
         * kept more values live through the K loop than the registers hold and spilled
         * inside it */
#pragma unroll
        for (int seg = 0; seg < TILE_SK_SEGS; ++seg) {
            if (u >= u1)
                break;
            const int t = u / sk.nk;
            kb0 = u - t * sk.nk;
            ns = min(sk.nk - kb0, u1 - u);
            m0 = (t / sk.gx) * BM;
            n0 = (t % sk.gx) * BN;
            u += ns;
            __syncthreads(); /* the previous segment's last LDS reads (s_flag in sX0) */
            asm volatile("" : "+v"(tid));
            lane = tid & 63;
            wr = tid >> 2;
            wq = tid & 3;
            run();
            /* again after the K loop: the epilogue's offsets are formed here, not held through it */
            asm volatile("" : "+v"(tid));
            lane = tid & 63;
            if (ns == sk.nk || tile_sk_fixup<TM, TN, T, CMAX>(acc, sk, g, t, part, ctr, *(unsigned *)sX0, tid))
                store_tile();
        }
    }
}

/* ---------------------------------------------------------- split-K host side */
#ifndef TILE_SPLIT_MIN_STEPS
#define TILE_SPLIT_MIN_STEPS 8 /* fewest 64-wide K steps per split */
#endif
#include <thread>
#include <unordered_map>

/* A split-K workspace: f32 partial tiles plus one arrival counter per output tile. The
 * counters are zero between launches: the last workgroup of each tile clears its own, so
 * a workspace stays valid as long as every launch that used it ran to completion.
 * Capacity: 2 x CUs x 65536 floats and 2 x CUs counters. The 256 x 256 tiles (65536 floats)
 * split only to fill each CU once (tiles x splits <= CUs), the 256 x 128 ones likewise, the
 * smaller ones at most 2 x CUs x 8192 floats; Stream-K takes two 256 x 256 partial slots
 * and one counter per workgroup (one workgroup per CU). tile_split_plan and
 * tile_big_sk_launch check their plans against the capacity and fall back (unsplit, or
 * whole tiles) where they would not fit. */
#define GLINT_SPLIT_TILE_FLOATS_MAX 65536
static inline size_t glint_split_ctr_bytes(size_t nctr) { return (nctr * sizeof(unsigned) + 255) & ~(size_t)255; }

/* Zero n counters on a stream (a kernel, not a memset node, so it is also safe to record
 * into a graph). */
static __global__ void k_glint_zero_u32(unsigned *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

/* The split-K workspaces of a stream on the current device: at most two, each allocated
 * once at full capacity (hipMalloc; its counters zeroed by a kernel on `st`) and never
 * grown:
 *   - the eager one, used by launches that are not being captured;
 *   - the graph one, bound by every launch captured on the stream. The first capture takes
 *     the stream's eager workspace over as the graph one (the next eager launch allocates a
 *     fresh eager one), later captures bind the same graph workspace. So replays and eager
 *     calls never share counters, graphs captured on one stream share theirs (their replays
 *     must not overlap one another), and capture -> eager cycles allocate nothing after the
 *     first.
 * A capture on a stream that has neither cannot allocate (the launch then runs unsplit):
 * make one eager call, or call the library's workspace reserve, first. `may_alloc` false:
 * return a workspace only if the stream already has one (never allocates).
 * hipStreamPerThread is keyed by host thread, since each thread's per-thread stream is a
 * different queue behind the same handle. glint_split_ws_release frees both. Returns false
 * if no workspace can be had. */
struct GlintSplitWsEntry {
    char *eager = nullptr, *graph = nullptr;
};
static inline std::mutex &glint_split_ws_mu() {
    static std::mutex mu;
    return mu;
}
static inline std::unordered_map<uint64_t, GlintSplitWsEntry> &glint_split_ws_cache() {
    static std::unordered_map<uint64_t, GlintSplitWsEntry> cache;
    return cache;
}
static inline bool glint_split_ws_key(hipStream_t st, uint64_t &key) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return false;
    key = (uint64_t)(uintptr_t)st;
    if (st == hipStreamPerThread)
        key = (uint64_t)std::hash<std::thread::id>{}(std::this_thread::get_id()) | 1u; /* handles are even */
    key = key * 131u + (uint64_t)dev;
    return true;
}
static inline size_t glint_split_ws_bytes(size_t &cb, size_t &nctr, size_t &part_floats) {
    const size_t cus = (size_t)glint_cu_count();
    nctr = 2 * cus;
    part_floats = 2 * cus * GLINT_SPLIT_TILE_FLOATS_MAX;
    cb = glint_split_ctr_bytes(nctr);
    return cb + part_floats * sizeof(float);
}
static inline bool glint_split_ws_stream(hipStream_t st, GlintSplitWs &ws, bool may_alloc = true) {
    uint64_t key = 0;
    if (!glint_split_ws_key(st, key))
        return false;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess)
        return false;
    size_t cb = 0, nctr = 0, part_floats = 0;
    const size_t bytes = glint_split_ws_bytes(cb, nctr, part_floats);
    std::lock_guard<std::mutex> lock(glint_split_ws_mu());
    GlintSplitWsEntry &e = glint_split_ws_cache()[key];
    char *base = nullptr;
    if (cap != hipStreamCaptureStatusNone) {
        if (e.graph == nullptr) {
            e.graph = e.eager; /* may be null: then the capture runs unsplit */
            e.eager = nullptr;
        }
        base = e.graph;
    } else {
        if (e.eager == nullptr && may_alloc) {
            char *b = nullptr;
            if (hipMalloc((void **)&b, bytes) != hipSuccess)
                return false;
            k_glint_zero_u32<<<1, 256, 0, st>>>((unsigned *)b, cb / sizeof(unsigned));
            if (hipGetLastError() != hipSuccess) {
                (void)hipFree(b); /* nothing was enqueued on it */
                return false;
            }
            e.eager = b;
        }
        base = e.eager;
    }
    if (base == nullptr)
        return false;
    ws = GlintSplitWs{(float *)(base + cb), (unsigned *)base, part_floats, nctr};
    return true;
}

/* Frees the stream's workspaces (after waiting for the stream). Graphs captured on the
 * stream before the call must not be replayed after it. Not during capture. Returns 0, -1
 * if the stream is capturing or the runtime fails. */
static inline int glint_split_ws_release(hipStream_t st) {
    uint64_t key = 0;
    if (!glint_split_ws_key(st, key))
        return -1;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
        return -1;
    if (hipStreamSynchronize(st) != hipSuccess)
        return -1;
    GlintSplitWsEntry e;
    {
        std::lock_guard<std::mutex> lock(glint_split_ws_mu());
        auto it = glint_split_ws_cache().find(key);
        if (it == glint_split_ws_cache().end())
            return 0;
        e = it->second;
        glint_split_ws_cache().erase(it);
    }
    int rc = 0;
    if (e.eager && hipFree(e.eager) != hipSuccess)
        rc = -1;
    if (e.graph && hipFree(e.graph) != hipSuccess)
        rc = -1;
    return rc;
}

/* Splits of K for a grid of `tiles` output tiles when `slots` workgroups should run at
 * once: enough to fill the slots, each split at least `min_steps` of the nK K steps.
 * Returns the steps per split (kps); the grid's z extent is ceil(nK / kps). */
static inline int glint_split_kps(int64_t tiles, int64_t slots, int nK, int min_steps) {
    int64_t ks = tiles > 0 ? slots / tiles : 1;
    ks = std::min<int64_t>(std::min<int64_t>(ks, TILE_SPLIT_MAX), nK / std::max(min_steps, 1));
    if (ks <= 1)
        return nK;
    return (int)((nK + ks - 1) / ks);
}

/* Split plan for a gx x gy tile grid over nS K steps: fills the CUs once (a second resident
 * workgroup per CU measured slower: they contend for the LDS). Sets kps and ks and the
 * workspace: the caller's `fixed` one if given, else the stream's. A split that does not
 * fit the workspace, or a stream without one (capture), runs unsplit; with a `fixed`
 * workspace that is too small the plan is refused instead (returns false), so the caller
 * can report it. */
static inline bool tile_split_plan(hipStream_t st, unsigned gx, unsigned gy, int nS, size_t tile_floats, int &kps,
                                   int &ks, GlintSplitWs &ws, int per_cu = 1, const GlintSplitWs *fixed = nullptr) {
    const int64_t tiles = (int64_t)gx * gy;
    kps = glint_split_kps(tiles, (int64_t)per_cu * glint_cu_count(), nS, TILE_SPLIT_MIN_STEPS);
    ks = (nS + kps - 1) / kps;
    ws = GlintSplitWs{nullptr, nullptr, 0, 0};
    if (ks <= 1)
        return true;
    const bool got = fixed ? (ws = *fixed, true) : glint_split_ws_stream(st, ws);
    const bool fits = got && (size_t)ks * tiles * tile_floats <= ws.part_floats && (size_t)tiles <= ws.nctr;
    if (!fits) {
        if (fixed)
            return false;
        kps = nS;
        ks = 1;
        ws = GlintSplitWs{nullptr, nullptr, 0, 0};
    }
    return true;
}

/* Launch k_tile_mfma over an M x N output. K % 64 == 0, M, N >= 1. */
/* Each launcher returns false, launching nothing, only when a `fixed` workspace is too
 * small for the split plan. */
template <int BM, int BN, int WM, int WN, int R, class P, class Out, int NP = 1>
static bool tile_mfma_launch(const P &p, const uint16_t *x, typename Out::T *y, int M, int N, int K, hipStream_t st,
                             const GlintSplitWs *fixed = nullptr) {
    static_assert(BM * BN <= GLINT_SPLIT_TILE_FLOATS_MAX, "split workspace capacity");
    const unsigned gx = (unsigned)((N + BN - 1) / BN), gy = (unsigned)((M + BM - 1) / BM);
    int kps, ks;
    GlintSplitWs ws;
    if (!tile_split_plan(st, gx, gy, K >> 6, (size_t)BM * BN, kps, ks, ws, 1, fixed))
        return false;
    k_tile_mfma<BM, BN, WM, WN, R, P, Out, NP><<<dim3(gx, gy, (unsigned)ks), 64 * WM * WN, 0, st>>>(
        p, x, y, M, N, K, kps, ws.part, ws.ctr);
    return true;
}

/* Launch k_tile_big over an M x N output. K % 64 == 0, M, N >= 1, M * K < 2^31 and
 * N * K < 2^36 (its 32-bit offsets; tile_big_fits). */
static inline bool tile_big_fits(int M, int N, int K) {
    return (int64_t)M * K < ((int64_t)1 << 31) && (int64_t)N * K < ((int64_t)1 << 36);
}
#ifndef TILE_BIG
#define TILE_BIG 1 /* M >= 256 may take the 256 x 256 k_tile_big (tile_big_pays) */
#endif
/* The 256 x 256 tile beats the 256 x 128 one once it has about 3/4 of a tile per CU (measured
 * at M = 512 .. 8192 on the 14336 x 4096 and 4096 x 14336 shapes: 9-14% faster there, up to
 * 1.8x slower with fewer tiles, where split K cannot fill the device as well). */
static inline bool tile_big_pays(int M, int N) {
    return (int64_t)((M + 255) / 256) * ((N + 255) / 256) * 4 >= (int64_t)3 * glint_cu_count();
}
template <int R, class P, class Out>
static bool tile_big_launch(const P &p, const uint16_t *x, typename Out::T *y, int M, int N, int K, hipStream_t st,
                            const GlintSplitWs *fixed = nullptr) {
    const unsigned gx = (unsigned)((N + 255) / 256), gy = (unsigned)((M + 255) / 256);
    int kps, ks;
    GlintSplitWs ws;
    if (!tile_split_plan(st, gx, gy, K >> 6, (size_t)256 * 256, kps, ks, ws, 1, fixed))
        return false;
    k_tile_big<R, P, Out><<<dim3(gx, gy, (unsigned)ks), 512, 0, st>>>(p, x, y, M, N, K, kps, ws.part, ws.ctr,
                                                                       TileSK{0, 1, 1, 1});
    return true;
}

/* Where the 256 x 256 tiles are too few to pay on their own but split K makes them fill
 * every CU exactly once (4096 x 14336 at M = 1024: 64 tiles x 4 splits; M = 2048: 128 x 2),
 * k_tile_big with split K beats k_tile_mfma's 256 x 128 tiles by 7-8%; where the split
 * leaves CUs idle it loses (M = 512 on either shape). */
static inline bool tile_big_split_fills(int M, int N, int K) {
    const int64_t tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    const int kps = glint_split_kps(tiles, glint_cu_count(), K >> 6, TILE_SPLIT_MIN_STEPS);
    const int64_t ks = ((K >> 6) + kps - 1) / kps;
    return ks > 1 && tiles * ks == glint_cu_count();
}
/* k_tile_big split as tile_big_split_fills plans it; launches nothing and returns false if
 * the plan does not come out split (no workspace, or `fixed` too small), so the caller can
 * take the 256 x 128 tiles instead. */
template <int R, class P, class Out>
static bool tile_big_split_launch(const P &p, const uint16_t *x, typename Out::T *y, int M, int N, int K,
                                  hipStream_t st, const GlintSplitWs *fixed = nullptr) {
    const unsigned gx = (unsigned)((N + 255) / 256), gy = (unsigned)((M + 255) / 256);
    int kps, ks;
    GlintSplitWs ws;
    if (!tile_split_plan(st, gx, gy, K >> 6, (size_t)256 * 256, kps, ks, ws, 1, fixed) || ks <= 1)
        return false;
    k_tile_big<R, P, Out><<<dim3(gx, gy, (unsigned)ks), 512, 0, st>>>(p, x, y, M, N, K, kps, ws.part, ws.ctr,
                                                                       TileSK{0, 1, 1, 1});
    return true;
}

/* Stream-K k_tile_big (TileSK): one workgroup per CU over the 256 x 256 tiles' units. */
#ifndef TILE_SK
#define TILE_SK 1 /* 0: never Stream-K; 1: where tile_sk_pays; 2: wherever it can run */
#endif
#define TILE_SK_CMAX 4 /* most workgroups sharing one tile */
/* cmax: the most workgroups one tile can have; segs: the most tiles one workgroup touches
 * (both 0 where units >= 2^31: no plan) */
static inline TileSK tile_sk_plan(int64_t tiles, int nk, int gx, int &cmax, int &segs) {
    const int64_t units = tiles * nk;
    if (units >= ((int64_t)1 << 31) || units < 1) {
        cmax = segs = 0;
        return TileSK{0, 1, 1, 1};
    }
    const int wgs = (int)std::min<int64_t>(glint_cu_count(), units);
    /* ranges are floor(units / wgs) or one more units long: nk units meet at most cmax of
     * them, and a range meets at most segs tiles */
    const int64_t len = units / wgs, len_max = (units + wgs - 1) / wgs;
    cmax = (int)((nk - 1 + len - 1) / len) + 1;
    segs = (int)((len_max - 1 + nk - 1) / nk) + 1;
    return TileSK{(int)units, wgs, nk, gx};
}
/* Share of the CUs a launch of `wgs` workgroups (one resident per CU, equal work) keeps
 * busy on average over its rounds. */
static inline double tile_fill(int64_t wgs) {
    const int64_t cus = glint_cu_count(), rounds = (wgs + cus - 1) / cus;
    return (double)wgs / (double)(rounds * cus);
}
/* Stream-K against the whole-tile plans the dispatch would otherwise take. Measured on the
 * 14336 x 4096 and 4096 x 14336 shapes (6 rotated weight copies, one box): a Stream-K K
 * step costs about 1.2x a whole-tile one, mostly the split tiles' f32 partials going
 * through memory, so it wins only where the whole tiles leave many CUs idle. M = 1536 gate
 * (336 tiles, 66% fill) 261 -> 219 us; M = 1536 down (192 256 x 128 tiles, 75%) 257 -> 214
 * us. It lost at 87.5% fill: M = 1024 gate 137 -> 150 us, M = 2048 gate 268 -> 274 us
 * (448 tiles), M = 512 gate 92 -> 102 us against the 256 x 128 tiles; and it gains nothing
 * where a K split already fills the CUs exactly (M = 1024 and 2048 down). */
static inline bool tile_sk_pays(int M, int N, int K) {
    if (TILE_SK == 2)
        return true;
    const int64_t big = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    if (tile_big_pays(M, N))
        return tile_fill(big) < 0.7;
    if (tile_big_split_fills(M, N, K))
        return false;
    /* the 256 x 128 tiles with their K split */
    const int64_t t2 = (int64_t)((M + 255) / 256) * ((N + 127) / 128);
    const int kps = glint_split_kps(t2, glint_cu_count(), K >> 6, TILE_SPLIT_MIN_STEPS);
    return tile_fill(t2 * (((K >> 6) + kps - 1) / kps)) < 0.8;
}
/* Launches Stream-K k_tile_big; returns false, launching nothing, where the plan does not
 * fit (more than TILE_SK_CMAX workgroups per tile or TILE_SK_SEGS tiles per workgroup, or
 * a workspace short of 2 partial tiles per workgroup: a stream being captured without one,
 * or a `fixed` one that is too small), so the caller takes the whole-tile launch. */
template <int R, class P, class Out>
static bool tile_big_sk_launch(const P &p, const uint16_t *x, typename Out::T *y, int M, int N, int K, hipStream_t st,
                               const GlintSplitWs *fixed = nullptr) {
    const int gx = (N + 255) / 256, gy = (M + 255) / 256;
    int cmax = 0, segs = 0;
    const TileSK sk = tile_sk_plan((int64_t)gx * gy, K >> 6, gx, cmax, segs);
    if (cmax < 1 || cmax > TILE_SK_CMAX || segs > TILE_SK_SEGS)
        return false;
    GlintSplitWs ws;
    const bool got = fixed ? (ws = *fixed, true) : glint_split_ws_stream(st, ws);
    if (!got || (size_t)2 * sk.wgs * (256 * 256) > ws.part_floats || (size_t)sk.wgs > ws.nctr)
        return false;
    if (cmax <= 2)
        k_tile_big<R, P, Out, 2><<<sk.wgs, 512, 0, st>>>(p, x, y, M, N, K, 0, ws.part, ws.ctr, sk);
    else
        k_tile_big<R, P, Out, TILE_SK_CMAX><<<sk.wgs, 512, 0, st>>>(p, x, y, M, N, K, 0, ws.part, ws.ctr, sk);
    return true;
}

/* Launch k_tile_ss over an M x N output. K % 64 == 0, M, N >= 1. */
template <int BM, int BN, int RX, class P, class Out>
static bool tile_ss_launch(const P &p, const uint16_t *x, typename Out::T *y, int M, int N, int K, hipStream_t st,
                           int per_cu = 1, const GlintSplitWs *fixed = nullptr) {
    const unsigned gx = (unsigned)((N + BN - 1) / BN), gy = (unsigned)((M + BM - 1) / BM);
    int kps, ks;
    GlintSplitWs ws;
    if (!tile_split_plan(st, gx, gy, K >> 6, (size_t)BM * BN, kps, ks, ws, per_cu, fixed))
        return false;
    k_tile_ss<BM, BN, RX, P, Out><<<dim3(gx, gy, (unsigned)ks), 256, 0, st>>>(p, x, y, M, N, K, kps, ws.part, ws.ctr);
    return true;
}

#endif
