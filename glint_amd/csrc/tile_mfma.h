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
 *   LDS_WORDS, setup(float *lds)                  LDS the producer needs (filled before step 0)
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

/* s_waitcnt immediate for vmcnt(0) alone (gfx9 encoding: vmcnt [3:0] and [15:14] = 0,
 * expcnt [6:4] and lgkmcnt [11:8] at their maxima). On gfx9 stores count in vmcnt too. */
#define GLINT_WAIT_VMCNT0 0x0F70
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
    /* v[8 q + 2 b] / v[8 q + 2 b + 1]: cells of the even / odd element of byte b of word q */
    __device__ __forceinline__ void lookup(const Regs &r, float (&v)[16], int lane) const {
        const uint32_t lb = lane & 31;
        const uint32_t H[2] = {r.h.x, r.h.y}, P[2] = {r.p.x, r.p.y};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t E = glint_codes_even(H[q], P[q]);
            const uint32_t O = glint_codes_odd(H[q], P[q]);
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
};

template <int BM, int BN, int WM, int WN, int R, class P, class Out>
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
    __shared__ float ptab[P::LDS_WORDS > 0 ? P::LDS_WORDS : 1];
    __shared__ __attribute__((aligned(16))) uint16_t sX[2][BM * TILE_LDW];
    __shared__ __attribute__((aligned(16))) uint16_t sW[2][BN * TILE_LDW];
    __shared__ unsigned s_last;
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
        uint32_t packed[8];
        p.finish(sg.w, v, packed);
        *(glint_u32x4 *)(sW[buf] + tile_ofs(wr, 2 * wq)) = glint_u32x4{packed[0], packed[1], packed[2], packed[3]};
        *(glint_u32x4 *)(sW[buf] + tile_ofs(wr, 2 * wq + 1)) = glint_u32x4{packed[4], packed[5], packed[6], packed[7]};
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
        glint_bf16x8 af[2][TM], bfr[2][TN];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            /* rows (16-row tile base) + lane % 16, chunk 4 ks + lane / 16; the swizzle does not
             * change when a row moves by a multiple of 16 */
            const int fofs = tile_ofs(lane & 15, 4 * ks + (lane >> 4));
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[ks][a] = __builtin_bit_cast(
                    glint_bf16x8, *(const glint_u32x4 *)(sX[cur] + (wm * TM * 16 + a * 16) * TILE_LDW + fofs));
#pragma unroll
            for (int b = 0; b < TN; ++b)
                bfr[ks][b] = __builtin_bit_cast(
                    glint_bf16x8, *(const glint_u32x4 *)(sW[cur] + (wn * TN * 16 + b * 16) * TILE_LDW + fofs));
        }
        float v[16];
        p.lookup(nx.w, v, lane);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[ks][a], bfr[ks][b], acc[a][b], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        store(cur ^ 1, nx, v); /* past the end: a clamped copy nobody reads */
        gload(j + 1 + R, nx);
        __syncthreads();
    };

    p.setup(ptab);
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

    if (gridDim.z > 1) {
        /* Partials and counters are accessed with device-scope relaxed atomics, which are
         * coherent across the XCDs' separate L2 caches without the L2 write-back and
         * invalidate that device-scope fences cost. Ordering: a workgroup's partial stores
         * have completed (vmcnt 0) before the barrier that precedes its counter increment,
         * and the reducer issues its partial loads after it has seen the final count.
         * Partial element e of thread t sits at e T + t. */
        const unsigned tile = blockIdx.y * gridDim.x + blockIdx.x;
        const size_t tsz = (size_t)BM * BN, zstride = (size_t)gridDim.x * gridDim.y * tsz;
        float *mine = part + blockIdx.z * zstride + tile * tsz;
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    __hip_atomic_store(mine + ((a * TN + b) * 4 + i) * T + tid, acc[a][b][i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0);
        __syncthreads();
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(&ctr[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     gridDim.z - 1;
        __syncthreads();
        if (!s_last)
            return;
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
                const int e = c0 + c, a = e / (TN * 4), b = (e / 4) % TN, i = e % 4;
                float s = blockIdx.z == 0 ? acc[a][b][i] : v[0][c];
#pragma unroll
                for (int z = 1; z < TILE_SPLIT_MAX; ++z)
                    if ((unsigned)z <= zl)
                        s += (unsigned)z == blockIdx.z ? acc[a][b][i] : v[z][c];
                acc[a][b][i] = s;
            }
        }
        if (tid == 0)
            __hip_atomic_store(&ctr[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
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

/* ---------------------------------------------------------- split-K host side */
#ifndef TILE_SPLIT_MIN_STEPS
#define TILE_SPLIT_MIN_STEPS 8 /* fewest 64-wide K steps per split */
#endif
#include <unordered_map>

/* Per (device, stream) split-K workspace: partial tiles plus arrival counters that are zero
 * between launches. Launches on one stream run in order, so they can share it; launches
 * on different streams get different ones. Growing it frees the old buffer (hipFree waits
 * for the device) and zeroes the new counters with a blocking hipMemset, so a stream
 * being captured into a graph cannot grow it: glint_split_ws then returns false and the
 * caller runs without splitting. */
struct GlintSplitWs {
    float *part;
    unsigned *ctr;
};
static inline bool glint_split_ws(hipStream_t st, size_t part_floats, size_t ntiles, GlintSplitWs &ws) {
    struct Entry {
        char *base;
        size_t part_floats, ntiles;
    };
    static std::mutex mu;
    static std::unordered_map<uint64_t, Entry> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return false;
    const uint64_t key = (uint64_t)(uintptr_t)st * 64u + (uint64_t)dev;
    std::lock_guard<std::mutex> lock(mu);
    Entry &e = cache[key];
    if (e.base == nullptr || e.part_floats < part_floats || e.ntiles < ntiles) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
            return false;
        const size_t pf = std::max(part_floats, e.part_floats), nt = std::max(ntiles, e.ntiles);
        const size_t ctr_bytes = (nt * sizeof(unsigned) + 255) & ~(size_t)255;
        if (e.base != nullptr && (hipStreamSynchronize(st) != hipSuccess || hipFree(e.base) != hipSuccess))
            return false;
        e = Entry{nullptr, 0, 0};
        char *b = nullptr;
        if (hipMalloc((void **)&b, ctr_bytes + pf * sizeof(float)) != hipSuccess)
            return false;
        if (hipMemset(b, 0, ctr_bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
            (void)hipFree(b);
            return false;
        }
        e = Entry{b, pf, nt};
    }
    const size_t ctr_bytes = (e.ntiles * sizeof(unsigned) + 255) & ~(size_t)255;
    ws.ctr = (unsigned *)e.base;
    ws.part = (float *)(e.base + ctr_bytes);
    return true;
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

/* Launch k_tile_mfma over an M x N output, splitting K when the tiles alone would leave
 * resident slots idle. K % 64 == 0, M, N >= 1. */
template <int BM, int BN, int WM, int WN, int R, class P, class Out>
static void tile_mfma_launch(const P &p, const uint16_t *x, typename Out::T *y, int M, int N, int K, hipStream_t st) {
    constexpr int T = 64 * WM * WN;
    auto kern = k_tile_mfma<BM, BN, WM, WN, R, P, Out>;
    const int nS = K >> 6; /* 64-wide K steps */
    const unsigned gx = (unsigned)((N + BN - 1) / BN), gy = (unsigned)((M + BM - 1) / BM);
    const int64_t tiles = (int64_t)gx * gy;
    /* one workgroup per CU: a second resident workgroup measured slower (they contend for
     * the LDS), so the split count aims at filling the CUs once */
    int kps = glint_split_kps(tiles, glint_cu_count(), nS, TILE_SPLIT_MIN_STEPS);
    int ks = (nS + kps - 1) / kps;
    GlintSplitWs ws{nullptr, nullptr};
    if (ks > 1 && !glint_split_ws(st, (size_t)ks * tiles * BM * BN, (size_t)tiles, ws)) {
        kps = nS;
        ks = 1;
    }
    kern<<<dim3(gx, gy, (unsigned)ks), T, 0, st>>>(p, x, y, M, N, K, kps, ws.part, ws.ctr);
}

#endif
