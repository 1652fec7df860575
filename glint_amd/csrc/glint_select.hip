/* K-major decode path for gfx950: layout conversion, parent-only (fold) GEMV, channel
 * selection and the selected-plug correction (reference mojo/p7_glint_gemv_km.mojo,
 * mojo/p7_select_device.mojo, mojo/p7_glint_select_decode.mojo; semantics in
 * include/glint_select.h).
 *
 * k_kmajor_pack_planes — 64 rows x 64 channels per workgroup through LDS: 8-byte loads of
 *   the row-major planes, 4-byte stores of the K-major rows.
 * k_gemv_km_fold — a lane owns KM_FOLD_RPL = 8 output rows (4 B of a K-major hole row), so
 *   a wave reads 256 B contiguous per channel; the 8 waves of a workgroup take 8 parts of the
 *   workgroup's channel slice (grid.y) and meet in LDS; the slices of a row block meet in
 *   the last of its workgroups to finish (arrival counters), in slice order. Per element:
 *   one v_perm for the
 *   address, one lookup in the 64-copy PARENT table, one FMA by the wave-uniform x[c];
 *   the block scale is applied once per run of channels inside a 64-block.
 * k_select_topk — one workgroup: keys in LDS, rank thresholds by a two-level radix select
 *   (LDS histograms of the top 8 and low 7 key bits), the price / relational / floor rules,
 *   then a block scan that writes the kept channels in ascending order.
 * k_apply_corr_km — the fold kernel's mapping (KM_CORR_RPL = 8 rows per lane) over the
 *   selected list (count read on the device), with the 256-entry delta table
 *   (CELLS - PARENT) in 64 lane copies.
 */
#include <algorithm>
#include <type_traits>

#include "glint_common.h"
#include "glint_select.h"

static __constant__ float kParent[16] = GLINT_PARENT_INIT;

#define KM_T 256

/* ------------------------------------------------------------------- layout */
#define KP_ROWS 64
#define KP_LDS_ROW 36 /* 32 bytes of a row's 64 channels + 4 bytes of padding */

/* Workgroup (channel tile c0 = 64 bx, row tile r0 = 64 by). Load: thread t reads bytes
 * [c0/2 + 8 (t % 4), +8) of row r0 + t / 4 of both planes. Store: thread t writes the
 * K-major bytes [(r0 + 16 (t % 4)) / 2, +8) of channel c0 + t / 4. */
__global__ __launch_bounds__(KM_T) void k_kmajor_pack_planes(const uint8_t *__restrict__ hole,
                                                             const uint8_t *__restrict__ plug,
                                                             uint8_t *__restrict__ hole_k, uint8_t *__restrict__ plug_k,
                                                             int N, int K) {
    __shared__ uint8_t th[KP_ROWS * KP_LDS_ROW], tp[KP_ROWS * KP_LDS_ROW];
    const int t = threadIdx.x;
    const int c0 = blockIdx.x * 64, r0 = blockIdx.y * KP_ROWS;
    {
        const int row = t >> 2, q = t & 3;
        uint2 vh = make_uint2(0u, 0u), vp = vh;
        if (r0 + row < N) {
            const int64_t off = ((int64_t)(r0 + row) * K + c0) / 2 + 8 * q;
            vh = *(const uint2 *)(hole + off);
            vp = *(const uint2 *)(plug + off);
        }
        *(uint32_t *)(th + row * KP_LDS_ROW + 8 * q) = vh.x;
        *(uint32_t *)(th + row * KP_LDS_ROW + 8 * q + 4) = vh.y;
        *(uint32_t *)(tp + row * KP_LDS_ROW + 8 * q) = vp.x;
        *(uint32_t *)(tp + row * KP_LDS_ROW + 8 * q + 4) = vp.y;
    }
    __syncthreads();
    const int cc = t >> 2, q = t & 3;
    const int rb = 16 * q; /* first of this thread's 16 rows in the tile */
    if (r0 + rb >= N)
        return;
    uint32_t oh[2] = {0u, 0u}, op[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int sh = 4 * (cc & 1);
        const uint32_t h = (th[(rb + i) * KP_LDS_ROW + (cc >> 1)] >> sh) & 15u;
        const uint32_t p = (tp[(rb + i) * KP_LDS_ROW + (cc >> 1)] >> sh) & 15u;
        oh[i >> 3] |= h << (4 * (i & 7));
        op[i >> 3] |= p << (4 * (i & 7));
    }
    /* 4-byte stores: a K-major row is N / 2 bytes, a multiple of 4 (N % 8 == 0) */
    const int64_t dst = (int64_t)(c0 + cc) * (N / 2) + (r0 + rb) / 2;
    *(uint32_t *)(hole_k + dst) = oh[0];
    *(uint32_t *)(plug_k + dst) = op[0];
    if (r0 + rb + 16 <= N) { /* else the matrix ends after 8 of the 16 rows */
        *(uint32_t *)(hole_k + dst + 4) = oh[1];
        *(uint32_t *)(plug_k + dst + 4) = op[1];
    }
}

__global__ __launch_bounds__(KM_T) void k_kmajor_scales(const float *__restrict__ absmax, float *__restrict__ scales_k,
                                                        int N, int nb) {
    const int64_t total = (int64_t)N * nb, stride = (int64_t)gridDim.x * KM_T;
    for (int64_t o = (int64_t)blockIdx.x * KM_T + threadIdx.x; o < total; o += stride) {
        const int64_t cb = o / N, r = o % N;
        scales_k[o] = absmax[r * nb + cb];
    }
}

/* ------------------------------------------------------------------ fold GEMV */
#define KM_SUB 8                /* waves per workgroup = parts of a channel slice */
#define KM_WG (64 * KM_SUB)
#ifndef KM_U
#define KM_U 4 /* channels per batch (two batches in flight per wave); a multiple of 4 dividing 64 */
#endif
static_assert(KM_U % 4 == 0 && 64 % KM_U == 0, "fold batch");
#ifndef KM_FOLD_RPL
#define KM_FOLD_RPL 8 /* fold: output rows per lane (8, 16 or 32) */
#endif
#ifndef KM_CORR_RPL
#define KM_CORR_RPL 8 /* correction: output rows per lane (8, 16 or 32) */
#endif

__device__ __forceinline__ float km_bf16(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

/* RPL consecutive floats (this lane's rows of one scale row) */
template <int RPL>
__device__ __forceinline__ void km_load(const float *__restrict__ p, float (&v)[RPL]) {
#pragma unroll
    for (int i = 0; i < RPL / 4; ++i) {
        const glint_f32x4 t = *(const glint_f32x4 *)(p + 4 * i);
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}

/* acc[j] = fmaf(table[code of row j], xv, acc[j]) for this lane's RPL rows. E[q]/O[q] hold
 * the code bytes of the even/odd rows of word q (byte k -> rows 8 q + 2k, 8 q + 2k + 1).
 * All RPL lookups are issued before the first FMA (sched_barrier), so their LDS latencies
 * overlap instead of each FMA waiting for its own lookup. */
template <int RPL>
__device__ __forceinline__ void km_lookup_fma(const float *lds, const uint32_t (&E)[RPL / 8],
                                              const uint32_t (&O)[RPL / 8], uint32_t lane4, float xv,
                                              float (&acc)[RPL]) {
    float tv[RPL];
#pragma unroll
    for (int q = 0; q < RPL / 8; ++q) {
        tv[8 * q + 0] = glint_lds_f32(lds, glint_cell_addr<0>(E[q], lane4));
        tv[8 * q + 1] = glint_lds_f32(lds, glint_cell_addr<0>(O[q], lane4));
        tv[8 * q + 2] = glint_lds_f32(lds, glint_cell_addr<1>(E[q], lane4));
        tv[8 * q + 3] = glint_lds_f32(lds, glint_cell_addr<1>(O[q], lane4));
        tv[8 * q + 4] = glint_lds_f32(lds, glint_cell_addr<2>(E[q], lane4));
        tv[8 * q + 5] = glint_lds_f32(lds, glint_cell_addr<2>(O[q], lane4));
        tv[8 * q + 6] = glint_lds_f32(lds, glint_cell_addr<3>(E[q], lane4));
        tv[8 * q + 7] = glint_lds_f32(lds, glint_cell_addr<3>(O[q], lane4));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < RPL; ++j)
        acc[j] = fmaf(tv[j], xv, acc[j]);
}

/* The workgroup's KM_SUB part sums meet in LDS and are added in order (row sum v of row
 * r0 + rr). One slice (nsl == 1): y[r] = v, plus y[r] first when ADD. Several slices, no
 * ctr: v goes to part[sl N + r] and k_km_combine adds the slices. Several with ctr: the
 * slices meet in the last workgroup of the row block to arrive. Each stores v to
 * part[sl N + r] with device-coherent stores, all complete before the barrier ahead of its
 * counter increment; the last one adds the slices' rows in slice order (its own from LDS),
 * as k_km_combine does, adds y when ADD, stores y and sets ctr[bx] back to zero. */
template <bool ADD, int RPL>
__device__ __forceinline__ void km_finish(float *lds, const float (&tot)[RPL], int r0, int N, float *__restrict__ y,
                                          float *__restrict__ part, unsigned *ctr, int nsl, int sl) {
    constexpr int ROWS = 64 * RPL;
    __shared__ unsigned s_last;
    const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
    __syncthreads(); /* the lookup table is dead: the part sums go over it */
#pragma unroll
    for (int i = 0; i < RPL / 4; ++i)
        *(glint_f32x4 *)(lds + q * ROWS + RPL * lane + 4 * i) =
            glint_f32x4{tot[4 * i], tot[4 * i + 1], tot[4 * i + 2], tot[4 * i + 3]};
    __syncthreads();
    for (int rr = threadIdx.x; rr < ROWS; rr += KM_WG) {
        if (r0 + rr >= N)
            break;
        float v = lds[rr];
#pragma unroll
        for (int k = 1; k < KM_SUB; ++k)
            v = v + lds[k * ROWS + rr];
        if (nsl == 1)
            y[r0 + rr] = ADD ? y[r0 + rr] + v : v;
        else if (!ctr)
            part[(int64_t)sl * N + r0 + rr] = v;
        else {
            lds[rr] = v; /* only this thread reads lds[rr] again */
            __hip_atomic_store(part + (int64_t)sl * N + r0 + rr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (nsl == 1 || !ctr)
        return;
    __builtin_amdgcn_s_waitcnt(GLINT_WAIT_VMCNT0);
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(&ctr[blockIdx.x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)nsl - 1u;
    __syncthreads();
    if (!s_last)
        return;
    for (int rr = threadIdx.x; rr < ROWS; rr += KM_WG) {
        if (r0 + rr >= N)
            break;
        const float own = lds[rr];
        const float *col = part + r0 + rr;
        float acc = 0.f;
        for (int s0 = 0; s0 < nsl; s0 += 8) { /* 8 slices' loads in flight, added in order */
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                v[i] = __hip_atomic_load(col + (int64_t)min(s0 + i, nsl - 1) * N, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int s = s0 + i;
                if (s < nsl) {
                    const float t = s == sl ? own : v[i];
                    acc = s == 0 ? t : acc + t;
                }
            }
        }
        y[r0 + rr] = ADD ? y[r0 + rr] + acc : acc;
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(&ctr[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Workgroup (row block bx, channel slice by): wave q walks part q of the slice as runs of
 * channels inside one 64-block; out[by N + r] (y when there is one slice) = the slice's
 * sum for row r. N % 32 == 0; rows of lanes past N are clamped and not stored. */
template <int RPL>
__global__ __launch_bounds__(KM_WG) void k_gemv_km_fold(const uint8_t *__restrict__ hole_bytes,
                                                        const float *__restrict__ scales_k,
                                                        const uint16_t *__restrict__ x, float *__restrict__ y,
                                                        float *__restrict__ part, unsigned *ctr, int N, int ksl) {
    constexpr int ROWS = 64 * RPL, NW = RPL / 8; /* rows per workgroup, code words per lane */
    using HV = typename std::conditional<RPL == 32, glint_u32x4,
                                         typename std::conditional<RPL == 16, glint_u32x2, uint32_t>::type>::type;
    static_assert(RPL == 8 || RPL == 16 || RPL == 32, "rows per lane");
    static_assert(KM_SUB * ROWS >= 16 * 64, "PARENT table fits the part buffer");
    const HV *__restrict__ hole_k = (const HV *)hole_bytes;
    __shared__ __attribute__((aligned(16))) float lds[KM_SUB * ROWS]; /* PARENT table at offset 0, then parts */
    for (int i = threadIdx.x; i < 16 * 64; i += KM_WG)
        lds[i] = kParent[i >> 6];
    __syncthreads();
    const int lane = threadIdx.x & 63, q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane4 = (uint32_t)lane * 4u;
    const int r0 = blockIdx.x * ROWS;
    const int rc = min(r0 + RPL * lane, N - RPL); /* this lane's first row, clamped */
    const int64_t rowv = N / RPL;                 /* RPL / 2-byte vectors per K-major row */
    const int sub = ksl / KM_SUB;
    const int c0 = blockIdx.y * ksl + q * sub, c1 = c0 + sub;
    float tot[RPL], acc[RPL], sc[RPL];
#pragma unroll
    for (int j = 0; j < RPL; ++j)
        tot[j] = 0.f;
    /* Batches of KM_U channels (a batch never crosses a 64-block: parts are multiples of
     * KM_U and blocks multiples of 64), the next batch's loads in flight while this one is
     * looked up. A run is the batches of one block: acc restarts at its first batch and is
     * folded into tot by the block scale after its last, in channel order. */
    auto load_batch = [&](int c, HV (&wv)[KM_U]) {
        c = min(c, c1 - KM_U); /* past the part: a clamped reload nobody uses */
#pragma unroll
        for (int u = 0; u < KM_U; ++u)
            wv[u] = __builtin_nontemporal_load(&hole_k[(int64_t)(c + u) * rowv + rc / RPL]);
    };
    HV wa[KM_U], wb[KM_U];
    auto batch = [&](int c, const HV (&wv)[KM_U]) {
        if (c == c0 || (c & 63) == 0) { /* a run starts: its block scales, acc from zero */
            km_load<RPL>(scales_k + (int64_t)(c >> 6) * N + rc, sc);
#pragma unroll
            for (int j = 0; j < RPL; ++j)
                acc[j] = 0.f;
        }
        /* the batch's KM_U x values in wave-uniform 8-B loads, waited for once before the
         * lookups (a scalar load per channel would make every lookup wait for it) */
        uint32_t xs[KM_U / 2];
#pragma unroll
        for (int k = 0; k < KM_U / 4; ++k) {
            const glint_u32x2 xw = *(const glint_u32x2 *)(x + c + 4 * k);
            xs[2 * k] = xw.x;
            xs[2 * k + 1] = xw.y;
        }
#pragma unroll
        for (int u = 0; u < KM_U; ++u) {
            const float xv = (u & 1) ? glint_bf16hi(xs[u >> 1]) : glint_bf16lo(xs[u >> 1]);
            uint32_t W[NW];
            __builtin_memcpy(W, &wv[u], sizeof(W));
            uint32_t E[NW], O[NW];
#pragma unroll
            for (int q = 0; q < NW; ++q) {
                E[q] = W[q] & 0x0F0F0F0Fu;
                O[q] = (W[q] >> 4) & 0x0F0F0F0Fu;
            }
            km_lookup_fma<RPL>(lds, E, O, lane4, xv, acc);
        }
        if (c + KM_U == c1 || ((c + KM_U) & 63) == 0) { /* the run ends */
#pragma unroll
            for (int j = 0; j < RPL; ++j)
                tot[j] = fmaf(acc[j], sc[j], tot[j]);
        }
    };
    load_batch(c0, wa);
    int c = c0;
    for (; c + 2 * KM_U <= c1; c += 2 * KM_U) {
        load_batch(c + KM_U, wb);
        batch(c, wa);
        load_batch(c + 2 * KM_U, wa);
        batch(c + KM_U, wb);
    }
    if (c < c1)
        batch(c, wa);
    km_finish<false, RPL>(lds, tot, r0, N, y, part, ctr, gridDim.y, blockIdx.y);
}

/* y[r] = ((part[r] + part[N + r]) + ...) + part[(ks - 1) N + r], plus y[r] first when ADD. */
template <bool ADD>
__global__ __launch_bounds__(KM_T) void k_km_combine(const float *__restrict__ part, float *__restrict__ y, int N, int ks) {
    const int r = blockIdx.x * KM_T + threadIdx.x;
    if (r >= N)
        return;
    /* slices in groups of 8 with all 8 loads in flight, added in slice order */
    float acc = part[r];
    int s = 1;
    for (; s + 8 <= ks; s += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = part[(int64_t)(s + i) * N + r];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            acc = acc + v[i];
    }
    for (; s < ks; ++s)
        acc = acc + part[(int64_t)s * N + r];
    y[r] = ADD ? y[r] + acc : acc;
}

/* ------------------------------------------------------------------ selection */
#define SEL_T 1024
#define SEL_MAX_K 32768

/* |x| of a 15-bit key for the relational threshold: (128 + mantissa) 2^(e - 134) with the
 * exponent clamped to [-60, 40], 0 for zero and subnormal keys (an exact product). */
__device__ __forceinline__ float sel_mag(int k) {
    const int ex = k >> 7;
    const int n = min(max(ex - 134, -60), 40);
    return ex > 0 ? (float)(128 + (k & 127)) * __uint_as_float((uint32_t)(n + 127) << 23) : 0.0f;
}

/* Threshold T and the kept list (the rule in include/glint_select.h). rank(n) = the largest
 * 15-bit T with count(key >= T) >= n is a radix select over two LDS histograms: 256 bins of
 * key >> 7 (built once), then 128 bins of key & 127 inside the chosen bin; that is the T
 * the rule's bit-by-bit bisection finds, since the count is non-increasing in T; n <= 0
 * gives 32767 and n > K gives 0, as the bisection does. The relational price sums |x| in
 * f32 over the 1024 threads' ranges of ceil(K / 1024) channels and then pairwise in LDS,
 * the order the rule fixes. The kept channels are written in ascending order through a
 * block scan. */
__global__ __launch_bounds__(SEL_T) void k_select_topk(const uint16_t *__restrict__ x, int K, int nsel, int tkey,
                                                       int nfloor, int32_t *__restrict__ idx, int32_t *__restrict__ cnt,
                                                       int32_t *__restrict__ cnt_log, int slot) {
    __shared__ uint16_t keys[SEL_MAX_K];
    __shared__ int hc[256], hf[128]; /* coarse and fine histograms */
    __shared__ int wsum[SEL_T / 64];
    __shared__ float red[SEL_T];
    __shared__ int s_bin, s_above, s_thr;
    const int t = threadIdx.x, lane = t & 63;
    const int per = (K + SEL_T - 1) / SEL_T;
    const int lo = min(t * per, K), hi = min(lo + per, K);
    if (t < 256)
        hc[t] = 0;
    __syncthreads();
    for (int i = t; i < K; i += SEL_T) {
        const int k = x[i] & 0x7FFF;
        keys[i] = (uint16_t)k;
        atomicAdd(&hc[k >> 7], 1);
    }
    __syncthreads();
    /* every thread calls rank with the same n (its barriers are block-wide) */
    auto rank = [&](int n) -> int {
        if (n <= 0)
            return 32767;
        if (t < 128)
            hf[t] = 0;
        if (t == 0) {
            s_bin = -1;
            s_above = 0;
            s_thr = 0; /* no bin qualifies when count(all) < n: everything is kept */
        }
        __syncthreads();
        if (t < 64) { /* lane l: coarse bins 4 l .. 4 l + 3; suffix counts */
            const int v0 = hc[4 * lane], v1 = hc[4 * lane + 1], v2 = hc[4 * lane + 2], v3 = hc[4 * lane + 3];
            const int sum = v0 + v1 + v2 + v3;
            int inc = sum; /* sum over lanes lane .. 63 */
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int v = __shfl_down(inc, o, 64);
                if (lane + o < 64)
                    inc += v;
            }
            const int c4 = inc - sum, c3 = c4 + v3, c2 = c3 + v2, c1 = c2 + v1, c0 = c1 + v0; /* c_j = count(bin >= 4 l + j) */
            const int cs[5] = {c0, c1, c2, c3, c4};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (cs[j] >= n && cs[j + 1] < n) { /* exactly one bin, when count(all) >= n */
                    s_bin = 4 * lane + j;
                    s_above = cs[j + 1];
                }
        }
        __syncthreads();
        const int bin = s_bin;
        if (bin >= 0) {
            for (int i = t; i < K; i += SEL_T) {
                const int k = keys[i];
                if ((k >> 7) == bin)
                    atomicAdd(&hf[k & 127], 1);
            }
            __syncthreads();
            if (t < 64) { /* lane l: fine bins 2 l, 2 l + 1 */
                const int need = n - s_above;
                const int v0 = hf[2 * lane], v1 = hf[2 * lane + 1];
                const int sum = v0 + v1;
                int inc = sum;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const int v = __shfl_down(inc, o, 64);
                    if (lane + o < 64)
                        inc += v;
                }
                const int c2 = inc - sum, c1 = c2 + v1, c0 = c1 + v0;
                if (c0 >= need && c1 < need)
                    s_thr = (bin << 7) | (2 * lane);
                if (c1 >= need && c2 < need)
                    s_thr = (bin << 7) | (2 * lane + 1);
            }
        }
        __syncthreads();
        const int r = s_thr;
        __syncthreads(); /* s_thr is reused by the next call */
        return r;
    };
    const int cap = rank(nsel);
    int thr = max(cap, tkey);
    if (tkey < 0) { /* relational price: tau = -tkey / 1024 times mean |x| */
        float acc = 0.0f;
        for (int i = lo; i < hi; ++i)
            acc += sel_mag(keys[i]);
        red[t] = acc;
        __syncthreads();
#pragma unroll
        for (int off = SEL_T / 2; off >= 1; off >>= 1) {
            if (t < off)
                red[t] = red[t] + red[t + off];
            __syncthreads();
        }
        float tv = red[0] / (float)K * (float)(-tkey) / 1024.0f;
        int rk = 1;
        if (tv > 0.0f) {
            int e2 = 0;
            while (tv >= 2.0f && e2 < 100) {
                tv *= 0.5f;
                ++e2;
            }
            while (tv < 1.0f && e2 > -120) {
                tv *= 2.0f;
                --e2;
            }
            rk = min(max(((e2 + 127) << 7) | (int)((tv - 1.0f) * 128.0f), 1), 32767);
        }
        thr = max(thr, rk);
    }
    if (nfloor > 0 && tkey != 0)
        thr = max(cap, min(thr, rank(nfloor)));
    if (nsel == 0)
        thr = 32768;
    int mine = 0;
    for (int i = lo; i < hi; ++i)
        mine += keys[i] >= thr;
    /* exclusive scan of mine over the block: inclusive within the wave, then wave offsets */
    int inc = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(inc, o, 64);
        if (lane >= o)
            inc += v;
    }
    if (lane == 63)
        wsum[t >> 6] = inc;
    __syncthreads();
    int base = 0, total = 0;
#pragma unroll
    for (int i = 0; i < SEL_T / 64; ++i) {
        base += (i < (t >> 6)) ? wsum[i] : 0;
        total += wsum[i];
    }
    int pos = base + inc - mine;
    for (int i = lo; i < hi; ++i)
        if (keys[i] >= thr)
            idx[pos++] = i;
    if (t == 0) {
        cnt[0] = total;
        if (cnt_log)
            cnt_log[slot] = total;
    }
}

/* ---------------------------------------------------------------- correction */
/* Workgroup (row block bx, list chunk by): the chunk is cut into KM_SUB parts, wave q walks
 * part q as runs of consecutive list entries inside one 64-block (the list is ascending,
 * so a block's channels are adjacent). Delta = CELLS - PARENT sits in LDS as 64 lane
 * copies, addressed by the code byte (h << 4 | p). One chunk adds into y; several write
 * part[by N + r] for k_km_combine<true>. */
template <int RPL>
__global__ __launch_bounds__(KM_WG) void k_apply_corr_km(const uint8_t *__restrict__ hole_bytes,
                                                         const uint8_t *__restrict__ plug_bytes,
                                                         const float *__restrict__ scales_k,
                                                         const uint16_t *__restrict__ x, const int32_t *__restrict__ idx,
                                                         const int32_t *__restrict__ cnt, float *__restrict__ y,
                                                         float *__restrict__ part, unsigned *ctr, int N, int ks) {
    constexpr int ROWS = 64 * RPL, NW = RPL / 8; /* rows per workgroup, code words per lane */
    using HV = typename std::conditional<RPL == 32, glint_u32x4,
                                         typename std::conditional<RPL == 16, glint_u32x2, uint32_t>::type>::type;
    static_assert(RPL == 8 || RPL == 16 || RPL == 32, "rows per lane");
    const HV *__restrict__ hole_k = (const HV *)hole_bytes, *__restrict__ plug_k = (const HV *)plug_bytes;
    constexpr int LDSW = KM_SUB * ROWS > GLINT_LDS_CELLS64_WORDS ? KM_SUB * ROWS : GLINT_LDS_CELLS64_WORDS;
    __shared__ __attribute__((aligned(16))) float lds[LDSW]; /* delta table, then parts */
    /* 4 adjacent copies of an entry per 16-B store: entry hp = word / 64 */
    for (int i = threadIdx.x; i < GLINT_LDS_CELLS64_WORDS / 4; i += KM_WG) {
        const int hp = i >> 4;
        const float d = (&kCells[0][0])[hp] - kParent[hp >> 4];
        *(glint_f32x4 *)(lds + 4 * i) = glint_f32x4{d, d, d, d};
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane4 = (uint32_t)lane * 4u;
    const int r0 = blockIdx.x * ROWS;
    const int rc = min(r0 + RPL * lane, N - RPL);
    const int64_t rowv = N / RPL;
    const int cn = cnt[0];
    const int chunk = (cn + ks - 1) / ks, sub = (chunk + KM_SUB - 1) / KM_SUB;
    const int lo = blockIdx.y * chunk, hi = min(lo + chunk, cn);
    const int i0 = min(lo + q * sub, hi), i1 = min(i0 + sub, hi);
    float tot[RPL], acc[RPL];
#pragma unroll
    for (int j = 0; j < RPL; ++j)
        tot[j] = acc[j] = 0.f;
    int cur = -1;
    auto flush = [&]() {
        float sc[RPL];
        km_load<RPL>(scales_k + (int64_t)cur * N + rc, sc);
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            tot[j] = fmaf(acc[j], sc[j], tot[j]);
            acc[j] = 0.f;
        }
    };
    for (int i = i0; i < i1; ++i) {
        const int c = idx[i];
        const HV hv = hole_k[(int64_t)c * rowv + rc / RPL], pv = plug_k[(int64_t)c * rowv + rc / RPL];
        if ((c >> 6) != cur) {
            if (cur >= 0)
                flush();
            cur = c >> 6;
        }
        const float xv = km_bf16(x[c]);
        uint32_t Hs[NW], Ps[NW];
        __builtin_memcpy(Hs, &hv, sizeof(Hs));
        __builtin_memcpy(Ps, &pv, sizeof(Ps));
        uint32_t E[NW], O[NW];
#pragma unroll
        for (int q = 0; q < NW; ++q) {
            E[q] = glint_codes_even(Hs[q], Ps[q]);
            O[q] = glint_codes_odd(Hs[q], Ps[q]);
        }
        km_lookup_fma<RPL>(lds, E, O, lane4, xv, acc);
    }
    if (cur >= 0)
        flush();
    km_finish<true, RPL>(lds, tot, r0, N, y, part, ctr, ks, blockIdx.y);
}

/* -------------------------------------------------------------------- C ABI */
static int km_launched() { return hipGetLastError() == hipSuccess ? 0 : -3; }

bool glint_stream_workspace(hipStream_t st, GlintSplitWs *ws); /* glint_htile.hip */

/* Arrival counters for `blocks` row blocks: the split-K workspace counters (zero between
 * launches) of a stream that already has a workspace, or null when it has none (these
 * calls never allocate one: glint_htile_workspace_reserve or an earlier split launch
 * provides it) or too few: the slices then meet in k_km_combine. */
static unsigned *km_counters(hipStream_t st, unsigned blocks) {
    GlintSplitWs ws;
    if (!glint_stream_workspace(st, &ws) || ws.nctr < blocks)
        return nullptr;
    return ws.ctr;
}

GLINT_API int glint_kmajor_pack(const uint8_t *hole, const uint8_t *plug, const float *absmax, int N, int K,
                                uint8_t *hole_k, uint8_t *plug_k, float *scales_k, hipStream_t stream) {
    if (!hole || !plug || !absmax || !hole_k || !plug_k || !scales_k)
        return -1;
    if (N < 8 || (N % 8) != 0 || K < 64 || (K % 64) != 0 || !glint_aligned(hole, 8) || !glint_aligned(plug, 8) ||
        !glint_aligned(hole_k, 4) || !glint_aligned(plug_k, 4))
        return -2;
    k_kmajor_pack_planes<<<dim3(K / 64, (N + KP_ROWS - 1) / KP_ROWS), KM_T, 0, stream>>>(hole, plug, hole_k, plug_k,
                                                                                     N, K);
    const int64_t total = (int64_t)N * (K / 64);
    const unsigned g = (unsigned)std::min<int64_t>((total + KM_T - 1) / KM_T, 65535);
    k_kmajor_scales<<<g, KM_T, 0, stream>>>(absmax, scales_k, N, K / 64);
    return km_launched();
}

GLINT_API int glint_gemv_km_fold(const uint8_t *hole_k, const float *scales_k, const uint16_t *x, float *y, int N, int K,
                                 int ksg, float *part, hipStream_t stream) {
    if (!hole_k || !scales_k || !x || !y || (ksg > 1 && !part))
        return -1;
    if (N < 32 || (N % 32) != 0 || ksg < 1 || K < 64 || (K % (64 * ksg)) != 0 || !glint_aligned(hole_k, 16) ||
        !glint_aligned(scales_k, 16) || !glint_aligned(x, 16))
        return -2;
    const dim3 grid((N + 64 * KM_FOLD_RPL - 1) / (64 * KM_FOLD_RPL), ksg);
    unsigned *ctr = ksg > 1 ? km_counters(stream, grid.x) : nullptr;
    k_gemv_km_fold<KM_FOLD_RPL><<<grid, KM_WG, 0, stream>>>(hole_k, scales_k, x, y, part, ctr, N, K / ksg);
    if (ksg > 1 && !ctr)
        k_km_combine<false><<<(N + KM_T - 1) / KM_T, KM_T, 0, stream>>>(part, y, N, ksg);
    return km_launched();
}

GLINT_API int glint_select_topk_ex(const uint16_t *x, int K, int nsel, int tkey, int nfloor, int32_t *idx,
                                   int32_t *cnt, int32_t *cnt_log, int slot, hipStream_t stream) {
    if (!x || !idx || !cnt)
        return -1;
    if (K < 1 || K > SEL_MAX_K || (cnt_log && slot < 0))
        return -2;
    k_select_topk<<<1, SEL_T, 0, stream>>>(x, K, nsel, tkey, nfloor, idx, cnt, cnt_log, slot);
    return km_launched();
}

GLINT_API int glint_select_topk(const uint16_t *x, int K, int nsel, int32_t *idx, int32_t *cnt, hipStream_t stream) {
    return glint_select_topk_ex(x, K, nsel, 0, 0, idx, cnt, nullptr, 0, stream);
}

GLINT_API int glint_apply_corr_km(const uint8_t *hole_k, const uint8_t *plug_k, const float *scales_k,
                                  const uint16_t *x, const int32_t *idx, const int32_t *cnt, float *y, int N, int K,
                                  int ks, float *part, hipStream_t stream) {
    if (!hole_k || !plug_k || !scales_k || !x || !idx || !cnt || !y || (ks > 1 && !part))
        return -1;
    if (N < 32 || (N % 32) != 0 || K < 64 || (K % 64) != 0 || ks < 1 || !glint_aligned(hole_k, 16) ||
        !glint_aligned(plug_k, 16) || !glint_aligned(scales_k, 16))
        return -2;
    const dim3 grid((N + 64 * KM_CORR_RPL - 1) / (64 * KM_CORR_RPL), ks);
    unsigned *ctr = ks > 1 ? km_counters(stream, grid.x) : nullptr;
    k_apply_corr_km<KM_CORR_RPL><<<grid, KM_WG, 0, stream>>>(hole_k, plug_k, scales_k, x, idx, cnt, y, part, ctr, N,
                                                             ks);
    if (ks > 1 && !ctr)
        k_km_combine<true><<<(N + KM_T - 1) / KM_T, KM_T, 0, stream>>>(part, y, N, ks);
    return km_launched();
}
