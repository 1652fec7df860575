/* GLINT encode (BF16/F32 -> hole/plug nibble planes + f32 absmax) and expand
 * (planes -> f32 / BF16) for gfx950.
 *
 * Semantics: reference cuda/glint_encode.cu:41-114 and glint_np.py:25-92 (absmax skips
 * NaN; v = (s == 0) ? 0 : w / s in f32; first-minimum nearest parent, then nearest
 * child of that parent; element 2e in the low nibble; BF16 = RNE with the NaN rule).
 *
 * Fast encode (bs = 64, BF16, aligned): one pass, one 16-byte load per lane per
 * 512-element wave chunk. Lane l of the chunk owns elements [8l, 8l+8), so a 64-block is
 * 8 lanes: absmax is a packed-u16 max over BF16 magnitudes plus a 3-step DPP max. For a
 * block with 2^-90 <= absmax < 2^90 and no NaN the code is looked up from
 * q = RN(w * RN(1/s)), one multiply: for every bf16 pair in that range q gives the code of
 * the correctly rounded w / s and |q| <= 1 (tests/native/check_encode_quotient.c walks all
 * 374,549,760 of them), and RN(1/s) of a bf16 s is a 128-entry LDS table plus an integer
 * subtract. Other blocks (zero, tiny, huge, inf or NaN present) take the NaN-skipping
 * absmax and the IEEE divide. The nearest-code search is one LDS bucket lookup and one
 * compare (glint_codebook.h, verified against the scan for every float in [-1, 1]).
 * Everything else (any bs, F32 input, tails, unaligned pointers) runs the generic pair.
 */
#include "glint_common.h"
#include "glint_codebook.h"
#include "glint_cells.h"
#include "glint_encode.h"

#include <stdio.h>

#include <algorithm>

__constant__ GlintCodeEntry kCodeTable[GLINT_CODE_BUCKETS] = {
#include "glint_code_table.inc"
};

/* code(v) = base + (v > thr) from an entry table in LDS or constant memory.
 * v is an f32 divide or fma result, so at worst a quiet NaN; v_med3_f32 returns
 * min3(v, -1, 1) = -1 for a NaN input, which selects bucket 0 like the host's
 * fminf(fmaxf(v, -1), 1) in glint_codebook.h. */
template <typename Tab>
__device__ __forceinline__ uint32_t glint_code_of(float v, const Tab *tab) {
    const float c = __builtin_amdgcn_fmed3f(v, -1.0f, 1.0f);
    const uint32_t b = min(__float_as_uint(fmaf(c, 256.0f, GLINT_CODE_MAGIC)) - GLINT_CODE_MAGIC_BITS,
                           (uint32_t)(GLINT_CODE_BUCKETS - 1)); /* never out of the table */
    const GlintCodeEntry e = tab[b];
    return e.base + (v > __uint_as_float(e.thr) ? 1u : 0u);
}

/* ------------------------------------------------------------------ fast encode */
typedef unsigned short glint_u16x2 __attribute__((ext_vector_type(2)));
typedef short glint_i16x2 __attribute__((ext_vector_type(2)));

/* Max BF16 magnitude of the two halves of d, NaN skipped, as (mag + 0x7F) in i16 lanes:
 * a NaN magnitude (0x7F81..0x7FFF) becomes negative and never wins; inf (0x7F80)
 * becomes 0x7FFF. */
__device__ __forceinline__ glint_i16x2 glint_mag_key(uint32_t d) {
    const glint_u16x2 m = __builtin_bit_cast(glint_u16x2, d & 0x7FFF7FFFu) + (glint_u16x2)(0x7F);
    return __builtin_bit_cast(glint_i16x2, m);
}

/* LDS form of the bucket table: entry b = {threshold bits, S(base), S(base + 1), R(b)} with
 * the "spread" code S(c) = hole | plug << 16 = (c >> 4) | (c & 15) << 16, so a lane folds
 * its 4 codes into hole nibbles (bits 0..15) and plug nibbles (bits 16..31) with one
 * shift-or each, and the reciprocal word R (glint_recip_word). ENC_COPIES copies, entry b
 * of copy j at byte (b * ENC_COPIES + j) * 16, lane l reading copy l % ENC_COPIES, to
 * spread the random lookups over the banks. */
#ifndef ENC_COPIES
#define ENC_COPIES 4
#endif
static_assert(ENC_COPIES >= 1 && ENC_COPIES <= 64 && (ENC_COPIES & (ENC_COPIES - 1)) == 0, "power-of-two table copies");
#define ENC_ENTRY_SHIFT (4 + __builtin_ctz(ENC_COPIES)) /* log2 of the byte stride of one entry's copies */
#ifndef ENC_THREADS
#define ENC_THREADS 1024
#endif
#ifndef ENC_UNROLL
#define ENC_UNROLL 1
#endif
#ifndef ENC_WPE /* minimum waves per SIMD the register allocation must allow */
#define ENC_WPE 4
#endif
#ifndef ENC_PIECE_CHUNKS
#define ENC_PIECE_CHUNKS (1 << 17) /* most 512-element chunks per k_encode_bf16_b64 launch (67 M elements) */
#endif

__device__ __forceinline__ uint32_t glint_spread_code(uint32_t c) { return (c >> 4) | ((c & 15u) << 16); }

/* R(b) for b < 128: bits(RN(1/(1 + b/128))) + 0x3F800000 + (b << 16). A normal bf16
 * s = 2^(E-127) (1 + b/128) has RN(1/s) = RN(1/(1 + b/128)) 2^(127-E) (exact scaling while
 * the result is normal), whose bits are R(b) - bits(s) since bits(s) = E << 23 | b << 16.
 * The divide is IEEE (correctly rounded); tests/native/check_encode_quotient.c checks the
 * identity for every s the fast path takes. */
__device__ __forceinline__ uint32_t glint_recip_word(int b) {
    return b < 128 ? __float_as_uint(1.0f / (1.0f + (float)b * 0.0078125f)) + 0x3F800000u + ((uint32_t)b << 16) : 0u;
}

__device__ __forceinline__ glint_u32x4 glint_code_lds_entry(GlintCodeEntry e, int b) {
    return glint_u32x4{e.thr, glint_spread_code(e.base), glint_spread_code(e.base + 1), glint_recip_word(b)};
}

/* Spread code of v (|v| <= 1 or a quiet NaN; see glint_code_of). `lane_k` is this lane's
 * constant making the byte address (bucket << 7) + lane_k land on its own copy. */
__device__ __forceinline__ uint32_t glint_spread_of(float v, const glint_u32x4 *tab, uint32_t lane_k) {
    const float c = __builtin_amdgcn_fmed3f(v, -1.0f, 1.0f);
    const uint32_t addr = (__float_as_uint(fmaf(c, 256.0f, GLINT_CODE_MAGIC)) * (ENC_COPIES * 16u)) + lane_k;
    const glint_u32x4 e = *(const glint_u32x4 *)((const char *)tab + addr);
    return v > __uint_as_float(e.x) ? e.z : e.y;
}

/* Spread code of q with |q| <= 1 (no clamp: the fast path's quotients never leave
 * [-1, 1], so the bucket is in [0, 512]). */
__device__ __forceinline__ uint32_t glint_spread_fast(float q, const glint_u32x4 *tab, uint32_t lane_k) {
    const uint32_t addr = (__float_as_uint(fmaf(q, 256.0f, GLINT_CODE_MAGIC)) * (ENC_COPIES * 16u)) + lane_k;
    const glint_u32x4 e = *(const glint_u32x4 *)((const char *)tab + addr);
    return q > __uint_as_float(e.x) ? e.z : e.y;
}

template <int CTRL>
__device__ __forceinline__ int glint_max_dpp(int v) {
    /* bound_ctrl with full masks lets the DPP move fold into v_max_i32_dpp */
    return max(v, __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true));
}

/* Largest BF16 magnitude bits of a lane's 8 values (NaN not skipped: a NaN, 0x7F81 and up,
 * wins and sends its block to the exact path). */
__device__ __forceinline__ uint32_t glint_mag_max(const glint_u32x4 d) {
    const glint_u16x2 a = __builtin_bit_cast(glint_u16x2, d.x & 0x7FFF7FFFu);
    const glint_u16x2 b = __builtin_bit_cast(glint_u16x2, d.y & 0x7FFF7FFFu);
    const glint_u16x2 c = __builtin_bit_cast(glint_u16x2, d.z & 0x7FFF7FFFu);
    const glint_u16x2 e = __builtin_bit_cast(glint_u16x2, d.w & 0x7FFF7FFFu);
    const glint_u16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(a, b), __builtin_elementwise_max(c, e));
    return max((uint32_t)m.x, (uint32_t)m.y);
}

/* Block absmax bits with NaN skipped (glint_mag_key), reduced over the 8 lanes. */
__device__ __forceinline__ uint32_t glint_absmax_skip_nan(const glint_u32x4 d) {
    glint_i16x2 k = __builtin_elementwise_max(glint_mag_key(d.x), glint_mag_key(d.y));
    k = __builtin_elementwise_max(k, __builtin_elementwise_max(glint_mag_key(d.z), glint_mag_key(d.w)));
    int m16 = max(max((int)k.x, (int)k.y), 0x7F) - 0x7F;
    m16 = glint_max_dpp<GLINT_DPP_QUAD_1032>(m16);
    m16 = glint_max_dpp<GLINT_DPP_QUAD_2301>(m16);
    m16 = glint_max_dpp<GLINT_DPP_ROW_HALF_MIRROR>(m16);
    return (uint32_t)m16 << 16;
}

__device__ __forceinline__ void glint_encode_chunk(const glint_u32x4 d, const glint_u32x4 *tab, uint32_t lane_k,
                                                   uint32_t lane_r, int64_t chunk, int lane,
                                                   uint32_t *__restrict__ hole, uint32_t *__restrict__ plug,
                                                   float *__restrict__ absmax) {
    /* magnitude max of this lane's 8 values, then of the 8 lanes that share the block (the
     * DPP moves stay inside each aligned group of 8 lanes) */
    int m16 = (int)glint_mag_max(d);
    m16 = glint_max_dpp<GLINT_DPP_QUAD_1032>(m16);
    m16 = glint_max_dpp<GLINT_DPP_QUAD_2301>(m16);
    m16 = glint_max_dpp<GLINT_DPP_ROW_HALF_MIRROR>(m16);
    uint32_t sbits = (uint32_t)m16 << 16;

    const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
    float w[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        w[2 * j] = glint_bf16lo(dw[j]);
        w[2 * j + 1] = glint_bf16hi(dw[j]);
    }
    /* element 4h + i contributes its hole nibble at bit 4i and plug nibble at 16 + 4i */
    uint32_t acc[2];
    if (sbits - 0x12800000u < 0x6C800000u - 0x12800000u) { /* 2^-90 <= s < 2^90, so no NaN or inf */
        /* entry m (the mantissa of s, bits 16..22) at byte m * ENC_COPIES * 16 */
        const uint32_t rw =
            *(const uint32_t *)((const char *)tab + ((sbits >> (16 - ENC_ENTRY_SHIFT)) & (127u << ENC_ENTRY_SHIFT)) + lane_r);
        const float y = __uint_as_float(rw - sbits); /* RN(1/s) */
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t a = glint_spread_fast(w[4 * h] * y, tab, lane_k);
#pragma unroll
            for (int i = 1; i < 4; ++i)
                a |= glint_spread_fast(w[4 * h + i] * y, tab, lane_k) << (4 * i);
            acc[h] = a;
        }
    } else {
        sbits = glint_absmax_skip_nan(d);
        const float s = __uint_as_float(sbits);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t a = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                a |= glint_spread_of((s == 0.0f) ? 0.0f : w[4 * h + i] / s, tab, lane_k) << (4 * i);
            acc[h] = a;
        }
    }
    hole[chunk * 64 + lane] = __builtin_amdgcn_perm(acc[1], acc[0], 0x05040100u);
    plug[chunk * 64 + lane] = __builtin_amdgcn_perm(acc[1], acc[0], 0x07060302u);
    if ((lane & 7) == 0)
        absmax[chunk * 8 + (lane >> 3)] = __uint_as_float(sbits);
}

/* One wave handles groups of ENC_UNROLL consecutive chunks: groups wave, wave + nwaves, ...
 * two groups in flight (register double buffer, unconditional clamped loads, full rounds
 * so the wait counter can count them); the table fill's loads go out first and its LDS
 * writes after the first two groups' loads. Chunks past the last full group are spread
 * one per wave at the end. */
__global__ __launch_bounds__(ENC_THREADS, ENC_WPE) void k_encode_bf16_b64(const glint_u32x4 *__restrict__ w,
                                                                 uint32_t *__restrict__ hole,
                                                                 uint32_t *__restrict__ plug,
                                                                 float *__restrict__ absmax, int64_t nchunks) {
    __shared__ __attribute__((aligned(16))) glint_u32x4 tab[GLINT_CODE_BUCKETS * ENC_COPIES];
    const int lane = threadIdx.x & 63;
    /* bucket * ENC_COPIES * 16 + lane_k == byte offset of entry (bucket, lane % ENC_COPIES):
     * the fma result's bits are 2^23's plus the bucket, so subtract 2^23's bits times the
     * entry stride (mod 2^32) */
    const uint32_t lane_k =
        (uint32_t)(lane % ENC_COPIES) * 16u - GLINT_CODE_MAGIC_BITS * (uint32_t)(ENC_COPIES * 16);
    const uint32_t lane_r = (uint32_t)(lane % ENC_COPIES) * 16u + 12u; /* word 3 of this lane's copy */
    /* wave-uniform, so group arithmetic stays in scalar registers */
    const int wave = (int)blockIdx.x * (ENC_THREADS / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = (int)gridDim.x * (ENC_THREADS / 64);
    const int ngroups = (int)(nchunks / ENC_UNROLL);
    const int my = wave < ngroups ? (ngroups - wave + nwaves - 1) / nwaves : 0; /* groups wave + i nwaves */
    const int last = max(ngroups - 1, 0);

    constexpr int kEntries = GLINT_CODE_BUCKETS * ENC_COPIES;
    constexpr int kFill = (kEntries + 1023) / 1024; /* entries per thread at 1024 threads */
    GlintCodeEntry fe[kFill];
    int fi[kFill];
#pragma unroll
    for (int k = 0; k < kFill; ++k) {
        fi[k] = min((int)threadIdx.x + k * (int)blockDim.x, kEntries - 1);
        fe[k] = kCodeTable[fi[k] / ENC_COPIES];
    }
    /* unconditional loads (a branch here would make every later wait count the worst
     * path); chunk indices are clamped to the last chunk for the case of no full group */
    const int64_t lastc = nchunks - 1;
    glint_u32x4 da[ENC_UNROLL], db[ENC_UNROLL];
    {
        const int64_t ga = (int64_t)min(wave, last) * ENC_UNROLL, gb = (int64_t)min(wave + nwaves, last) * ENC_UNROLL;
#pragma unroll
        for (int u = 0; u < ENC_UNROLL; ++u)
            da[u] = __builtin_nontemporal_load(&w[min(ga + u, lastc) * 64 + lane]);
#pragma unroll
        for (int u = 0; u < ENC_UNROLL; ++u)
            db[u] = __builtin_nontemporal_load(&w[min(gb + u, lastc) * 64 + lane]);
    }
#pragma unroll
    for (int k = 0; k < kFill; ++k) /* clamped indices rewrite the last entry with its own value */
        tab[fi[k]] = glint_code_lds_entry(fe[k], fi[k] / ENC_COPIES);
    for (int e = threadIdx.x + kFill * blockDim.x; e < kEntries; e += blockDim.x) /* blockDim < 1024 only */
        tab[e] = glint_code_lds_entry(kCodeTable[e / ENC_COPIES], e / ENC_COPIES);
    __syncthreads();

    int i = 0;
    for (; i + 2 <= my; i += 2) {
        const int64_t c0 = (int64_t)(wave + i * nwaves) * ENC_UNROLL;
#pragma unroll
        for (int u = 0; u < ENC_UNROLL; ++u)
            glint_encode_chunk(da[u], tab, lane_k, lane_r, c0 + u, lane, hole, plug, absmax);
        const int64_t ga = (int64_t)min(wave + (i + 2) * nwaves, last) * ENC_UNROLL;
#pragma unroll
        for (int u = 0; u < ENC_UNROLL; ++u)
            da[u] = __builtin_nontemporal_load(&w[(ga + u) * 64 + lane]);
        const int64_t c1 = (int64_t)(wave + (i + 1) * nwaves) * ENC_UNROLL;
#pragma unroll
        for (int u = 0; u < ENC_UNROLL; ++u)
            glint_encode_chunk(db[u], tab, lane_k, lane_r, c1 + u, lane, hole, plug, absmax);
        const int64_t gb = (int64_t)min(wave + (i + 3) * nwaves, last) * ENC_UNROLL;
#pragma unroll
        for (int u = 0; u < ENC_UNROLL; ++u)
            db[u] = __builtin_nontemporal_load(&w[(gb + u) * 64 + lane]);
    }
    if (i < my) {
        const int64_t c0 = (int64_t)(wave + i * nwaves) * ENC_UNROLL;
#pragma unroll
        for (int u = 0; u < ENC_UNROLL; ++u)
            glint_encode_chunk(da[u], tab, lane_k, lane_r, c0 + u, lane, hole, plug, absmax);
    }
    const int64_t c = (int64_t)ngroups * ENC_UNROLL + wave; /* at most ENC_UNROLL - 1 leftover chunks */
    if (c < nchunks)
        glint_encode_chunk(w[c * 64 + lane], tab, lane_k, lane_r, c, lane, hole, plug, absmax);
}

/* ---------------------------------------------------------------- generic encode */
__device__ __forceinline__ float glint_load_w(const uint16_t *w, int64_t i) { return __uint_as_float((uint32_t)w[i] << 16); }
__device__ __forceinline__ float glint_load_w(const float *w, int64_t i) { return w[i]; }

/* absmax of blocks [b0, b1): one wave per block, NaN skipped (fabsf(NaN) > m is false). */
template <typename T>
__global__ __launch_bounds__(256) void k_absmax_generic(const T *__restrict__ w, int64_t n, int bs, int64_t b0,
                                                        int64_t b1, float *__restrict__ absmax) {
    const int lane = threadIdx.x & 63;
    const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x >> 6);
    for (int64_t b = b0 + (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); b < b1; b += nwaves) {
        const int64_t i0 = b * bs;
        const int64_t i1 = min(i0 + bs, n);
        float m = 0.0f;
        for (int64_t i = i0 + lane; i < i1; i += 64) {
            const float a = fabsf(glint_load_w(w, i));
            if (a > m)
                m = a;
        }
        m = glint_wave_max(m); /* no NaN left among the partial maxima */
        if (lane == 0)
            absmax[b] = m;
    }
}

/* packed bytes [e0, e1): v = (s == 0) ? 0 : w / s (IEEE divide), code lookup, pack. */
template <typename T>
__global__ __launch_bounds__(256) void k_encode_generic(const T *__restrict__ w, const float *__restrict__ absmax,
                                                        int64_t n, int bs, int64_t e0, int64_t e1,
                                                        uint8_t *__restrict__ hole, uint8_t *__restrict__ plug) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = e0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < e1; e += stride) {
        uint32_t c[2] = {0u, 0u};
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int64_t i = 2 * e + t;
            if (i < n) {
                const float s = absmax[i / bs];
                const float v = (s == 0.0f) ? 0.0f : glint_load_w(w, i) / s;
                c[t] = glint_code_of(v, kCodeTable);
            }
        }
        hole[e] = (uint8_t)((c[0] >> 4) | (c[1] & 0xF0u));
        plug[e] = (uint8_t)((c[0] & 15u) | ((c[1] & 15u) << 4));
    }
}

static int glint_num_cus() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return 256;
    if (!cached[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

static unsigned glint_grid(int64_t work_items, int per_block, int max_blocks) {
    int64_t g = (work_items + per_block - 1) / per_block;
    if (g > max_blocks)
        g = max_blocks;
    return (unsigned)(g < 1 ? 1 : g);
}

template <typename T>
static int encode_device(const T *d_w, int64_t n, int bs, uint8_t *d_hole, uint8_t *d_plug, float *d_am,
                         hipStream_t st) {
    if (n < 0 || bs <= 0)
        return -1;
    if (n == 0)
        return 0;
    if (!d_w || !d_hole || !d_plug || !d_am)
        return -1;
    const int cus = glint_num_cus();
    int64_t n_fast = 0;
    if (sizeof(T) == 2 && bs == 64 && glint_aligned(d_w, 16) && glint_aligned(d_hole, 4) && glint_aligned(d_plug, 4) &&
        glint_aligned(d_am, 4))
        n_fast = (n / 512) * 512;
    if (n_fast) {
        const int64_t nchunks = n_fast / 512;
        /* Tensors above ENC_PIECE_CHUNKS chunks go as equal consecutive pieces, one launch
         * each on the stream (the bytes are the same): one launch over the 525 M-element
         * embedding ran at 57-59% of HBM, eight pieces of 66 M elements at 62-64% (16 pieces
         * 59%); the Llama-3-8B set on 4 streams 62.0 -> 63.5%. */
        const int64_t pieces = (nchunks + ENC_PIECE_CHUNKS - 1) / ENC_PIECE_CHUNKS;
        const int64_t per = (nchunks + pieces - 1) / pieces;
        const int resident = (int)glint_resident_grid((const void *)k_encode_bf16_b64, ENC_THREADS, 0);
        for (int64_t c0 = 0; c0 < nchunks; c0 += per) {
            const int64_t nc = std::min(per, nchunks - c0);
            /* a group per wave while there are enough groups, at most the resident blocks;
             * the leftover chunks (< ENC_UNROLL) need fewer waves than one block has */
            const unsigned grid = glint_grid(nc, (ENC_THREADS / 64) * ENC_UNROLL, resident);
            k_encode_bf16_b64<<<grid, ENC_THREADS, 0, st>>>((const glint_u32x4 *)d_w + c0 * 64,
                                                            (uint32_t *)d_hole + c0 * 64, (uint32_t *)d_plug + c0 * 64,
                                                            d_am + c0 * 8, nc);
        }
    }
    if (n_fast < n) {
        const int64_t b0 = n_fast / bs, b1 = (n + bs - 1) / bs;
        k_absmax_generic<T><<<glint_grid(b1 - b0, 4, cus * 16), 256, 0, st>>>(d_w, n, bs, b0, b1, d_am);
        const int64_t e0 = n_fast / 2, e1 = (n + 1) / 2;
        k_encode_generic<T><<<glint_grid(e1 - e0, 256, cus * 16), 256, 0, st>>>(d_w, d_am, n, bs, e0, e1, d_hole,
                                                                                 d_plug);
    }
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* ------------------------------------------------------------------ expand */
/* A group is 32 consecutive elements (16 B of each plane) inside one absmax block
 * (bs % 32 == 0). Each lane issues the loads of EU groups before converting any, looks
 * cells up in the 64-copy LDS table (one v_perm_b32 per address) and writes 64 B (BF16)
 * or 128 B (f32) per group. */
#define EXPAND_THREADS 1024
#define EXPAND_U 4
#ifndef EXPAND_NT_STORE
#define EXPAND_NT_STORE 0 /* 1: nontemporal output stores */
#endif

template <typename T>
__device__ __forceinline__ void glint_store_out(T v, T *p) {
    if (EXPAND_NT_STORE)
        __builtin_nontemporal_store(v, p);
    else
        *p = v;
}

template <bool BF16>
__device__ __forceinline__ void expand_group(const float *ltab, uint32_t lane4, glint_u32x4 hv, glint_u32x4 pv, float a,
                                             void *__restrict__ out, int64_t g) {
    const uint32_t H[4] = {hv.x, hv.y, hv.z, hv.w}, P[4] = {pv.x, pv.y, pv.z, pv.w};
    float r[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t E = glint_codes_even(H[q], P[q]);
        const uint32_t O = glint_codes_odd(H[q], P[q]);
        r[8 * q + 0] = glint_lds_f32(ltab, glint_cell_addr<0>(E, lane4)) * a;
        r[8 * q + 1] = glint_lds_f32(ltab, glint_cell_addr<0>(O, lane4)) * a;
        r[8 * q + 2] = glint_lds_f32(ltab, glint_cell_addr<1>(E, lane4)) * a;
        r[8 * q + 3] = glint_lds_f32(ltab, glint_cell_addr<1>(O, lane4)) * a;
        r[8 * q + 4] = glint_lds_f32(ltab, glint_cell_addr<2>(E, lane4)) * a;
        r[8 * q + 5] = glint_lds_f32(ltab, glint_cell_addr<2>(O, lane4)) * a;
        r[8 * q + 6] = glint_lds_f32(ltab, glint_cell_addr<3>(E, lane4)) * a;
        r[8 * q + 7] = glint_lds_f32(ltab, glint_cell_addr<3>(O, lane4)) * a;
    }
    if (BF16) {
        glint_u32x4 *o = (glint_u32x4 *)out + g * 4;
        if (a == a) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                glint_store_out(
                    glint_u32x4{glint_pack_bf16x2(r[8 * q], r[8 * q + 1]), glint_pack_bf16x2(r[8 * q + 2], r[8 * q + 3]),
                                glint_pack_bf16x2(r[8 * q + 4], r[8 * q + 5]), glint_pack_bf16x2(r[8 * q + 6], r[8 * q + 7])},
                    &o[q]);
        } else { /* NaN absmax: the reference NaN rule for every element */
            uint16_t *o16 = (uint16_t *)out + g * 32;
            for (int j = 0; j < 32; ++j)
                o16[j] = glint_f32_to_bf16(r[j]);
        }
    } else {
        glint_f32x4 *o = (glint_f32x4 *)out + g * 8;
#pragma unroll
        for (int q = 0; q < 8; ++q)
            glint_store_out(glint_f32x4{r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3]}, &o[q]);
    }
}

template <bool BF16>
__global__ __launch_bounds__(EXPAND_THREADS) void k_expand_fast(const glint_u32x4 *__restrict__ hole,
                                                                const glint_u32x4 *__restrict__ plug,
                                                                const float *__restrict__ absmax, void *__restrict__ out,
                                                                int64_t ngroups, int bs) {
    __shared__ __attribute__((aligned(16))) float ltab[GLINT_LDS_CELLS64_WORDS];
    __shared__ float stage[256];
    const uint32_t lane4 = (threadIdx.x & 63) * 4u;
    const int64_t nthreads = (int64_t)gridDim.x * EXPAND_THREADS;
    const int64_t t0 = (int64_t)blockIdx.x * EXPAND_THREADS + threadIdx.x;
    const int gpb = bs >> 5; /* groups per absmax block */
    /* first batch of loads goes out before the table fill */
    glint_u32x4 hv[EXPAND_U], pv[EXPAND_U];
    float av[EXPAND_U];
    int64_t g = t0;
#pragma unroll
    for (int u = 0; u < EXPAND_U; ++u) {
        const int64_t gu = min(g + u * nthreads, ngroups - 1);
        hv[u] = __builtin_nontemporal_load(&hole[gu]);
        pv[u] = __builtin_nontemporal_load(&plug[gu]);
        av[u] = absmax[gu / gpb];
    }
    glint_fill_cells_lds64(ltab, stage);
    for (; g < ngroups; g += EXPAND_U * nthreads) {
#pragma unroll
        for (int u = 0; u < EXPAND_U; ++u) {
            const int64_t gu = g + u * nthreads;
            if (gu < ngroups)
                expand_group<BF16>(ltab, lane4, hv[u], pv[u], av[u], out, gu);
            const int64_t gn = min(gu + EXPAND_U * nthreads, ngroups - 1);
            hv[u] = __builtin_nontemporal_load(&hole[gn]);
            pv[u] = __builtin_nontemporal_load(&plug[gn]);
            av[u] = absmax[gn / gpb];
        }
    }
}

/* One element per thread over [i0, n): any bs, any alignment. */
template <bool BF16>
__global__ __launch_bounds__(256) void k_expand_generic(const uint8_t *__restrict__ hole, const uint8_t *__restrict__ plug,
                                                        const float *__restrict__ absmax, void *__restrict__ out,
                                                        int64_t i0, int64_t n, int bs) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = i0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int sh = (int)(i & 1) * 4;
        const float r = kCells[(hole[i >> 1] >> sh) & 15][(plug[i >> 1] >> sh) & 15] * absmax[i / bs];
        if (BF16)
            ((uint16_t *)out)[i] = glint_f32_to_bf16(r);
        else
            ((float *)out)[i] = r;
    }
}

/* Run-mapped expand (power-of-two bs >= 8, n % 2048 == 0 part): a wave chunk is 256 runs of
 * 8 elements; lane l owns runs 64 s + l (s < 4), i.e. one dword of each plane per run, so
 * every plane load of a wave reads 256 B contiguous and every BF16 store writes 1 KiB
 * contiguous (f32: two 16-B stores, 2 KiB). Chunks are double-buffered in registers with
 * unconditional (clamped) loads in full rounds. */
#ifndef EXPANDR_THREADS
#define EXPANDR_THREADS 512 /* 14336 x 4096 BF16 32.8 -> 30.8 us against 1024 (both two per CU, the table's LDS) */
#endif
#ifndef EXPANDR_GRID_DIV
#define EXPANDR_GRID_DIV 2 /* launch the resident grid / this: one workgroup (8 waves) per CU streams best */
#endif
#ifndef EXPANDR_HWCVT
#define EXPANDR_HWCVT 1 /* BF16 by v_cvt_pk_bf16_f32 (RNE); NaN absmax takes the scalar rule */
#endif

struct ExpandChunk {
    uint32_t h[4], p[4];
    float a[4];
};

/* Loads of wave chunk c: runs c*256 + 64 s + lane. `abase` = c * (2048 >> shift) is the
 * chunk's first absmax index (bs <= 2048, so a chunk starts on a block boundary). */
__device__ __forceinline__ void expand_load_chunk(const uint32_t *__restrict__ hole, const uint32_t *__restrict__ plug,
                                                  const float *__restrict__ absmax, int64_t c, int lane, int shift,
                                                  ExpandChunk &ck) {
    const uint32_t *h = hole + c * 256, *p = plug + c * 256;
    const float *a = absmax + (c << (11 - shift));
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        ck.h[s] = __builtin_nontemporal_load(h + s * 64 + lane);
        ck.p[s] = __builtin_nontemporal_load(p + s * 64 + lane);
        ck.a[s] = a[(uint32_t)(s * 512 + lane * 8) >> shift];
    }
}

__device__ __forceinline__ uint32_t expand_pack2(float lo, float hi) {
#if EXPANDR_HWCVT
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
#else
    return glint_pack_bf16x2(lo, hi);
#endif
}

template <bool BF16>
__device__ __forceinline__ void expand_chunk(const float *ltab, uint32_t lane4, const ExpandChunk &ck, void *__restrict__ out,
                                             int64_t c, int lane) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t E = glint_codes_even(ck.h[s], ck.p[s]);
        const uint32_t O = glint_codes_odd(ck.h[s], ck.p[s]);
        const float a = ck.a[s];
        float r[8];
        r[0] = glint_lds_f32(ltab, glint_cell_addr<0>(E, lane4)) * a;
        r[1] = glint_lds_f32(ltab, glint_cell_addr<0>(O, lane4)) * a;
        r[2] = glint_lds_f32(ltab, glint_cell_addr<1>(E, lane4)) * a;
        r[3] = glint_lds_f32(ltab, glint_cell_addr<1>(O, lane4)) * a;
        r[4] = glint_lds_f32(ltab, glint_cell_addr<2>(E, lane4)) * a;
        r[5] = glint_lds_f32(ltab, glint_cell_addr<2>(O, lane4)) * a;
        r[6] = glint_lds_f32(ltab, glint_cell_addr<3>(E, lane4)) * a;
        r[7] = glint_lds_f32(ltab, glint_cell_addr<3>(O, lane4)) * a;
        const int64_t run = c * 256 + s * 64 + lane;
        if (BF16) {
            glint_u32x4 v;
            if (a == a) {
                v = glint_u32x4{expand_pack2(r[0], r[1]), expand_pack2(r[2], r[3]), expand_pack2(r[4], r[5]),
                                expand_pack2(r[6], r[7])};
            } else { /* NaN absmax: the reference NaN rule for every element */
                v = glint_u32x4{(uint32_t)glint_f32_to_bf16(r[0]) | (uint32_t)glint_f32_to_bf16(r[1]) << 16,
                                (uint32_t)glint_f32_to_bf16(r[2]) | (uint32_t)glint_f32_to_bf16(r[3]) << 16,
                                (uint32_t)glint_f32_to_bf16(r[4]) | (uint32_t)glint_f32_to_bf16(r[5]) << 16,
                                (uint32_t)glint_f32_to_bf16(r[6]) | (uint32_t)glint_f32_to_bf16(r[7]) << 16};
            }
            ((glint_u32x4 *)out)[run] = v;
        } else {
            ((glint_f32x4 *)out)[2 * run] = glint_f32x4{r[0], r[1], r[2], r[3]};
            ((glint_f32x4 *)out)[2 * run + 1] = glint_f32x4{r[4], r[5], r[6], r[7]};
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <bool BF16>
__global__ __launch_bounds__(EXPANDR_THREADS) void k_expand_runs(const uint32_t *__restrict__ hole,
                                                                 const uint32_t *__restrict__ plug,
                                                                 const float *__restrict__ absmax,
                                                                 void *__restrict__ out, int64_t nchunks, int shift) {
    __shared__ __attribute__((aligned(16))) float ltab[GLINT_LDS_CELLS64_WORDS];
    const int lane = threadIdx.x & 63;
    const uint32_t lane4 = (uint32_t)lane * 4u;
    /* wave-uniform, so chunk arithmetic stays in scalar registers */
    const int wave = (int)blockIdx.x * (EXPANDR_THREADS / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = (int)gridDim.x * (EXPANDR_THREADS / 64);
    const int nch = (int)nchunks;
    const int my = wave < nch ? (nch - wave + nwaves - 1) / nwaves : 0; /* chunks wave + i nwaves */
    const int last = nch - 1;
    GlintCellFill fill;
    glint_cells_fill_load(fill);
    ExpandChunk ca, cb;
    expand_load_chunk(hole, plug, absmax, min(wave, last), lane, shift, ca);
    expand_load_chunk(hole, plug, absmax, min(wave + nwaves, last), lane, shift, cb);
    glint_cells_fill_store(ltab, fill);
    __syncthreads();
    int i = 0;
    for (; i + 2 <= my; i += 2) {
        expand_chunk<BF16>(ltab, lane4, ca, out, wave + i * nwaves, lane);
        expand_load_chunk(hole, plug, absmax, min(wave + (i + 2) * nwaves, last), lane, shift, ca);
        expand_chunk<BF16>(ltab, lane4, cb, out, wave + (i + 1) * nwaves, lane);
        expand_load_chunk(hole, plug, absmax, min(wave + (i + 3) * nwaves, last), lane, shift, cb);
    }
    if (i < my)
        expand_chunk<BF16>(ltab, lane4, ca, out, (int64_t)wave + (int64_t)i * nwaves, lane);
}

template <bool BF16>
static int expand_device(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_am, int64_t n, int bs, void *d_out,
                         hipStream_t st) {
    if (!d_hole || !d_plug || !d_am || !d_out || bs <= 0)
        return -1;
    if (n <= 0)
        return 0;
    const int cus = glint_num_cus();
    int64_t n_fast = 0;
    const bool aligned = glint_aligned(d_hole, 16) && glint_aligned(d_plug, 16) && glint_aligned(d_am, 4) &&
                         glint_aligned(d_out, 16);
    if (aligned && bs >= 8 && bs <= 2048 && (bs & (bs - 1)) == 0 && n >= 2048 && n / 2048 < (1LL << 30)) {
        n_fast = (n / 2048) * 2048;
        const int64_t nchunks = n_fast / 2048;
        const int64_t resident = std::max<int64_t>(1, glint_resident_grid((const void *)k_expand_runs<BF16>, EXPANDR_THREADS, 0) / EXPANDR_GRID_DIV);
        const int64_t wanted = (nchunks + EXPANDR_THREADS / 64 - 1) / (EXPANDR_THREADS / 64);
        const unsigned grid = (unsigned)(wanted < resident ? wanted : resident);
        /* one launch: split into pieces as the encode is, the 525 M-element embedding
         * expanded at 59% of HBM against 62% whole */
        k_expand_runs<BF16><<<grid, EXPANDR_THREADS, 0, st>>>((const uint32_t *)d_hole, (const uint32_t *)d_plug, d_am,
                                                               d_out, nchunks, __builtin_ctz((unsigned)bs));
    } else if (aligned && bs % 32 == 0 && n >= 32) { /* ngroups >= 1: the kernel clamps to ngroups - 1 */
        n_fast = (n / 32) * 32;
        const int64_t ngroups = n_fast / 32;
        const int resident = (int)glint_resident_grid((const void *)k_expand_fast<BF16>, EXPAND_THREADS, 0);
        k_expand_fast<BF16><<<glint_grid(ngroups, EXPAND_THREADS * EXPAND_U, resident), EXPAND_THREADS, 0, st>>>(
            (const glint_u32x4 *)d_hole, (const glint_u32x4 *)d_plug, d_am, d_out, ngroups, bs);
    }
    if (n_fast < n)
        k_expand_generic<BF16><<<glint_grid(n - n_fast, 256, cus * 16), 256, 0, st>>>(d_hole, d_plug, d_am, d_out,
                                                                                      n_fast, n, bs);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* ------------------------------------------------------------------ C ABI */
GLINT_API int glint_encode_n_absmax(int64_t n, int blocksize) {
    if (blocksize <= 0)
        return 0;
    return (int)((n + blocksize - 1) / blocksize);
}

GLINT_API int glint_encode_n_packed(int64_t n) { return (int)((n + 1) / 2); }

GLINT_API int glint_encode_bf16_device(const uint16_t *d_w, int64_t n, int bs, uint8_t *d_hole, uint8_t *d_plug,
                                       float *d_absmax, struct ihipStream_t *stream) {
    return encode_device<uint16_t>(d_w, n, bs, d_hole, d_plug, d_absmax, (hipStream_t)stream);
}

GLINT_API int glint_encode_f32_device(const float *d_w, int64_t n, int bs, uint8_t *d_hole, uint8_t *d_plug,
                                      float *d_absmax, struct ihipStream_t *stream) {
    return encode_device<float>(d_w, n, bs, d_hole, d_plug, d_absmax, (hipStream_t)stream);
}

/* Host-pointer encode: allocate, copy in, encode, copy out, free (synchronous). */
template <typename T>
static int encode_host(const T *w, int64_t n, int bs, uint8_t *hole, uint8_t *plug, float *absmax) {
    if (n < 0 || bs <= 0)
        return -1;
    if (n == 0)
        return 0;
    if (!w || !hole || !plug || !absmax)
        return -1;
    const size_t npack = (size_t)((n + 1) / 2), nam = (size_t)((n + bs - 1) / bs);
    T *d_w = nullptr;
    uint8_t *d_h = nullptr, *d_p = nullptr;
    float *d_a = nullptr;
    int rc = -1;
    if (hipMalloc((void **)&d_w, (size_t)n * sizeof(T)) != hipSuccess || hipMalloc((void **)&d_h, npack) != hipSuccess ||
        hipMalloc((void **)&d_p, npack) != hipSuccess || hipMalloc((void **)&d_a, nam * sizeof(float)) != hipSuccess)
        goto done;
    if (hipMemcpy(d_w, w, (size_t)n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
        goto done;
    rc = -3;
    if (encode_device<T>(d_w, n, bs, d_h, d_p, d_a, 0) != 0 || hipDeviceSynchronize() != hipSuccess)
        goto done;
    if (hipMemcpy(hole, d_h, npack, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(plug, d_p, npack, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(absmax, d_a, nam * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess)
        goto done;
    rc = 0;
done:
    (void)hipFree(d_w);
    (void)hipFree(d_h);
    (void)hipFree(d_p);
    (void)hipFree(d_a);
    return rc;
}

GLINT_API int glint_encode_bf16_host(const uint16_t *w, int64_t n, int bs, uint8_t *hole, uint8_t *plug, float *absmax) {
    return encode_host<uint16_t>(w, n, bs, hole, plug, absmax);
}

GLINT_API int glint_encode_f32_host(const float *w, int64_t n, int bs, uint8_t *hole, uint8_t *plug, float *absmax) {
    return encode_host<float>(w, n, bs, hole, plug, absmax);
}

template <bool BF16>
static int expand_host(const uint8_t *hole, const uint8_t *plug, const float *absmax, int64_t n, int bs, void *out) {
    if (bs <= 0 || n < 0)
        return -1;
    if (n == 0)
        return 0;
    if (!hole || !plug || !absmax || !out)
        return -1;
    const size_t npack = (size_t)((n + 1) / 2), nam = (size_t)((n + bs - 1) / bs);
    const size_t out_bytes = (size_t)n * (BF16 ? 2 : 4);
    uint8_t *d_h = nullptr, *d_p = nullptr;
    float *d_a = nullptr;
    void *d_o = nullptr;
    int rc = -3;
    if (hipMalloc((void **)&d_h, npack) != hipSuccess || hipMalloc((void **)&d_p, npack) != hipSuccess ||
        hipMalloc((void **)&d_a, nam * sizeof(float)) != hipSuccess || hipMalloc(&d_o, out_bytes) != hipSuccess)
        goto done;
    if (hipMemcpy(d_h, hole, npack, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d_p, plug, npack, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d_a, absmax, nam * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
        goto done;
    if (expand_device<BF16>(d_h, d_p, d_a, n, bs, d_o, 0) != 0 || hipDeviceSynchronize() != hipSuccess)
        goto done;
    if (hipMemcpy(out, d_o, out_bytes, hipMemcpyDeviceToHost) != hipSuccess)
        goto done;
    rc = 0;
done:
    (void)hipFree(d_h);
    (void)hipFree(d_p);
    (void)hipFree(d_a);
    (void)hipFree(d_o);
    return rc;
}

GLINT_API int glint_expand_packed_to_f32_host(const uint8_t *hole, const uint8_t *plug, const float *absmax, int64_t n,
                                              int bs, float *out) {
    return expand_host<false>(hole, plug, absmax, n, bs, out);
}

GLINT_API int glint_expand_packed_to_bf16_host(const uint8_t *hole, const uint8_t *plug, const float *absmax, int64_t n,
                                               int bs, uint16_t *out) {
    return expand_host<true>(hole, plug, absmax, n, bs, out);
}

GLINT_API int glint_expand_packed_to_f32_device(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                                                int64_t n, int bs, float *d_out, struct ihipStream_t *stream) {
    return expand_device<false>(d_hole, d_plug, d_absmax, n, bs, d_out, (hipStream_t)stream);
}

GLINT_API int glint_expand_packed_to_bf16_device(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                                                 int64_t n, int bs, uint16_t *d_out, struct ihipStream_t *stream) {
    return expand_device<true>(d_hole, d_plug, d_absmax, n, bs, d_out, (hipStream_t)stream);
}
