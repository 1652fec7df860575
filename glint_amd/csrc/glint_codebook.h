/* GLINT encode decision function, shared by the host table generator, the CPU
 * verifier and the HIP kernels.
 *
 * The reference encode (cuda/glint_encode.cu:67-99, glint_np.py:41-52) maps the
 * block-scaled value v = w / absmax to a byte code c = 16*hole + plug by two
 * first-minimum linear scans in f32:
 *     hole = first argmin_k |v - PARENT[k]|,  plug = first argmin_j |v - CELLS[hole][j]|
 * (strict '<', so a tie keeps the lower index and NaN keeps index 0).
 *
 * c(v) is a non-decreasing step function of v on [-1, 1] that visits every code
 * 0..255 in order, so c(v) = #{ i : v > T_i } for 255 f32 thresholds T_1 < ... < T_255
 * (T_i = the largest float with c < i). Adjacent thresholds are >= 4.9e-3 apart,
 * more than the 1/256 width of the buckets below, so every bucket holds at most one
 * threshold and
 *     c(v) = base[b] + (v > thr[b]),   b = glint_code_bucket(v).
 * gen_code_table.c derives (thr, base) from glint_code_scan and verifies the lookup
 * against the scan for every float in [-1, 1].
 */
#ifndef GLINT_CODEBOOK_H_
#define GLINT_CODEBOOK_H_

#include <stdint.h>
#include <string.h>
#include <math.h>

#define GLINT_CODE_BUCKETS 513
/* fmaf(v, 256, GLINT_CODE_MAGIC) lands on an integer-valued float in
 * [2^23, 2^23 + 512]; its low mantissa bits are the bucket index. */
#define GLINT_CODE_MAGIC 8388864.0f       /* 2^23 + 256 */
#define GLINT_CODE_MAGIC_BITS 0x4B000000u /* bit pattern of 2^23 */

static inline uint32_t glint_f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float glint_u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* First index of the minimum of |v - tab[k]| over 16 entries (strict '<'). */
static inline int glint_first_min16(const float *tab, float v) {
    int best = 0;
    float bd = fabsf(v - tab[0]);
    for (int k = 1; k < 16; ++k) {
        const float d = fabsf(v - tab[k]);
        if (d < bd) {
            bd = d;
            best = k;
        }
    }
    return best;
}

/* Reference code of v: 16*hole + plug. */
static inline int glint_code_scan(const float *parent16, const float *cells256, float v) {
    const int h = glint_first_min16(parent16, v);
    const int p = glint_first_min16(cells256 + 16 * h, v);
    return 16 * h + p;
}

/* Bucket of v. NaN goes to bucket 0 (fmaxf returns the non-NaN operand), whose
 * base is 0 and whose compare is false for NaN, so NaN encodes to code 0 as in the
 * reference scan. Callers only pass |v| <= 1 or a quiet NaN (v is always the result
 * of an f32 divide or fma, never a signaling NaN). */
static inline uint32_t glint_code_bucket(float v) {
    const float c = fminf(fmaxf(v, -1.0f), 1.0f);
    return glint_f2u(fmaf(c, 256.0f, GLINT_CODE_MAGIC)) - GLINT_CODE_MAGIC_BITS;
}

#endif
