/* Exhaustive check of the three-plane BF16 split behind the f32-out H-TILE on MFMA.
 *
 * For an f32 weight w the kernel (GlintTileProducer::finish_split) forms
 *     hi  = w with its low 16 bits cleared,
 *     r1  = RN(w - hi)          (0 instead when w is infinite),
 *     mid = r1 with its low 16 bits cleared,
 *     lo  = RN(r1 - mid),
 * and stores the upper 16 bits of each as a BF16 operand. The MFMA then multiplies every
 * plane with the BF16 x, so y sums x * w exactly term by term iff, for every w,
 *   1. both subtractions are exact, and hi + mid + lo == w (checked in double);
 *   2. lo has no bits below its upper 16 (lo is a BF16 value as it stands).
 * This walks every f32 bit pattern. Both properties hold for every finite w with
 * |w| >= 2^-110 (below, lo can fall under the smallest normal and its low bits carry
 * weight; the error is then < 2^-126 absolute); an infinite w gives (hi, mid, lo) =
 * (w, 0, 0); a NaN w gives a NaN hi. In the kernel w is the product CELLS * absmax, so a
 * NaN w is quiet (bit 22 set, in the upper half); signaling patterns are not walked.
 * Exit 0 when that holds.
 * Build: gcc -O2 -ffp-contract=off -fopenmp check_split3.c -lm */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

int main(int argc, char **argv) {
    /* `--stride S` walks every S-th pattern only (the sanitizer build's quick pass) */
    int64_t stride = 1;
    if (argc == 3 && strcmp(argv[1], "--stride") == 0)
        stride = atoll(argv[2]);
    if (stride < 1)
        return 2;
    long bad_sum = 0, bad_lo = 0, bad_special = 0, tiny = 0, checked = 0;
#pragma omp parallel for reduction(+ : bad_sum, bad_lo, bad_special, tiny, checked) schedule(static, 1 << 16)
    for (int64_t b = 0; b < ((int64_t)1 << 32); b += stride) {
        if (((uint32_t)b & 0x7FC00000u) == 0x7F800000u && ((uint32_t)b & 0x003FFFFFu) != 0)
            continue; /* signaling NaN: never the result of the multiply that makes w */
        const float w = u2f((uint32_t)b);
        const float hi = u2f((uint32_t)b & 0xFFFF0000u);
        float r1 = w - hi;
        if (isinf(w))
            r1 = 0.0f;
        const float mid = u2f(f2u(r1) & 0xFFFF0000u);
        const float lo = r1 - mid;
        if (isnan(w)) {
            bad_special += !isnan(hi);
            continue;
        }
        if (isinf(w)) {
            bad_special += !(hi == w && mid == 0.0f && lo == 0.0f);
            continue;
        }
        if (fabsf(w) < 0x1p-110f) {
            ++tiny;
            continue;
        }
        ++checked;
        bad_sum += ((double)hi + (double)mid + (double)lo != (double)w) || ((double)w - hi != (double)r1);
        bad_lo += (f2u(lo) & 0xFFFFu) != 0;
    }
    printf("split3: %ld finite weights checked, %ld sums differ, %ld lo not BF16, %ld special mismatches "
           "(%ld below 2^-110 skipped)\n",
           checked, bad_sum, bad_lo, bad_special, tiny);
    return (bad_sum || bad_lo || bad_special) ? 1 : 0;
}
