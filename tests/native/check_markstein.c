/* Exhaustive check of the encode's fast divide for bf16 inputs.
 *
 * For a block absmax s with 2^-90 <= s < 2^90 the encode computes
 *     y = RN(1/s);  q = RN(w*y);  r = RN(w - q*s) (one fma);  v = RN(q + r*y) (one fma)
 * (Markstein's correction step, P. Markstein, IBM J. Res. Dev. 34(1), 1990) instead of
 * an IEEE divide. This program walks every bf16 s in that range and every bf16 w with
 * 0 <= w <= s (the sign is symmetric) and checks:
 *   1. v has the bits of the correctly rounded w/s whenever w >= 2^-100 and w/s is a
 *      normal float (otherwise the residual r = w - q*s or the quotient itself is
 *      subnormal and loses bits; every such pair has |w/s| < 2^-10 since s >= 2^-90);
 *   2. v and w/s always map to the same GLINT code (the smallest decision threshold
 *      is 2.47e-3 > 2^-9, so every |v| < 2^-9 encodes as code 0x78).
 * Exit 0 when both hold for every pair.
 * Build: gcc -O2 -ffp-contract=off -fopenmp -I include -I glint_amd/csrc check_markstein.c -lm */
#include "glint_cells.h"
#include "glint_codebook.h"

#include <stdio.h>

static float bf(uint32_t b16) { return glint_u2f(b16 << 16); }

int main(void) {
    const uint32_t s_lo = 0x12800000u >> 16, s_hi = 0x6C800000u >> 16; /* 2^-90, 2^90 */
    const float *par = GLINT_PARENT, *cel = &GLINT_CELLS[0][0];
    long pairs = 0, bits_bad = 0, code_bad = 0, tiny_differ = 0;
#pragma omp parallel for reduction(+ : pairs, bits_bad, code_bad, tiny_differ) schedule(dynamic, 16)
    for (uint32_t sb = s_lo; sb < s_hi; ++sb) {
        const float s = bf(sb);
        const float y = 1.0f / s;
        for (uint32_t wb = 0; wb <= sb; ++wb) {
            const float w = bf(wb);
            const float q = w * y;
            const float r = fmaf(-q, s, w);
            const float v = fmaf(r, y, q);
            const float ref = w / s;
            ++pairs;
            if (glint_f2u(v) != glint_f2u(ref)) {
                if (w >= 0x1p-100f && ref >= 0x1p-126f) ++bits_bad;
                else ++tiny_differ;
            }
            if (glint_code_scan(par, cel, v) != glint_code_scan(par, cel, ref)) ++code_bad;
        }
    }
    printf("markstein: %ld pairs; %ld differ with w >= 2^-100 and w/s normal; %ld differ below; %ld code mismatches\n",
           pairs, bits_bad, tiny_differ, code_bad);
    return (bits_bad || code_bad) ? 1 : 0;
}
