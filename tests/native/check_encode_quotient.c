/* Exhaustive check of the encode's fast quotient for bf16 inputs.
 *
 * For a block absmax s with 2^-90 <= s < 2^90 (no NaN or inf in the block) the encode
 * looks the code up from
 *     y = RN(1/s)  (bits R(m) - bits(s), R(m) = bits(RN(1/(1 + m/128))) + 0x3F800000 + (m << 16)
 *                   for the 7-bit mantissa field m of s),
 *     q = RN(w * y)
 * instead of the correctly rounded v = RN(w / s) the format defines. q can differ from v
 * by an ulp; what must hold is that the code does not. This program walks every bf16 s in
 * that range and every bf16 w with |w| <= s, both signs, and checks:
 *   1. the bits R(m) - bits(s) equal RN(1/s) (the table identity);
 *   2. |q| <= 1, so the bucket lookup needs no clamp (bucket in [0, 512]);
 *   3. code(q) == code(v) by the reference's first-minimum scan;
 *   4. the same with q flushed to zero when subnormal (a flush-to-zero multiply).
 * Exit 0 when all hold for every pair.
 * Build: gcc -O2 -ffp-contract=off -fopenmp -I include -I glint_amd/csrc check_encode_quotient.c -lm */
#include "glint_cells.h"
#include "glint_codebook.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bf(uint32_t b16) { return glint_u2f(b16 << 16); }

int main(int argc, char **argv) {
    /* `--stride S` takes every S-th absmax only (the sanitizer build's quick pass) */
    uint32_t stride = 1;
    if (argc == 3 && strcmp(argv[1], "--stride") == 0)
        stride = (uint32_t)atoi(argv[2]);
    if (stride < 1)
        return 2;
    const uint32_t s_lo = 0x12800000u >> 16, s_hi = 0x6C800000u >> 16; /* 2^-90, 2^90 */
    const float *par = GLINT_PARENT, *cel = &GLINT_CELLS[0][0];
    long pairs = 0, recip_bad = 0, range_bad = 0, code_bad = 0, ftz_bad = 0, q_differs = 0;
#pragma omp parallel for reduction(+ : pairs, recip_bad, range_bad, code_bad, ftz_bad, q_differs) schedule(dynamic, 16)
    for (uint32_t sb = s_lo; sb < s_hi; sb += stride) {
        const uint32_t sbits = sb << 16, m = sb & 127u;
        const float s = glint_u2f(sbits);
        const uint32_t R = glint_f2u(1.0f / (1.0f + (float)m * 0.0078125f)) + 0x3F800000u + (m << 16);
        const float y = glint_u2f(R - sbits);
        if (glint_f2u(y) != glint_f2u(1.0f / s))
            ++recip_bad;
        for (uint32_t wb = 0; wb <= sb; ++wb) {
            for (int neg = 0; neg < 2; ++neg) {
                const float w = neg ? -bf(wb) : bf(wb);
                const float q = w * y;
                const float v = w / s;
                ++pairs;
                if (!(fabsf(q) <= 1.0f))
                    ++range_bad;
                if (glint_f2u(q) != glint_f2u(v))
                    ++q_differs;
                const int want = glint_code_scan(par, cel, v);
                if (glint_code_scan(par, cel, q) != want)
                    ++code_bad;
                const float qz = fabsf(q) < 0x1p-126f ? 0.0f * q : q;
                if (glint_code_scan(par, cel, qz) != want)
                    ++ftz_bad;
            }
        }
    }
    printf("quotient: %ld pairs (%ld with q != w/s); %ld reciprocal mismatches, %ld |q| > 1, "
           "%ld code mismatches, %ld flush-to-zero code mismatches\n",
           pairs, q_differs, recip_bad, range_bad, code_bad, ftz_bad);
    return (recip_bad || range_bad || code_bad || ftz_bad) ? 1 : 0;
}
