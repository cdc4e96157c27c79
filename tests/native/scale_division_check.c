/*
 * Exhaustive-in-the-scale check of the sibling kernel's division scheme
 * (flaggems-vllm_amd/csrc/inv_rope_fp8_quant.hip, div_by_scale): for every
 * positive finite bf16 amax, s = RN(amax * RN(1/448)) as the kernel forms it,
 * and numerators x = every bf16 value of magnitude <= amax drawn on a stride
 * (plus +-amax, +-0 and the smallest magnitudes), the Markstein quotient
 *     y = RN(1/s); q0 = RN(x*y); rn = fma(s, q0, -x); q = fma(-rn, y, q0)
 * must equal IEEE x / s bit for bit whenever |x/s| >= 2^-12, and have its sign
 * below that (every e4m3 code there is +-0), including for x = +-0.
 * Prints the number of mismatches and exits non-zero if there is any.
 * Build: gcc -O2 -ffp-contract=off -mfma scale_division_check.c -lm
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float div_by_scale(float x, float s, float y)
{
    float q0 = x * y;
    /* volatile: gcc -O2 -mfma would otherwise fold the negation of rn into the
       first fma, which is not exact for signed zeros */
    volatile float rn = fmaf(s, q0, -x);
    return fmaf(-rn, y, q0);
}

int main(int argc, char** argv)
{
    int stride = argc > 1 ? atoi(argv[1]) : 7;
    const float c = (float)(1.0 / 448.0);
    const float eps = 1e-10f;
    long checked = 0, bad = 0;
    for (uint32_t a16 = 1; a16 < 0x7f80; ++a16) {
        float amax = u2f(a16 << 16);
        float s = (amax > eps ? amax : eps) * c;
        float y = 1.0f / s;
        for (uint32_t x16 = 0; x16 <= a16; x16 += (x16 + stride > a16 && x16 != a16) ? (a16 - x16) : stride) {
            for (int sg = 0; sg < 2; ++sg) {
                float x = u2f((x16 << 16) | (sg ? 0x80000000u : 0));
                float want = x / s, got = div_by_scale(x, s, y);
                ++checked;
                if (fabsf(want) >= 0x1p-12f) {
                    if (f2u(want) != f2u(got)) ++bad;
                } else if (signbit(want) != signbit(got)) {
                    ++bad;
                }
            }
            if (x16 == a16) break;
        }
    }
    printf("checked %ld quotients, %ld mismatches\n", checked, bad);
    return bad != 0;
}
