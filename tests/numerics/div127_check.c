/* div127_check.c - exhaustive check behind q8_1_scale (tinystrata_amd/csrc/tsx_device.hpp): for every non-negative
 * finite float a, Markstein's corrected product with the correctly rounded reciprocal of 127,
 *   q0 = a * RN(1/127);  d = fma(fma(-127, q0, a), RN(1/127), q0)
 * equals the IEEE quotient a / 127.  Prints the number of mismatches (0 expected).  Built and run by
 * tests/test_numerics.py; plain C, any host. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const float R = 1.0f / 127.0f;
    unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t i = 0; i < (int64_t) 0x7F800000; ++i) {
        const uint32_t b = (uint32_t) i;
        float a;
        memcpy(&a, &b, 4);
        const float q0 = a * R;
        const float d = fmaf(fmaf(-127.0f, q0, a), R, q0);
        const float e = a / 127.0f;
        if (memcmp(&d, &e, 4) != 0) ++bad;
    }
    printf("mismatches %llu\n", bad);
    return 0;
}
