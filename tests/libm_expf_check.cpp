// Host check of tau.rs_amd/csrc/libm_expf.hpp against the system expf.
// Usage: libm_expf_check [stride]  -- walks float bit patterns 0..2^32-1 in
// steps of `stride` (1 = every float) and prints "checked N mismatches M".
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../tau.rs_amd/csrc/libm_expf.hpp"

int main(int argc, char** argv) {
    const unsigned long long stride = argc > 1 ? strtoull(argv[1], nullptr, 10) : 1;
    unsigned long long checked = 0, mismatches = 0;
#pragma omp parallel for schedule(static) reduction(+ : checked, mismatches)
    for (unsigned long long u = 0; u < (1ull << 32); u += stride) {
        float x;
        const unsigned int bits = (unsigned int)u;
        memcpy(&x, &bits, 4);
        if (isnan(x)) continue;
        const float want = expf(x), got = tau_amd::expf_glibc(x);
        ++checked;
        if (memcmp(&want, &got, 4) != 0) {
            if (mismatches < 8) printf("x=%a expf=%a got=%a\n", x, want, got);  // per thread
            ++mismatches;
        }
    }
    printf("checked %llu mismatches %llu\n", checked, mismatches);
    return mismatches != 0;
}
