/* Compares expf_ref (llamd_rs_amd/csrc/expf_ref.h, the device's exp) with the
 * host libm's expf over a range of float bit patterns. Prints the number of
 * mismatches and the first one. Used by tests/test_expf.py. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "expf_ref.h"

int main(int argc, char **argv) {
    uint64_t lo = strtoull(argv[1], 0, 0), hi = strtoull(argv[2], 0, 0), step = strtoull(argv[3], 0, 0);
    uint64_t bad = 0, n = 0;
    uint32_t first = 0;
    for (uint64_t u = lo; u <= hi; u += step) {
        uint32_t v = (uint32_t)u;
        float x, a, b;
        memcpy(&x, &v, 4);
        a = expf(x);
        b = expf_ref(x);
        uint32_t ua, ub;
        memcpy(&ua, &a, 4);
        memcpy(&ub, &b, 4);
        n++;
        if (ua != ub && !(isnan(a) && isnan(b))) {
            if (!bad) first = v;
            bad++;
        }
    }
    printf("%llu %llu %08x\n", (unsigned long long)n, (unsigned long long)bad, first);
    return 0;
}
