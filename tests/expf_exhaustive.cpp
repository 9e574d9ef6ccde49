// Exhaustive check of anedvd::expf_exact (the routing kernel's exp) against the
// host libm expf over all 2^32 float inputs.  Built and run by tests/test_expf.py.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "expf_exact.h"

int main()
{
    static const uint64_t tab[32] = ANEDVD_EXP2_TABLE;
    long long bad = 0, checked = 0;
#pragma omp parallel for reduction(+ : bad, checked) schedule(static)
    for (long long b = 0; b < (1LL << 32); b++) {
        uint32_t u = (uint32_t)b;
        float x;
        memcpy(&x, &u, 4);
        float want = expf(x), got = anedvd::expf_exact(x, tab);
        uint32_t wu, gu;
        memcpy(&wu, &want, 4);
        memcpy(&gu, &got, 4);
        int same = (wu == gu) || (isnan(want) && isnan(got));
        if (!same) {
            if (bad < 5) printf("mismatch x=%a libm=%a mine=%a\n", x, want, got);
            bad++;
        }
        checked++;
    }
    printf("checked %lld mismatches %lld\n", checked, bad);
    return bad != 0;
}
