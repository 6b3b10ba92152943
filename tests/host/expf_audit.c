/* expf_audit.c - the device's restatement of the engine's expf (k3g_expf.h, compiled here
 * for the host) against this machine's C library expf on every one of the 2^32 float
 * inputs: the same bits everywhere (NaN for NaN). Prints the mismatch count and the first
 * few mismatches; exit status 0 only when there are none. With an argument "table", prints
 * the 32 table entries instead (checked against 2^(i/32) by the Python test). */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "k3g_expf.h"

int main(int argc, char **argv)
{
    if (argc > 1 && !strcmp(argv[1], "table")) {
        for (int i = 0; i < 32; ++i) printf("%016llx\n", (unsigned long long)k3x_exp2_tab(i));
        return 0;
    }
    long long bad = 0;
    unsigned first[8];
    int nfirst = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 16)
    for (long long i = 0; i < (1ll << 32); ++i) {
        const unsigned u = (unsigned)i;
        float x, a, b;
        memcpy(&x, &u, 4);
        a = expf(x);
        b = k3x_expf(x);
        unsigned ua, ub;
        memcpy(&ua, &a, 4);
        memcpy(&ub, &b, 4);
        if (ua != ub && !(isnan(a) && isnan(b))) {
            ++bad;
#pragma omp critical
            if (nfirst < 8) first[nfirst++] = u;
        }
    }
    printf("mismatches %lld\n", bad);
    for (int i = 0; i < nfirst; ++i) {
        float x;
        memcpy(&x, &first[i], 4);
        printf("  x = %a (0x%08x): libm %a, restatement %a\n", x, first[i], expf(x), k3x_expf(x));
    }
    return bad ? 1 : 0;
}
