// expf_check — host-side check of libm_expf (bread_expf.h) against the C
// library's expf: every float input from `first` to `last` (bit patterns,
// inclusive) taken `stride` apart.  Prints the number of inputs and of
// mismatches (NaN results compare equal regardless of payload); exit status
// 0 only with no mismatch.  Built by tests/test_expf.py against the library's
// header (breadv2_amd/csrc on the include path).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "bread_expf.h"

int main(int argc, char **argv)
{
    if (argc != 4) {
        fprintf(stderr, "usage: %s FIRST_HEX LAST_HEX STRIDE\n", argv[0]);
        return 2;
    }
    const uint64_t first = strtoull(argv[1], nullptr, 16), last = strtoull(argv[2], nullptr, 16);
    const uint64_t stride = strtoull(argv[3], nullptr, 10);
    if (stride == 0 || last > 0xFFFFFFFFull || first > last) return 2;
    uint64_t n = 0, bad = 0;
    for (uint64_t u = first; u <= last; u += stride) {
        float x;
        const uint32_t b = (uint32_t)u;
        memcpy(&x, &b, 4);
        const float a = expf(x), c = libm_expf(x);
        uint32_t ua, uc;
        memcpy(&ua, &a, 4);
        memcpy(&uc, &c, 4);
        n++;
        if (ua != uc && !(isnan(a) && isnan(c))) {
            if (bad < 5) fprintf(stderr, "mismatch at %08x: libm %08x restated %08x\n", b, ua, uc);
            bad++;
        }
    }
    printf("%llu %llu\n", (unsigned long long)n, (unsigned long long)bad);
    return bad ? 1 : 0;
}
