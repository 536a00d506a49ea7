// Compares hg::hg_expf with the C library's expf on every binary32 input.
// Built and run by tests/test_expf.py; prints "<variant> <mismatches>".
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "hg_expf.h"

int main() {
    unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long u = 0; u <= 0xffffffffLL; u++) {
        uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        float a = expf(x), c = hg::hg_expf(x);
        uint32_t ab, cb;
        memcpy(&ab, &a, 4);
        memcpy(&cb, &c, 4);
        if (ab != cb && !(std::isnan(a) && std::isnan(c))) bad++;
    }
    printf("%d %llu\n", HG_EXPF_VARIANT, bad);
    return 0;
}
