// Compares the libm expf restatement of questwend_amd/csrc/qwm_expf.h (the
// one the kernels use) with the C library's expf on every float input
// (NaNs: both must be NaN).  Prints the mismatch count and the first
// mismatching input; built and run by tests/test_expf.py.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../questwend_amd/csrc/qwm_expf.h"

int main() {
    long long bad = 0;
    unsigned long long first = ~0ull;
#pragma omp parallel for reduction(+ : bad) reduction(min : first) schedule(static)
    for (long long u = 0; u < (1LL << 32); ++u) {
        const uint32_t b = (uint32_t)u;
        float x;
        std::memcpy(&x, &b, 4);
        const float a = std::exp(x), m = qwm::libm_expf(x);
        uint32_t ua, um;
        std::memcpy(&ua, &a, 4);
        std::memcpy(&um, &m, 4);
        const bool same = std::isnan(a) ? std::isnan(m) : ua == um;
        if (!same) {
            ++bad;
            if ((unsigned long long)u < first) first = (unsigned long long)u;
        }
    }
    std::printf("%lld %llx\n", bad, first);
    return 0;
}
