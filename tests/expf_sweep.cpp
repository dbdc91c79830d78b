// Sweeps the device exponential's restatement (csrc/expf_ref.h, compiled for
// the host) against the host C library's expf over single-precision inputs.
// Usage: expf_sweep <stride>; prints the number of inputs whose bits differ.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "expf_ref.h"

int main(int argc, char **argv) {
    const long long stride = argc > 1 ? atoll(argv[1]) : 1;
    long long mism = 0, n = 0;
#pragma omp parallel for reduction(+ : mism, n) schedule(static)
    for (long long u = 0; u <= 0xFFFFFFFFLL; u += stride) {
        const unsigned int bits = (unsigned int)u;
        float x;
        memcpy(&x, &bits, 4);
        const float a = expf(x), b = gaje::expf_ref(x);
        unsigned int ua, ub;
        memcpy(&ua, &a, 4);
        memcpy(&ub, &b, 4);
        ++n;
        if (ua != ub && !(std::isnan(a) && std::isnan(b))) ++mism;
    }
    printf("%lld %lld\n", mism, n);
    return 0;
}
