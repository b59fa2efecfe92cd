// Host build of the device helper mass_fast (rexl3_amd/csrc/gbs_modeu.hpp), checked against the oracle's gbo_mass
// (the per-token mass definition) on every input the test writes: one "l M c2" hex-bit triple per line on stdin, the
// helper's value and the oracle's on stdout. Compiled by tests/test_mass_stream.py with hipcc as host code.
#include <cstdio>
#include <cstring>

#include "../rexl3_amd/csrc/gbs_modeu.hpp"
#include "../oracle/gbs_oracle.h"

static float bits(unsigned b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

int main() {
    unsigned a, b, c;
    while (std::scanf("%x %x %x", &a, &b, &c) == 3) {
        const float l = bits(a), M = bits(b), c2 = bits(c);
        // the fast form is defined where its preconditions hold; elsewhere the kernels call mass() itself
        const bool ok = gbs::modeu::mass_fast_ok(M, c2) && (l <= M || l == -INFINITY);
        const unsigned long long want = gbo_mass(l, M, c2);
        const unsigned long long got = ok ? gbs::modeu::mass_fast(l, M, c2) : want;
        std::printf("%llu %llu\n", got, want);
    }
    return 0;
}
