// Checks the kernels' host-computed fast division (FastDiv in
// flash-attention3_amd/csrc/fa3_bwd_internal.h) against the / operator:
// every divisor 1..5000 and a spread of larger ones, with every dividend
// 0..20000, the dividends around 2048 multiples of the divisor spread up to
// 2^31, and pseudo-random dividends below 2^31.  Exit status 1 on any mismatch.
#include <cstdint>
#include <cstdio>

#include "fa3_bwd_internal.h"

int main() {
    uint64_t state = 0x9E3779B97F4A7C15ull;
    auto next = [&]() {
        state ^= state << 13;
        state ^= state >> 7;
        state ^= state << 17;
        return state;
    };
    long long checked = 0;
    auto check = [&](int d, int n) {
        const fa3::FastDiv f = fa3::make_fastdiv(d);
        ++checked;
        if (fa3::fdiv(f, n) != n / d) {
            std::printf("mismatch: %d / %d -> %d (want %d)\n", n, d, fa3::fdiv(f, n), n / d);
            return false;
        }
        return true;
    };
    int divisors[6000];
    int nd = 0;
    for (int d = 1; d <= 5000; ++d) divisors[nd++] = d;
    for (int i = 0; i < 31; ++i) {
        const int p = 1 << i;
        divisors[nd++] = p;
        if (p > 1) divisors[nd++] = p - 1;
        if (p < (1 << 30)) divisors[nd++] = p + 1;
    }
    divisors[nd++] = 0x7FFFFFFF;
    for (int i = 0; i < nd; ++i) {
        const int d = divisors[i];
        for (int n = 0; n <= 20000; ++n)
            if (!check(d, n)) return 1;
        // around 2048 multiples of d spread over [0, 2^31)
        const long long q_max = 0x7FFFFFFFll / d;
        for (int k = 1; k <= 2048; ++k) {
            const long long m = (q_max * k / 2048) * d;
            for (int e = -1; e <= 1; ++e) {
                const long long n = m + e;
                if (n >= 0 && n < 0x7FFFFFFFll && !check(d, (int)n)) return 1;
            }
        }
        for (int r = 0; r < 2000; ++r)
            if (!check(d, (int)(next() & 0x7FFFFFFF))) return 1;
    }
    // the divisor slot of an unused map (0) divides as 1
    if (fa3::fdiv(fa3::make_fastdiv(0), 12345) != 12345) return 1;
    std::printf("fastdiv ok: %lld quotients\n", checked);
    return 0;
}
