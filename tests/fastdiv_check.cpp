// Checks hlm::fast_div (the multiply-high division of attn_common.h) against
// the compiler's integer division, on the host: every divisor up to 5000 with
// a sweep of dividends including the range ends, and dividends up to 2^22 for
// the divisors the producer meets (head counts, sequence lengths).  Prints
// "ok <cases>" or the first mismatch.
#include <cstdio>
#include <cstdlib>

#include "../hackable-lm_amd/hlm_attn/csrc/attn_common.h"

static long long g_cases = 0;

static bool check(int n, unsigned d) {
  const hlm::FastDiv f = hlm::fast_div_of(d);
  ++g_cases;
  if (hlm::fast_div(n, f) != (int)((unsigned)n / d)) {
    std::printf("mismatch n=%d d=%u got %d want %d (mul %u shift %d)\n", n, d, hlm::fast_div(n, f),
                (int)((unsigned)n / d), f.mul, f.shift);
    return false;
  }
  return true;
}

int main() {
  const int nmax = 0x7fffffff;
  for (unsigned d = 1; d <= 5000; ++d) {
    const hlm::FastDiv f = hlm::fast_div_of(d);
    if (f.shift < 31 || f.shift > 62) { std::printf("bad shift %d for d=%u\n", f.shift, d); return 1; }
    for (int n = 0; n < 3 * (int)d + 5; ++n)
      if (!check(n, d)) return 1;
    for (long long n = nmax; n > (long long)nmax - 3 * d - 5; --n)
      if (!check((int)n, d)) return 1;
    for (long long n = 7; n < nmax; n = n * 3 + 1)
      for (int e = -1; e <= 1; ++e)
        if (!check((int)(n + e), d)) return 1;
  }
  const unsigned ds[] = {2, 3, 4, 6, 8, 12, 16, 24, 25, 48, 96, 100, 128, 1000, 1024, 2047, 2048, 4096, 8191, 8192,
                         16384, 65536, 100003, 1u << 20, (1u << 30) + 1, 0x7fffffffu};
  for (unsigned d : ds)
    for (int n = 0; n < (1 << 22); ++n)
      if (!check(n, d)) return 1;
  std::printf("ok %lld\n", g_cases);
  return 0;
}
