// CPU check of sb::sincos_cw (semblend_amd/csrc/sb_sincos.h) against the C library's double
// sin and cos, both rounded to float, over the RoPE angles the kernels form:
//   mode "grid": x = (float)delta * f for every delta in [-D, D] and the 64 inverse
//                frequencies (fp32) of head_dim 128 at bases 1e4, 5e5 and 1e6;
//   mode "wide": 2^20 pseudo-random fp32 angles with magnitudes up to 2^32 (an int32
//                target position minus a valid donor position, times inv_freq <= 1).
// A float that differs from the library's is accepted only when the library's double value
// lies within `tie` (relative) of the midpoint between the two floats; the program prints
// the counts and exits 1 on any other difference.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../semblend_amd/csrc/sb_sincos.h"

static long g_total = 0, g_diff = 0, g_bad = 0;
static double g_maxerr = 0.0;  // max |ours - libm| / max(|libm|, 2^-30) in double

static void check_one(float x, double tie) {
  double s, c;
  sb::sincos_cw(static_cast<double>(x), &s, &c);
  const double rs = std::sin(static_cast<double>(x)), rc = std::cos(static_cast<double>(x));
  const double pairs[2][2] = {{s, rs}, {c, rc}};
  for (const auto& p : pairs) {
    ++g_total;
    const double e = std::fabs(p[0] - p[1]) / std::fmax(std::fabs(p[1]), 0x1p-30);
    if (e > g_maxerr) g_maxerr = e;
    const float a = static_cast<float>(p[0]), b = static_cast<float>(p[1]);
    if (a == b) continue;
    ++g_diff;
    const double mid = 0.5 * (static_cast<double>(a) + static_cast<double>(b));
    if (std::fabs(p[1] - mid) > tie * std::fabs(p[1])) {
      ++g_bad;
      if (g_bad <= 5)
        std::printf("mismatch x=%.9g ours=%.17g libm=%.17g\n", x, p[0], p[1]);
    }
  }
}

int main(int argc, char** argv) {
  const char* mode = argc > 1 ? argv[1] : "grid";
  if (!std::strcmp(mode, "grid")) {
    const long D = argc > 2 ? std::atol(argv[2]) : 65536;
    const double bases[3] = {1e4, 5e5, 1e6};
    for (double base : bases)
      for (int i = 0; i < 64; ++i) {
        const float f = static_cast<float>(1.0 / std::pow(base, (2.0 * i) / 128.0));
        for (long d = -D; d <= D; ++d) check_one(static_cast<float>(d) * f, 0x1p-48);
      }
  } else {
    uint64_t st = 0x9E3779B97F4A7C15ull;
    for (int n = 0; n < (1 << 20); ++n) {
      st ^= st << 13; st ^= st >> 7; st ^= st << 17;
      const double mag = std::ldexp(1.0, static_cast<int>(st % 32)) *
                         (1.0 + static_cast<double>((st >> 8) & 0xFFFFFF) / 16777216.0);
      const float x = static_cast<float>((st >> 40) & 1 ? -mag : mag);
      check_one(x, 0x1p-38);
    }
  }
  std::printf("%s: %ld values, %ld differ from the library's rounding, %ld outside the tie "
              "band; max relative difference in double %.3g\n",
              mode, g_total, g_diff, g_bad, g_maxerr);
  return g_bad ? 1 : 0;
}
