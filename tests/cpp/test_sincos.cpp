// drift_amd/csrc/sincos.hpp on the CPU against the C library's sin and cos:
// every angle the rope kernels make for positions 0 .. 2^16 - 1 at the rope
// bases and rotary widths the runner uses (the inverse frequency as the CPU
// reference makes it: double pow, rounded to float, float reciprocal; the
// angle a float product), plus random floats of every exponent up to 2^20.
// Prints the worst distance in double ulps and how many results are more than
// one ulp away; exits nonzero past 2 ulps.
#include <cinttypes>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>

#include "../../drift_amd/csrc/sincos.hpp"

namespace {

int64_t ordered(double v) {
  int64_t b;
  std::memcpy(&b, &v, 8);
  return b < 0 ? INT64_MIN - b : b;
}

}  // namespace

int main() {
  double worst = 0;
  long checked = 0, beyond_one = 0, refused = 0;
  auto check = [&](float angle) {
    double s, c;
    if (!drift::sincos_reduced(angle, &s, &c)) {
      ++refused;
      return;
    }
    const double es = std::fabs((double)(ordered(s) - ordered(std::sin((double)angle))));
    const double ec = std::fabs((double)(ordered(c) - ordered(std::cos((double)angle))));
    worst = std::fmax(worst, std::fmax(es, ec));
    beyond_one += (es > 1) + (ec > 1);
    ++checked;
  };
  for (double theta : {1e4, 1e6, 5e5, 1e5, 1e3})
    for (int rotary : {128, 64, 96, 44, 256})
      for (int pair = 0; pair < rotary / 2; ++pair) {
        const float inverse = 1.0f / (float)std::pow(theta, 2.0 * pair / rotary);
        for (int position = 0; position < (1 << 16); ++position) check((float)position * inverse);
      }
  std::mt19937_64 g(7);
  for (int i = 0; i < 4000000; ++i) {
    uint32_t bits = (uint32_t)g();
    bits = (bits & 0x807fffffu) | ((uint32_t)(80 + g() % 67) << 23);  // exponents 2^-47 .. 2^19
    float angle;
    std::memcpy(&angle, &bits, 4);
    check(angle);
  }
  check(1048576.0f);  // outside the reduction's range: refused
  std::printf("sincos_reduced: %ld angles, worst %.0f ulp, %ld beyond 1 ulp, %ld refused\n", checked, worst,
              beyond_one, refused);
  return worst <= 2 && refused == 1 ? 0 : 1;
}
