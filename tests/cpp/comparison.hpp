// The pass rule the reference's tests compare results with
// (tensor/Comparison.scala:32-74): an element passes when
// |actual - expected| <= absolute + relative * |expected|, compared in double;
// a NaN or an infinity passes only where the expected value is the same one.
#pragma once

#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

namespace drift::testing {

struct Tolerance {
  double absolute = 0.0, relative = 0.0;
};

struct Comparison {
  size_t count = 0, mismatches = 0;
  long long firstMismatch = -1;
  double maxAbsolute = 0.0, maxRelative = 0.0;

  bool passed() const { return mismatches == 0; }

  std::string summary() const {
    char text[160];
    std::snprintf(text, sizeof text, "%zu/%zu mismatches%s, max absolute %.3g, max relative %.3g", mismatches, count,
                  firstMismatch < 0 ? "" : (", first at " + std::to_string(firstMismatch)).c_str(), maxAbsolute,
                  maxRelative);
    return text;
  }

  static Comparison of(const std::vector<float>& expected, const std::vector<float>& actual, Tolerance tolerance) {
    if (expected.size() != actual.size())
      throw std::invalid_argument("requirement failed: comparing " + std::to_string(actual.size()) +
                                  " values with " + std::to_string(expected.size()));
    Comparison c;
    c.count = expected.size();
    for (size_t i = 0; i < expected.size(); ++i) {
      const double reference = expected[i], value = actual[i];
      bool passes;
      if (std::isnan(reference) || std::isnan(value)) {
        passes = std::isnan(reference) && std::isnan(value);
      } else if (std::isinf(reference) || std::isinf(value)) {
        passes = reference == value;
      } else {
        const double absolute = std::fabs(value - reference);
        c.maxAbsolute = std::max(c.maxAbsolute, absolute);
        if (reference != 0) c.maxRelative = std::max(c.maxRelative, absolute / std::fabs(reference));
        passes = absolute <= tolerance.absolute + tolerance.relative * std::fabs(reference);
      }
      if (!passes) {
        if (c.firstMismatch < 0) c.firstMismatch = (long long)i;
        ++c.mismatches;
      }
    }
    return c;
  }
};

}  // namespace drift::testing
