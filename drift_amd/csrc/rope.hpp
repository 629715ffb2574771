// Rotary-embedding pieces shared by the rope kernels and the attention
// inputs: the per-call arguments with the inverse frequencies made as the CPU
// reference makes them, the mRoPE section rules, the token's angles, and the
// turn of a pair (ops/CpuAttention.scala:89-146, kernels/rope.h:20-51).
#pragma once

#include <cmath>
#include <cstring>

#include "common.hpp"

namespace drift {
namespace {

constexpr int kMaxPairs = 256;  // head_dim up to 512

struct RopeArgs {
  float inverse[kMaxPairs];  // per pair, as the CPU computes it
  int32_t tokens, heads, dim, rotary, layout, sections;
  int32_t s[4];
};

__device__ __forceinline__ int rope_section(int pair, const RopeArgs& p) {
  switch (p.sections) {
    case DRIFT_SECTIONS_CONTIGUOUS:
      return pair < p.s[0] ? 0 : (pair < p.s[0] + p.s[1] ? 1 : 2);
    case DRIFT_SECTIONS_INTERLEAVED:
      if (pair % 3 == 1 && pair < 3 * p.s[1]) return 1;
      if (pair % 3 == 2 && pair < 3 * p.s[2]) return 2;
      return 0;
    case DRIFT_SECTIONS_AXES:
      return pair < p.s[0] ? 0 : (pair < p.s[0] + p.s[1] ? 1 : (pair < p.s[0] + p.s[1] + p.s[2] ? 2 : 3));
    default:
      return 0;
  }
}

// The token's cos and sin for every pair, into cs (LDS), by the block.
__device__ __forceinline__ void token_angles(const RopeArgs& p, const int32_t* positions, int64_t t, double2* cs) {
  const int half = p.rotary / 2;
  for (int j = threadIdx.x; j < half; j += blockDim.x) {
    const int32_t position = positions[(int64_t)rope_section(j, p) * p.tokens + t];
    const float angle = (float)position * p.inverse[j];
    double sn, cn;
    sincos((double)angle, &sn, &cn);
    cs[j] = make_double2(cn, sn);
  }
}

// The turn of one pair (a first, b second) in double, as the CPU does it.
__device__ __forceinline__ void turn(double a, double b, double c, double s, float& first, float& second) {
  first = (float)(a * c - b * s);
  second = (float)(a * s + b * c);
}

// The same turn with one rounding per output: a*c - b*s as fma(a, c, -(b*s)).
// It differs from the two-rounding form only when the double result lies
// within a double ulp of a float rounding boundary (about 2^-28 of values).
__device__ __forceinline__ void turn_fused(double a, double b, double c, double s, float& first, float& second) {
  first = (float)fma(a, c, -(b * s));
  second = (float)fma(a, s, b * c);
}

// Pair slot j of one head (slots cover the head: j < rotary/2 turn a pair,
// the rest copy two tail values), values read by load(d) and written by
// store(d, value). Reads before it writes.
template <typename Load, typename Store>
__device__ __forceinline__ void turn_slot(int j, int dim, int rotary, int layout, const double2* cs, Load load,
                                          Store store) {
  const int half = rotary / 2;
  if (j < half) {
    const int d0 = layout == DRIFT_ROPE_NEOX ? j : 2 * j;
    const int d1 = layout == DRIFT_ROPE_NEOX ? j + half : 2 * j + 1;
    const double a = load(d0), b = load(d1);
    float f, s;
    turn(a, b, cs[j].x, cs[j].y, f, s);
    store(d0, f);
    store(d1, s);
  } else {
    const int e = rotary + 2 * (j - half);
    const float v0 = load(e);
    const float v1 = e + 1 < dim ? (float)load(e + 1) : 0.0f;
    store(e, v0);
    if (e + 1 < dim) store(e + 1, v1);
  }
}

// The same into a head row of T.
template <typename T, typename Load>
__device__ __forceinline__ void turn_slot(int j, int dim, int rotary, int layout, const double2* cs, Load load,
                                          T* head_out) {
  turn_slot(j, dim, rotary, layout, cs, load, [&](int d, float v) { store_one(head_out + d, v); });
}

// ------------------------------------------------------------------ host side

inline int check_rope(const char* entry, int32_t tokens, int32_t heads, int32_t dim, int32_t rotary, int32_t layout,
               int32_t sections, const int32_t (&s)[4]) {
  if (tokens < 0 || heads < 0) return refuse("%s: %d tokens of %d heads", entry, tokens, heads);
  if (dim <= 0 || dim > 2 * kMaxPairs) return refuse("%s: heads of %d values (at most %d)", entry, dim, 2 * kMaxPairs);
  if (rotary < 0 || rotary % 2 != 0 || rotary > dim)
    return refuse("%s: %d rotary dimensions in heads of %d", entry, rotary, dim);
  if (layout != DRIFT_ROPE_NEOX && layout != DRIFT_ROPE_INTERLEAVED) return refuse("%s: no layout %d", entry, layout);
  if (sections < DRIFT_SECTIONS_SINGLE || sections > DRIFT_SECTIONS_AXES)
    return refuse("%s: no sections %d", entry, sections);
  if (sections == DRIFT_SECTIONS_AXES) {
    int count = 0, sum = 0;
    for (int a = 0; a < 4; ++a) {
      if (s[a] < 0 || (s[a] == 0 && a + 1 < 4 && s[a + 1] > 0))
        return refuse("%s: axes of %d %d %d %d pairs", entry, s[0], s[1], s[2], s[3]);
      count += s[a] > 0;
      sum += s[a];
    }
    if (count == 0 || 2 * sum != rotary)
      return refuse("%s: axes of %d %d %d %d pairs for %d rotary values", entry, s[0], s[1], s[2], s[3], rotary);
  }
  if ((sections == DRIFT_SECTIONS_CONTIGUOUS || sections == DRIFT_SECTIONS_INTERLEAVED) &&
      (s[0] < 0 || s[1] < 0 || s[2] < 0))
    return refuse("%s: sections %d %d %d", entry, s[0], s[1], s[2]);
  return 0;
}

// The inverse frequencies as the CPU reference makes them
// (ops/CpuAttention.scala:124-133).
inline void make_inverse(float (&inverse)[kMaxPairs], int32_t rotary, float theta, int32_t sections,
                         const int32_t (&s)[4]) {
  for (int pair = 0; pair < kMaxPairs; ++pair) {
    if (pair >= rotary / 2) {
      inverse[pair] = 0.0f;
      continue;
    }
    double exponent = 2.0 * pair / (double)rotary;
    if (sections == DRIFT_SECTIONS_AXES) {
      int start = 0, axis = 0;
      while (pair >= start + s[axis]) start += s[axis++];
      exponent = (double)(pair - start) / (double)s[axis];
    }
    inverse[pair] = 1.0f / (float)std::pow((double)theta, exponent);
  }
}

// A launch's rope arguments. The inverse frequencies depend only on (theta,
// rotary, sections and their sizes), which a model keeps for every layer, so
// each host thread keeps those of its last four configurations: a decode
// step's launches copy the table instead of taking up to 256 pow calls.
inline void fill_rope(RopeArgs& p, int32_t tokens, int32_t heads, int32_t dim, int32_t rotary, float theta, int32_t layout,
               int32_t sections, const int32_t (&s)[4]) {
  p.tokens = tokens;
  p.heads = heads;
  p.dim = dim;
  p.rotary = rotary;
  p.layout = layout;
  p.sections = sections;
  for (int a = 0; a < 4; ++a) p.s[a] = s[a];
  struct Tables {
    struct Key {
      float theta;
      int32_t rotary, sections, s[4];
    } key;
    float inverse[kMaxPairs];
    bool used;
  };
  constexpr int kKept = 4;
  thread_local Tables kept[kKept] = {};
  thread_local int next = 0;
  Tables::Key key;
  std::memset(&key, 0, sizeof key);  // no padding left undefined for the comparison
  key.theta = theta;
  key.rotary = rotary;
  key.sections = sections;
  for (int a = 0; a < 4; ++a) key.s[a] = s[a];
  for (Tables& t : kept)
    if (t.used && std::memcmp(&t.key, &key, sizeof key) == 0) {
      std::memcpy(p.inverse, t.inverse, sizeof p.inverse);
      return;
    }
  Tables& t = kept[next];
  next = (next + 1) % kKept;
  t.key = key;
  make_inverse(t.inverse, rotary, theta, sections, s);
  t.used = true;
  std::memcpy(p.inverse, t.inverse, sizeof p.inverse);
}

}  // namespace
}  // namespace drift
