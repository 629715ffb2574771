/*
 * Test infrastructure only (see cpu_ops.h): a C restatement of the drift
 * runner's CPU reference backend for the fused layer kernels' path. Built with
 * -ffp-contract=off and SSE arithmetic so each double and float operation
 * rounds exactly where the JVM's does.
 */
#include "cpu_ops.h"

#include <math.h>
#include <string.h>

static uint32_t float_bits(float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  return b;
}

static float bits_float(uint32_t b) {
  float v;
  memcpy(&v, &b, 4);
  return v;
}

/* CpuOps.toBfloat16 (ops/CpuOps.scala:52-57): round to nearest even on the
 * bit pattern; a NaN keeps its top half with the quiet bit set. */
uint16_t oracle_to_bf16(float value) {
  const uint32_t bits = float_bits(value);
  if (value != value) return (uint16_t)((bits >> 16) | 0x40u);
  return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

/* DType.BF16.decodeElement (tensor/DType.scala:99-102): the top half of an F32. */
float oracle_from_bf16(uint16_t bits) { return bits_float((uint32_t)bits << 16); }

/* Float.float16ToFloat as LittleEndian.float16 uses it
 * (tensor/LittleEndian.scala:45-46): exact, subnormals included; a NaN keeps
 * its significand shifted into the float's top bits. */
float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exponent = (h >> 10) & 0x1fu;
  const uint32_t significand = h & 0x3ffu;
  if (exponent == 0) {
    /* zero or subnormal: significand x 2^-24, exact in float */
    const float magnitude = (float)significand * 0x1p-24f;
    return sign ? -magnitude : magnitude;
  }
  if (exponent == 31) return bits_float(sign | 0x7f800000u | (significand << 13));
  return bits_float(sign | ((exponent + 112u) << 23) | (significand << 13));
}

/* Float.floatToFloat16 for finite values and infinities: round to nearest
 * even, overflow to infinity, subnormal results rounded on their own grid.
 * A NaN becomes a quiet NaN with the float's top significand bits (its
 * payload is not pinned against the JDK). */
uint16_t oracle_f32_to_f16(float value) {
  const uint32_t bits = float_bits(value);
  const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  const uint32_t magnitude = bits & 0x7fffffffu;
  if (magnitude > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((magnitude >> 13) & 0x3ffu));
  if (magnitude >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: rounds to infinity */
  const int exponent = (int)(magnitude >> 23) - 127;
  if (exponent < -25) return sign; /* below half the smallest subnormal */
  uint32_t significand = (magnitude & 0x7fffffu) | 0x800000u;
  int shift; /* bits dropped from the 24-bit significand */
  uint32_t biased;
  if (exponent < -14) {
    shift = 13 + (-14 - exponent);
    biased = 0;
  } else {
    shift = 13;
    biased = (uint32_t)(exponent + 15);
    significand &= 0x7fffffu;
  }
  uint32_t kept = significand >> shift;
  const uint32_t dropped = significand & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (dropped > half || (dropped == half && (kept & 1u))) kept += 1u;
  /* a carry out of the significand moves into the exponent field */
  return (uint16_t)(sign | ((biased << 10) + kept));
}

void oracle_f32_to_bf16_n(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_to_bf16(x[i]);
}

void oracle_bf16_to_f32_n(const uint16_t* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_from_bf16(x[i]);
}

void oracle_f32_to_f16_n(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(x[i]);
}

void oracle_f16_to_f32_n(const uint16_t* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(x[i]);
}

/* CpuOps.erf (ops/CpuOps.scala:26-50): odd; the Maclaurin series of erf
 * below 2.5, summed until a term no longer moves the sum; the continued
 * fraction of erfc, 60 levels deep, from 2.5 on. */
double oracle_erf(double x) {
  if (x < 0) return -oracle_erf(-x);
  if (x < 2.5) {
    double term = x, sum = x;
    int n = 0;
    while (fabs(term) > 1e-17 * fabs(sum)) {
      n += 1;
      term *= -x * x / n;
      sum += term / (2 * n + 1);
    }
    return 2 / sqrt(M_PI) * sum;
  }
  double fraction = 0.0;
  for (int n = 60; n >= 1; --n) fraction = (n / 2.0) / (x + fraction);
  return 1 - exp(-x * x) / sqrt(M_PI) / (x + fraction);
}

/* CpuNormalisation.activate (ops/CpuNormalisation.scala:11-20); kinds as
 * ops/Activation.scala:6-20: 0 SiLU, 1 GELU-tanh, 2 GELU-erf, 3 sigmoid,
 * 4 SiTU. */
double oracle_activate(int kind, double v) {
  switch (kind) {
    case 0:
      return v / (1 + exp(-v));
    case 1:
      return 0.5 * v * (1 + tanh(sqrt(2 / M_PI) * (v + 0.044715 * v * v * v)));
    case 2:
      return 0.5 * v * (1 + oracle_erf(v / sqrt(2)));
    case 3:
      return 1 / (1 + exp(-v));
    default:
      return 4 * tanh(v / 4) / (1 + exp(-v));
  }
}

/* CpuNormalisation.gatedUp (ops/CpuNormalisation.scala:22-24) */
static double gated_up(int kind, double v) { return kind == 4 ? 25 * tanh(v / 25) : v; }

/* CpuNormalisation.scaledActivation (ops/CpuNormalisation.scala:26-35): the
 * input scale, a float, multiplies the value in double. */
void oracle_activation(int kind, float input_scale, const float* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = (float)oracle_activate(kind, (double)input_scale * (double)x[i]);
}

/* CpuNormalisation.gated (ops/CpuNormalisation.scala:37-41) */
void oracle_gated(int kind, const float* gate, const float* up, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = (float)(oracle_activate(kind, (double)gate[i]) * gated_up(kind, (double)up[i]));
}

/* Ops.addRmsNorm's two steps (ops/NormalisationOps.scala:42-45): add
 * (ops/CpuElementwise.scala:9-13), then CpuNormalisation.rmsNorm
 * (ops/CpuNormalisation.scala:53-71): the squares summed in double, the factor
 * 1/sqrt(mean + eps) in double, each value x * factor * (w + offset) in
 * double, rounded to float. */
void oracle_rms_norm(float* x, const float* y, const float* weight, float* out, int64_t rows, int64_t cols,
                     float eps, float offset, int64_t weight_rows) {
  for (int64_t r = 0; r < rows; ++r) {
    float* row = x + r * cols;
    if (y)
      for (int64_t c = 0; c < cols; ++c) row[c] = (float)((double)row[c] + (double)y[r * cols + c]);
    double squares = 0.0;
    for (int64_t c = 0; c < cols; ++c) squares += (double)row[c] * (double)row[c];
    const double factor = 1 / sqrt(squares / (double)cols + (double)eps);
    const float* w = weight + (r % weight_rows) * cols;
    for (int64_t c = 0; c < cols; ++c)
      out[r * cols + c] = (float)((double)row[c] * factor * ((double)w[c] + (double)offset));
  }
}

/* CpuNormalisation.layerNorm (ops/CpuNormalisation.scala:128-151): mean, then
 * the variance about it (two passes, double), factor 1/sqrt(var + eps);
 * value = normal * (w or 1) + (b or 0). */
void oracle_layer_norm(const float* x, const float* weight, const float* bias, float* out, int64_t rows,
                       int64_t cols, float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = x + r * cols;
    double sum = 0.0;
    for (int64_t c = 0; c < cols; ++c) sum += (double)row[c];
    const double mean = sum / (double)cols;
    double squares = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
      const double d = (double)row[c] - mean;
      squares += d * d;
    }
    const double variance = squares / (double)cols;
    const double factor = 1 / sqrt(variance + (double)eps);
    for (int64_t c = 0; c < cols; ++c) {
      const double normal = ((double)row[c] - mean) * factor;
      const double value = normal * (weight ? (double)weight[c] : 1.0) + (bias ? (double)bias[c] : 0.0);
      out[r * cols + c] = (float)value;
    }
  }
}

/* CpuElementwise.modulate (ops/CpuElementwise.scala:33-38) */
void oracle_modulate(const float* x, const float* scale, const float* shift, float* out, int64_t rows,
                     int64_t cols) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      const int64_t i = r * cols + c;
      out[i] = (float)((double)x[i] * (1 + (double)scale[c]) + (double)shift[c]);
    }
}

/* The section a pair takes its position from (ops/CpuAttention.scala:98-108,
 * ops/Rope.scala:12-35). */
static int rope_section(int pair, int sections, const int32_t* s) {
  switch (sections) {
    case 1:
      return pair < s[0] ? 0 : (pair < s[0] + s[1] ? 1 : 2);
    case 2:
      if (pair % 3 == 1 && pair < 3 * s[1]) return 1;
      if (pair % 3 == 2 && pair < 3 * s[2]) return 2;
      return 0;
    case 3: {
      int end = 0;
      for (int a = 0; a < 4; ++a) {
        end += s[a];
        if (pair < end) return a;
      }
      return -1;
    }
    default:
      return 0;
  }
}

/* ops/CpuAttention.scala:124-133: pow in double, rounded to float, then a
 * float reciprocal. */
float oracle_rope_inverse_frequency(int pair, int rotary, float theta, int sections, const int32_t* s) {
  if (sections == 3) {
    const int axis = rope_section(pair, sections, s);
    int start = 0;
    for (int a = 0; a < axis; ++a) start += s[a];
    const int count = s[axis];
    return 1.0f / (float)pow((double)theta, (double)(pair - start) / (double)count);
  }
  return 1.0f / (float)pow((double)theta, 2.0 * pair / (double)rotary);
}

/* CpuAttention.rope (ops/CpuAttention.scala:92-146): value d of each head turns
 * with its partner (NeoX: d +- rotary/2; interleaved: d ^ 1) by the float angle
 * position * inverse frequency, in double; values from `rotary` on are copied. */
void oracle_rope(const float* x, const int32_t* positions, float* out, int tokens, int heads, int dim, int rotary,
                 float theta, int layout, int sections, const int32_t* s) {
  const int half = rotary / 2;
  for (int t = 0; t < tokens; ++t)
    for (int h = 0; h < heads; ++h) {
      const int64_t base = ((int64_t)t * heads + h) * dim;
      for (int d = 0; d < dim; ++d) {
        double value;
        if (d >= rotary) {
          value = (double)x[base + d];
        } else {
          int pair, first, partner;
          if (layout == 0) {
            pair = d % half;
            first = d < half;
            partner = first ? d + half : d - half;
          } else {
            pair = d / 2;
            first = d % 2 == 0;
            partner = first ? d + 1 : d - 1;
          }
          const float inverse = oracle_rope_inverse_frequency(pair, rotary, theta, sections, s);
          const int32_t p = positions[(int64_t)rope_section(pair, sections, s) * tokens + t];
          const float angle_f = (float)p * inverse;
          const double angle = (double)angle_f;
          const double a = first ? (double)x[base + d] : (double)x[base + partner];
          const double b = first ? (double)x[base + partner] : (double)x[base + d];
          value = first ? a * cos(angle) - b * sin(angle) : a * sin(angle) + b * cos(angle);
        }
        out[base + d] = (float)value;
      }
    }
}

/* CpuAttention.ropeTable (ops/CpuAttention.scala:53-87) */
void oracle_rope_table(const float* x, const float* cosines, const float* sines, float* out, int tokens, int heads,
                       int dim, int pairs, int per_head, int halves) {
  const int64_t count = (int64_t)tokens * heads * dim;
  for (int64_t index = 0; index < count; ++index) {
    const int d = (int)(index % dim);
    const int64_t row = per_head ? index / dim : index / ((int64_t)heads * dim);
    double value;
    if (halves) {
      if (d >= 2 * pairs) {
        value = (double)x[index];
      } else {
        const int m = d % pairs;
        const double c = (double)cosines[row * pairs + m], s = (double)sines[row * pairs + m];
        const double a = (double)x[index - d + m], b = (double)x[index - d + m + pairs];
        value = d < pairs ? a * c - b * s : b * c + a * s;
      }
    } else {
      const int m = d / 2;
      if (m >= pairs) {
        value = (double)x[index];
      } else {
        const double c = (double)cosines[row * pairs + m], s = (double)sines[row * pairs + m];
        const double a = (double)x[index - d % 2], b = (double)x[index - d % 2 + 1];
        value = d % 2 == 0 ? a * c - b * s : a * s + b * c;
      }
    }
    out[index] = (float)value;
  }
}

/* WanConfig.ropePairs (models/Wan.scala:35-41): frame, row and column pairs
 * of a head, d - 4*floor(d/6), 2*floor(d/6), 2*floor(d/6) values, halved. */
void oracle_wan_pairs(int head_dim, int32_t* pairs3) {
  const int side = 2 * (head_dim / 6);
  pairs3[0] = (head_dim - 2 * side) / 2;
  pairs3[1] = side / 2;
  pairs3[2] = side / 2;
}

/* Wan.angles (models/Wan.scala:324-361): per token and pair, the axis
 * position over theta^(2 index / (2 pairs_axis)) in double, then cos and sin
 * rounded to float. */
void oracle_wan_angles(int frames, int rows, int cols, int head_dim, double theta, float* cosines, float* sines) {
  int32_t axes[3];
  oracle_wan_pairs(head_dim, axes);
  const int pairs = head_dim / 2;
  const int64_t tokens = (int64_t)frames * rows * cols;
  for (int64_t i = 0; i < tokens * pairs; ++i) {
    const int64_t token = i / pairs;
    const int pair = (int)(i % pairs);
    int axis, index;
    if (pair < axes[0]) {
      axis = 0;
      index = pair;
    } else if (pair < axes[0] + axes[1]) {
      axis = 1;
      index = pair - axes[0];
    } else {
      axis = 2;
      index = pair - axes[0] - axes[1];
    }
    int64_t position;
    if (axis == 0)
      position = token / ((int64_t)rows * cols);
    else if (axis == 1)
      position = token / cols % rows;
    else
      position = token % cols;
    const double angle = (double)position / pow(theta, 2.0 * index / (double)(2 * axes[axis]));
    cosines[i] = (float)cos(angle);
    sines[i] = (float)sin(angle);
  }
}

/* CpuLinear.embedding (ops/CpuLinear.scala:12-41) over GgmlQuants.Q8_0
 * (tensor/GgmlQuants.scala:104-118): per 34-byte block, d = f16 at byte 0,
 * value j = float(int8 at byte 2 + j) * d in float. */
int64_t oracle_embedding_q8_0(const uint8_t* table, int64_t vocab, int64_t cols, const int32_t* ids, int64_t count,
                              float* out) {
  const int64_t blocks = cols / 32;
  const int64_t row_bytes = blocks * 34;
  for (int64_t t = 0; t < count; ++t) {
    const int64_t row = ids[t];
    if (row < 0 || row >= vocab) return t;
    const uint8_t* source = table + row * row_bytes;
    for (int64_t b = 0; b < blocks; ++b) {
      const uint8_t* block = source + b * 34;
      const float d = oracle_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
      for (int j = 0; j < 32; ++j) out[t * cols + b * 32 + j] = (float)(int8_t)block[2 + j] * d;
    }
  }
  return -1;
}

int64_t oracle_embedding_f32(const float* table, int64_t vocab, int64_t cols, const int32_t* ids, int64_t count,
                             float* out) {
  for (int64_t t = 0; t < count; ++t) {
    const int64_t row = ids[t];
    if (row < 0 || row >= vocab) return t;
    memcpy(out + t * cols, table + row * cols, (size_t)cols * 4);
  }
  return -1;
}

/* ---- storage types: tensor/GgmlQuants.scala, tensor/KQuants.scala,
 * tensor/IQuants.scala, tensor/RocmFp4.scala, tensor/DType.scala. Each
 * decoder restates the Scala's decodeBlock (or its per-element formula),
 * operation by operation in float, as the JVM evaluates it (no contraction:
 * the Makefile's -ffp-contract=off). ---- */

static uint32_t u8_at(const uint8_t* p, int64_t at) { return p[at]; }
static int32_t i8_at(const uint8_t* p, int64_t at) { return (int8_t)p[at]; }
static uint32_t u16_at(const uint8_t* p, int64_t at) { return (uint32_t)p[at] | ((uint32_t)p[at + 1] << 8); }
static uint32_t u32_at(const uint8_t* p, int64_t at) { return u16_at(p, at) | (u16_at(p, at + 2) << 16); }
static float f16_at(const uint8_t* p, int64_t at) { return oracle_f16_to_f32((uint16_t)u16_at(p, at)); }

/* GgmlQuants.fiveBit (GgmlQuants.scala:53-64) */
static int five_bit(const uint8_t* b, int64_t qh_at, int64_t qs_at, int j) {
  const uint32_t qh = u32_at(b, qh_at);
  const uint32_t nibbles = u8_at(b, qs_at + (j % 16));
  const uint32_t low = j < 16 ? (nibbles & 0xf) : (nibbles >> 4);
  return (int)(low | (((qh >> j) & 1u) << 4));
}

/* KQuants.twoBits, nibble, scaleAndMin (KQuants.scala:38-70) */
static int two_bits(const uint8_t* b, int64_t at, int e) {
  const int half = e / 128, plane = (e % 128) / 32;
  return (int)((u8_at(b, at + half * 32 + e % 32) >> (2 * plane)) & 3u);
}

static int nibble_k(const uint8_t* b, int64_t at, int e) {
  const int chunk = e / 32;
  return (int)((u8_at(b, at + (chunk / 2) * 32 + e % 32) >> (4 * (chunk % 2))) & 0xfu);
}

static void scale_and_min(const uint8_t* b, int64_t at, int j, int* scale, int* min) {
#define BYTE(i) ((int)u8_at(b, at + (i)))
  if (j < 4) {
    *scale = BYTE(j) & 63;
    *min = BYTE(j + 4) & 63;
  } else {
    *scale = (BYTE(j + 4) & 0xf) | ((BYTE(j - 4) >> 2) & 0x30);
    *min = (BYTE(j + 4) >> 4) | ((BYTE(j) >> 2) & 0x30);
  }
#undef BYTE
}

/* IQuants.Values (IQuants.scala:14-16) */
static const float kIq4Values[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* RocmFp4.Codebook and halfScale (RocmFp4.scala:21-39) */
static const float kRocmCodebook[16] = {0, 1, 2, 3, 4, 6, 8, 10, 0, -1, -2, -3, -4, -6, -8, -10};

float oracle_rocmfp4_half_scale(int byte) {
  if (byte > 0x7e) return 0.0f;
  const int exponent = byte >> 3, mantissa = byte & 7;
  if (exponent == 0) return ldexpf((float)mantissa, -10);
  return (float)(8 + mantissa) * ldexpf(1.0f, exponent - 11);
}

int oracle_format_block(int format, int* block_values, int* block_bytes) {
  int v = 32, n;
  switch (format) {
    case ORACLE_F32: v = 1; n = 4; break;
    case ORACLE_F16: case ORACLE_BF16: v = 1; n = 2; break;
    case ORACLE_Q4_0: n = 18; break;
    case ORACLE_Q4_1: n = 20; break;
    case ORACLE_Q5_0: n = 22; break;
    case ORACLE_Q5_1: n = 24; break;
    case ORACLE_Q8_0: n = 34; break;
    case ORACLE_Q4_K: v = 256; n = 144; break;
    case ORACLE_Q5_K: v = 256; n = 176; break;
    case ORACLE_Q6_K: v = 256; n = 210; break;
    case ORACLE_IQ4_NL: n = 18; break;
    case ORACLE_IQ4_XS: v = 256; n = 136; break;
    case ORACLE_ROCMFP4: n = 18; break;
    case ORACLE_ROCMFP4_FAST: n = 17; break;
    default: return -1;
  }
  *block_values = v;
  *block_bytes = n;
  return 0;
}

/* One block of `format` at b into out (block_values values). */
static void decode_block(int format, const uint8_t* b, float* out) {
  switch (format) {
    case ORACLE_F32: { uint32_t w = u32_at(b, 0); memcpy(out, &w, 4); return; }
    case ORACLE_F16: out[0] = f16_at(b, 0); return;
    case ORACLE_BF16: out[0] = oracle_from_bf16((uint16_t)u16_at(b, 0)); return;
    case ORACLE_Q4_0: { /* GgmlQuants.scala:13-29: d * (q - 8) */
      const float d = f16_at(b, 0);
      for (int j = 0; j < 16; ++j) {
        const uint32_t byte = u8_at(b, 2 + j);
        out[j] = d * (float)((int)(byte & 0xf) - 8);
        out[j + 16] = d * (float)((int)(byte >> 4) - 8);
      }
      return;
    }
    case ORACLE_Q4_1: { /* :31-49: d * q + m */
      const float d = f16_at(b, 0), m = f16_at(b, 2);
      for (int j = 0; j < 16; ++j) {
        const uint32_t byte = u8_at(b, 4 + j);
        out[j] = d * (float)(byte & 0xf) + m;
        out[j + 16] = d * (float)(byte >> 4) + m;
      }
      return;
    }
    case ORACLE_Q5_0: { /* :66-81: d * (q - 16) */
      const float d = f16_at(b, 0);
      for (int j = 0; j < 32; ++j) out[j] = d * (float)(five_bit(b, 2, 6, j) - 16);
      return;
    }
    case ORACLE_Q5_1: { /* :83-99: d * q + m */
      const float d = f16_at(b, 0), m = f16_at(b, 2);
      for (int j = 0; j < 32; ++j) out[j] = d * (float)five_bit(b, 4, 8, j) + m;
      return;
    }
    case ORACLE_Q8_0: { /* :101-117: q * d */
      const float d = f16_at(b, 0);
      for (int j = 0; j < 32; ++j) out[j] = (float)i8_at(b, 2 + j) * d;
      return;
    }
    case ORACLE_Q4_K: /* KQuants.scala:102-110: d * sc * q - dmin * m, per 32 */
      for (int e = 0; e < 256; ++e) {
        int scale, min;
        scale_and_min(b, 4, e / 32, &scale, &min);
        const float d = f16_at(b, 0) * (float)scale;
        const float m = f16_at(b, 2) * (float)min;
        out[e] = d * (float)nibble_k(b, 16, e) - m;
      }
      return;
    case ORACLE_Q5_K: /* :112-121 */
      for (int e = 0; e < 256; ++e) {
        int scale, min;
        scale_and_min(b, 4, e / 32, &scale, &min);
        const float d = f16_at(b, 0) * (float)scale;
        const float m = f16_at(b, 2) * (float)min;
        const int high = (int)((u8_at(b, 16 + e % 32) >> (e / 32)) & 1u);
        out[e] = d * (float)(nibble_k(b, 48, e) | (high << 4)) - m;
      }
      return;
    case ORACLE_Q6_K: /* :123-134: d * sc * (q - 32) */
      for (int e = 0; e < 256; ++e) {
        const int half = e / 128, r = e % 128;
        const int low = (int)((u8_at(b, half * 64 + r % 64) >> (4 * (r / 64))) & 0xfu);
        const int q = (low | (two_bits(b, 128, e) << 4)) - 32;
        const float d = f16_at(b, 208) * (float)i8_at(b, 192 + e / 16);
        out[e] = d * (float)q;
      }
      return;
    case ORACLE_IQ4_NL: { /* IQuants.scala:18-47 */
      const float d = f16_at(b, 0);
      for (int j = 0; j < 16; ++j) {
        const uint32_t byte = u8_at(b, 2 + j);
        out[j] = d * kIq4Values[byte & 0xf];
        out[j + 16] = d * kIq4Values[byte >> 4];
      }
      return;
    }
    case ORACLE_IQ4_XS: { /* :49-80 */
      const float d = f16_at(b, 0);
      const uint32_t high = u16_at(b, 2);
      for (int i = 0; i < 8; ++i) {
        const uint32_t low = (u8_at(b, 4 + i / 2) >> (4 * (i % 2))) & 0xf;
        const int ls = (int)(low | (((high >> (2 * i)) & 3u) << 4));
        const float scale = d * (float)(ls - 32);
        for (int j = 0; j < 16; ++j) {
          const uint32_t byte = u8_at(b, 8 + 16 * i + j);
          out[32 * i + j] = scale * kIq4Values[byte & 0xf];
          out[32 * i + j + 16] = scale * kIq4Values[byte >> 4];
        }
      }
      return;
    }
    default: { /* ROCmFP4, RocmFp4.scala:45-62: scales at 16 and 17 (dual) or 16 (fast) */
      const float low = oracle_rocmfp4_half_scale((int)u8_at(b, 16));
      const float high = oracle_rocmfp4_half_scale((int)u8_at(b, format == ORACLE_ROCMFP4 ? 17 : 16));
      for (int j = 0; j < 16; ++j) {
        const uint32_t byte = u8_at(b, j);
        out[j] = kRocmCodebook[byte & 0xf] * low;
        out[j + 16] = kRocmCodebook[byte >> 4] * high;
      }
      return;
    }
  }
}

int oracle_decode_row(int format, const uint8_t* row, int64_t cols, float* out) {
  int values, bytes;
  if (oracle_format_block(format, &values, &bytes) != 0 || cols % values != 0) return -1;
  for (int64_t b = 0; b < cols / values; ++b) decode_block(format, row + b * bytes, out + b * values);
  return 0;
}

/* ops/CpuLinear.scala:12-41 with any storage type: decoded rows as F32. */
int64_t oracle_embedding(int format, const uint8_t* table, int64_t vocab, int64_t cols, const int32_t* ids,
                         int64_t count, float* out) {
  int values, bytes;
  if (oracle_format_block(format, &values, &bytes) != 0 || cols % values != 0) return -2;
  const int64_t row_bytes = cols / values * bytes;
  for (int64_t t = 0; t < count; ++t) {
    const int64_t row = ids[t];
    if (row < 0 || row >= vocab) return t;
    oracle_decode_row(format, table + row * row_bytes, cols, out + t * cols);
  }
  return -1;
}

/* kernels/quantize.h:10-25: a wave of 32 lanes holds a block, lane l its
 * value l; amax is the fmaxf of |x| over the lanes, d = amax / 127.0f, the
 * code int(roundf(x / d)) (0 for d == 0), its int8 kept; lane 0 writes d and
 * d * float(sum of codes). fmaxf skips a NaN operand, so the order of the
 * lanes' butterfly does not change amax. A NaN quotient (a NaN x, or an
 * infinite d) gives code 0, as the GPU's float-to-int conversion does. */
void oracle_quantize_x(const float* x, int8_t* xq, float* xd, float* xs, int64_t blocks) {
  for (int64_t b = 0; b < blocks; ++b) {
    const float* v = x + b * 32;
    float amax = fabsf(v[0]);
    for (int i = 1; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    const float d = amax / 127.0f;
    int sum = 0;
    for (int i = 0; i < 32; ++i) {
      const float r = roundf(v[i] / d);
      const int code = (d == 0.0f || r != r) ? 0 : (int)r;
      xq[b * 32 + i] = (int8_t)code;
      sum += code;
    }
    xd[b] = d;
    xs[b] = d * (float)sum;
  }
}

/* ops/CpuElementwise.scala:40-49 gatedAdd: before(i) + gates(i % cols) *
 * added(i), in double (the reader widens every float), written as float. A
 * batch of samples takes sample r / rows_per_sample's gate row. */
void oracle_gated_add(float* x, const float* y, const float* gate, int64_t rows, int64_t cols,
                      int64_t rows_per_sample) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* g = gate + (r / rows_per_sample) * cols;
    for (int64_t c = 0; c < cols; ++c) {
      const int64_t i = r * cols + c;
      x[i] = (float)((double)x[i] + (double)g[c] * (double)y[i]);
    }
  }
}

/* ops/CpuElementwise.scala:51-67 modulateChunks: input(index) * (1 +
 * values(row + scale * channels + c)) + values(row + shift * channels + c),
 * row = r * chunks * channels, in double. */
void oracle_modulate_chunks(const float* x, const float* table, float* out, int64_t rows, int64_t channels,
                            int64_t chunks, int64_t shift, int64_t scale) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = table + r * chunks * channels;
    for (int64_t c = 0; c < channels; ++c) {
      const int64_t i = r * channels + c;
      out[i] = (float)((double)x[i] * (1.0 + (double)row[scale * channels + c]) + (double)row[shift * channels + c]);
    }
  }
}

/* ops/CpuElementwise.scala:69-79 gatedAddChunk: input(index) +
 * values(r * chunks * channels + gate * channels + c) * other(index). */
void oracle_gated_add_chunk(float* x, const float* y, const float* table, int64_t rows, int64_t channels,
                            int64_t chunks, int64_t gate) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* g = table + r * chunks * channels + gate * channels;
    for (int64_t c = 0; c < channels; ++c) {
      const int64_t i = r * channels + c;
      x[i] = (float)((double)x[i] + (double)g[c] * (double)y[i]);
    }
  }
}

/* ops/CpuElementwise.scala:81-85 rowGatedAdd: input(index) + gates(index /
 * cols) * other(index). */
void oracle_row_gated_add(float* x, const float* y, const float* gate, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      const int64_t i = r * cols + c;
      x[i] = (float)((double)x[i] + (double)gate[r] * (double)y[i]);
    }
}

/* ---- ConvRot's rotated linears ---- */

/* tensor/DType.scala:105-115 F8E4M3 ("fn"): bias 7, no infinities, NaN at
 * S.1111.111; Math.scalb is exact. */
float oracle_f8e4m3(int code) {
  const int exponent = (code >> 3) & 0xf, mantissa = code & 7;
  float magnitude;
  if (exponent == 0xf && mantissa == 7)
    magnitude = NAN;
  else if (exponent == 0)
    magnitude = ldexpf((float)mantissa, -9);
  else
    magnitude = (float)(8 + mantissa) * ldexpf(1.0f, exponent - 10);
  return (code & 0x80) ? -magnitude : magnitude;
}

/* tensor/ConvRot.scala:20-50 rotate: each `group` values from `from` times
 * the normalized regular Hadamard matrix, as rounds of four-point
 * butterflies over strides 1, 4, 16, ... below `group`, in float: half =
 * (a + b + c + d) * 0.5 summed left to right, then half - d, half - c,
 * half - b, half - a. */
void oracle_convrot_rotate(float* values, int64_t length, int64_t group) {
  for (int64_t start = 0; start < length; start += group)
    for (int64_t stride = 1; stride < group; stride *= 4)
      for (int64_t block = start; block < start + group; block += 4 * stride)
        for (int64_t i = block; i < block + stride; ++i) {
          const float a = values[i], b = values[i + stride], c = values[i + 2 * stride], d = values[i + 3 * stride];
          const float half = (a + b + c + d) * 0.5f;
          values[i] = half - d;
          values[i + stride] = half - c;
          values[i + 2 * stride] = half - b;
          values[i + 3 * stride] = half - a;
        }
}

/* ops/CpuBase.scala:40-81 rotatedRows before its rotation: rows [first,
 * first + count) of a rotated linear [rows, cols] as the int8 levels times
 * their row's scale. int8_tensorwise (codebook NULL): codes int8 [rows,
 * cols], scales one a row or one for all. asym_w4a8_int8: codes two 4-bit
 * a byte [rows, cols / 2] (the even column the low nibble); the level is
 * max(-127, min(127, rint(codebook[code] * relative))) in double with
 * Java's NaN-keeping min and max, relative the row's fp8 scale of the
 * column's group of group_size. */
void oracle_convrot_levels(const uint8_t* codes, const float* scales, int64_t scale_count, const float* codebook,
                           const uint8_t* relative, int64_t group_size, int64_t cols, int64_t first, int64_t count,
                           float* out) {
  for (int64_t r = 0; r < count; ++r) {
    const int64_t row = first + r;
    const float scale = scales[scale_count == 1 ? 0 : row];
    for (int64_t c = 0; c < cols; ++c) {
      float level;
      if (!codebook) {
        level = (float)(int8_t)codes[row * cols + c];
      } else {
        const uint8_t byte = codes[row * (cols / 2) + c / 2];
        const int code = (c % 2 == 0) ? (byte & 0xf) : ((byte >> 4) & 0xf);
        const float rel = oracle_f8e4m3(relative[row * (cols / group_size) + c / group_size]);
        const double rounded = rint((double)(codebook[code] * rel));
        const double low = rounded != rounded ? rounded : (127.0 < rounded ? 127.0 : rounded);
        level = (float)(low != low ? low : (-127.0 > low ? -127.0 : low));
      }
      out[r * cols + c] = level * scale;
    }
  }
}

/* ops/CpuBase.scala:40-81 rotatedRows: the levels above, every 256 columns
 * rotated (ConvRot.Group). */
void oracle_convrot_rows(const uint8_t* codes, const float* scales, int64_t scale_count, const float* codebook,
                         const uint8_t* relative, int64_t group_size, int64_t cols, int64_t first, int64_t count,
                         float* out) {
  oracle_convrot_levels(codes, scales, scale_count, codebook, relative, group_size, cols, first, count, out);
  oracle_convrot_rotate(out, count * cols, 256);
}

/* ops/CpuLinear.scala:12-41 for a rotated table: row ids[t] of the weight
 * [rows, cols] as the BF16 it holds, widened to F32. Returns the first id
 * outside [0, rows), -1 if none. */
int64_t oracle_convrot_embedding(const uint8_t* codes, const float* scales, int64_t scale_count,
                                 const float* codebook, const uint8_t* relative, int64_t group_size, int64_t rows,
                                 int64_t cols, const int32_t* ids, int64_t count, float* out) {
  for (int64_t t = 0; t < count; ++t) {
    const int64_t row = ids[t];
    if (row < 0 || row >= rows) return t;
    float* target = out + t * cols;
    oracle_convrot_rows(codes, scales, scale_count, codebook, relative, group_size, cols, row, 1, target);
    for (int64_t c = 0; c < cols; ++c) target[c] = oracle_from_bf16(oracle_to_bf16(target[c]));
  }
  return -1;
}
