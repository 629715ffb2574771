// Shared pieces of the fused layer kernels for gfx950 (CDNA4): wave64
// reductions, bf16 rounding with the runner's rules, 16-byte chunk I/O, and
// the host-side validation every entry point runs before it launches.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>

#include "../../include/drift_kernels.h"

namespace drift {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16

// BF16 bits to float: the top half of an F32 (tensor/DType.scala:99-102).
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

// Float to BF16 bits as CpuOps.toBfloat16 rounds (ops/CpuOps.scala:52-57):
// nearest even on the bit pattern; a NaN keeps its top half, quiet bit set.
// gfx950's v_cvt_pk_bf16_f32 does exactly this, two values per instruction
// (checked on the device over every class of pattern, NaN payloads and ties
// included: tests/test_gpu_elementwise.py::test_convert_round_trips).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint32_t bf16_bits(float v) { return pack_bf16(v, 0.0f) & 0xffffu; }

// ---------------------------------------------------------------- element types

// Inputs are read once and outputs written once: chunk loads and stores are
// non-temporal (they stream through the caches rather than fill them), which
// measures faster on every kernel here. A streaming copy on MI355X moves
// about 6.0 TB/s with plain loads and 6.4 TB/s with non-temporal ones.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 stream_load(const void* p) {
  const u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(q.x, q.y, q.z, q.w);
}

// A 16-byte chunk of a row: 4 floats or 8 bf16, unpacked to float.
template <typename T>
struct Chunk;

// Raw: the chunk as loaded (16 bytes in four VGPRs); unpack: its values as
// float. opaque() hides a raw chunk's value from the compiler, so a second
// pass re-unpacks it instead of keeping every converted value alive.
template <>
struct Chunk<float> {
  static constexpr int N = 4;
  using Raw = uint4;
  __device__ __forceinline__ static Raw load_raw(const float* p) { return stream_load(p); }
  __device__ __forceinline__ static void unpack(const Raw& q, float (&v)[4]) {
    v[0] = __uint_as_float(q.x);
    v[1] = __uint_as_float(q.y);
    v[2] = __uint_as_float(q.z);
    v[3] = __uint_as_float(q.w);
  }
  __device__ __forceinline__ static void load(const float* p, float (&v)[4]) { unpack(stream_load(p), v); }
  __device__ __forceinline__ static void store(float* p, const float (&v)[4]) {
    const u32x4 q = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
    __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(p));
  }
};

template <>
struct Chunk<uint16_t> {
  static constexpr int N = 8;
  using Raw = uint4;
  __device__ __forceinline__ static Raw load_raw(const uint16_t* p) { return stream_load(p); }
  __device__ __forceinline__ static void unpack(const Raw& q, float (&v)[8]) {
    v[0] = bf16_lo(q.x);
    v[1] = bf16_hi(q.x);
    v[2] = bf16_lo(q.y);
    v[3] = bf16_hi(q.y);
    v[4] = bf16_lo(q.z);
    v[5] = bf16_hi(q.z);
    v[6] = bf16_lo(q.w);
    v[7] = bf16_hi(q.w);
  }
  __device__ __forceinline__ static void load(const uint16_t* p, float (&v)[8]) { unpack(stream_load(p), v); }
  __device__ __forceinline__ static void store(uint16_t* p, const float (&v)[8]) {
    const u32x4 q = {pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7])};
    __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(p));
  }
};

__device__ __forceinline__ void opaque(uint4& q) { asm volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w)); }

// Scalar element access for the awkward-shape paths.
__device__ __forceinline__ float load_one(const float* p) { return *p; }
__device__ __forceinline__ float load_one(const uint16_t* p) { return __uint_as_float((uint32_t)*p << 16); }
__device__ __forceinline__ void store_one(float* p, float v) { *p = v; }
__device__ __forceinline__ void store_one(uint16_t* p, float v) { *p = (uint16_t)bf16_bits(v); }

// ---------------------------------------------------------------- reductions

// A double moved across lanes by a DPP pattern (both halves), within rows of
// 16 lanes.
template <int kCtrl>
__device__ __forceinline__ double dpp_move(double v) {
  const uint64_t bits = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)bits, kCtrl, 0xf, 0xf, true);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(bits >> 32), kCtrl, 0xf, 0xf, true);
  return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// floor(i / d) for 0 <= i < 2^50 from a multiply by 1/d: the product is
// within one of the quotient, and one step each way corrects it.
__device__ __forceinline__ int64_t quotient(int64_t i, int64_t d, double inverse) {
  int64_t q = (int64_t)((double)i * inverse);
  q -= (q * d > i);
  q += ((q + 1) * d <= i);
  return q;
}

// 1 / sqrt(m) by the hardware's reciprocal square root and two Newton steps
// (within a double ulp or two of the correctly rounded quotient of the
// correctly rounded root, which moves an F32 result only where it lies that
// close to a rounding boundary). Without a branch: a subnormal m is scaled
// into range first (2^256 m, the result times 2^128), and 0 and infinity give
// the division's own infinity and zero; NaN stays NaN. With NORMAL the caller
// knows m is at least 2^-1000 or not a number (a positive epsilon is added to
// it), and the scaling and the zero case are left out.
template <bool NORMAL = false>
__device__ __forceinline__ double inverse_sqrt(double m) {
  const bool tiny = !NORMAL && m < 0x1p-1000;
  const double ms = tiny ? m * 0x1p256 : m;
  double y = __builtin_amdgcn_rsq(ms);
  y = y * fma(-0.5 * ms * y, y, 1.5);
  y = y * fma(-0.5 * ms * y, y, 1.5);
  if constexpr (!NORMAL) {
    y = tiny ? y * 0x1p128 : y;
    y = m == 0.0 ? __builtin_huge_val() : y;
  }
  return m == __builtin_huge_val() ? 0.0 : y;
}

// Sum over aligned groups of `width` lanes (a power of two up to 64); every
// lane of a group gets the group's total. It is the xor butterfly (partners
// i ^ 1, i ^ 2, ...), its steps inside 16-lane rows taken by DPP moves: after
// the first two, the lanes of a quad hold one value, so the half-row and row
// mirrors (i <-> 7 - i, i <-> 15 - i) add the same partners as i ^ 4 and
// i ^ 8. The order is fixed, so a row's sum does not depend on how many rows
// share the launch.
template <int width>
__device__ __forceinline__ double group_sum(double v) {
  if constexpr (width > 1) v += dpp_move<0xb1>(v);   // quad_perm [1, 0, 3, 2]
  if constexpr (width > 2) v += dpp_move<0x4e>(v);   // quad_perm [2, 3, 0, 1]
  if constexpr (width > 4) v += dpp_move<0x141>(v);  // row_half_mirror
  if constexpr (width > 8) v += dpp_move<0x140>(v);  // row_mirror
#pragma unroll
  for (int mask = 16; mask < width; mask <<= 1) v += __shfl_xor(v, mask, width);
  return v;
}

// The same butterfly for a 32-bit value and an exact, order-free combine
// (max of floats, sum of integers): every lane of an aligned group of `width`
// lanes gets the group's result.
template <int kCtrl>
__device__ __forceinline__ int dpp_move32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xf, 0xf, true);
}

template <int width>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (width > 1) v = fmaxf(v, __int_as_float(dpp_move32<0xb1>(__float_as_int(v))));
  if constexpr (width > 2) v = fmaxf(v, __int_as_float(dpp_move32<0x4e>(__float_as_int(v))));
  if constexpr (width > 4) v = fmaxf(v, __int_as_float(dpp_move32<0x141>(__float_as_int(v))));
  if constexpr (width > 8) v = fmaxf(v, __int_as_float(dpp_move32<0x140>(__float_as_int(v))));
#pragma unroll
  for (int mask = 16; mask < width; mask <<= 1) v = fmaxf(v, __shfl_xor(v, mask, width));
  return v;
}

template <int width>
__device__ __forceinline__ int group_sum_int(int v) {
  if constexpr (width > 1) v += dpp_move32<0xb1>(v);
  if constexpr (width > 2) v += dpp_move32<0x4e>(v);
  if constexpr (width > 4) v += dpp_move32<0x141>(v);
  if constexpr (width > 8) v += dpp_move32<0x140>(v);
#pragma unroll
  for (int mask = 16; mask < width; mask <<= 1) v += __shfl_xor(v, mask, width);
  return v;
}

// Orders a wave's LDS writes before its lanes' reads of them, and back (the
// lanes of one wave exchanging through LDS need no block barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------- int8 side output

// Where a kernel also writes its output quantized for the runner's int8
// products (kernels/quantize.h:6-25): per block of 32 consecutive values of
// the flat output, int8 codes xq[32 b + i], the scale xd[b] = max|v| / 127 and
// xs[b] = xd[b] * sum of the codes. A null xq means no side output.
struct Quantized {
  int8_t* xq;
  float* xd;
  float* xs;
};

// A chunk's values as its store writes them: bf16 outputs rounded first, so
// the codes describe what the output tensor holds.
template <typename T, int N>
__device__ __forceinline__ void as_written(float (&v)[N]) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int j = 0; j < N; j += 2) {
      const uint32_t pair = pack_bf16(v[j], v[j + 1]);
      v[j] = bf16_lo(pair);
      v[j + 1] = bf16_hi(pair);
    }
  }
}

// Quantizes a lane's N consecutive values, which with the other 32 / N - 1
// lanes of its aligned lane group make up block `block`; every lane of the
// group calls. The code is round-half-away(v / d) with d = max|v| / 127, both
// divisions correctly rounded, and 0 where d is 0 or the quotient is NaN.
template <int N>
__device__ __forceinline__ void quantize_chunk(const float (&v)[N], int64_t block, Quantized q) {
  constexpr int G = 32 / N;
  float amax = fabsf(v[0]);
#pragma unroll
  for (int j = 1; j < N; ++j) amax = fmaxf(amax, fabsf(v[j]));
  amax = group_max<G>(amax);
  const float d = amax / 127.0f;
  int sum = 0;
  uint32_t bytes[(N + 3) / 4] = {};
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const float r = roundf(v[j] / d);
    const int code = (d == 0.0f || r != r) ? 0 : (int)r;
    sum += code;
    bytes[j / 4] |= ((uint32_t)code & 0xffu) << (8 * (j % 4));
  }
  const int member = threadIdx.x % G;
  int8_t* at = q.xq + block * 32 + member * N;
  if constexpr (N == 1)
    *at = (int8_t)bytes[0];
  else if constexpr (N == 4)
    *reinterpret_cast<uint32_t*>(at) = bytes[0];
  else
    *reinterpret_cast<uint2*>(at) = make_uint2(bytes[0], bytes[1]);
  sum = group_sum_int<G>(sum);
  if (member == 0) {
    q.xd[block] = d;
    q.xs[block] = d * (float)sum;
  }
}

// ---------------------------------------------------------------- host side

// quantize_x over `blocks` blocks of 32 values of x (quantize.hip): the side
// output of a write that could not quantize as it wrote.
int launch_quantize(const float* x, Quantized q, int64_t blocks, hipStream_t stream);
int launch_quantize(const uint16_t* x, Quantized q, int64_t blocks, hipStream_t stream);
// Whether a chunked kernel with N values per lane can store its codes (N
// bytes per lane, 4- or 8-byte aligned stores).
inline bool codes_storable(const int8_t* xq, int n) {
  return (reinterpret_cast<uintptr_t>(xq) & (uintptr_t)(n >= 8 ? 7 : n >= 4 ? 3 : 0)) == 0;
}
// Checks a side output's pointers and block count; nonzero (refused) if bad.
int check_quantized(const char* entry, Quantized q, int64_t values);

// Records why an entry point refused its arguments (thread-local), returns
// hipErrorInvalidValue.
int refuse(const char* format, ...);
// The result of a launch: the runtime's error, if any, recorded too.
int launched(const char* entry);
void clear_error();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// One-shot grids (a thread or wave per item, no loop) stream faster on MI355X
// than persistent grid-stride ones: dispatch order keeps the addresses in
// flight together, and finished waves are replaced at once. Kernels keep a
// grid-stride loop that runs once below this many blocks.
constexpr int64_t kOneShotBlocks = (int64_t)1 << 30;

// Workgroups for a grid-stride launch: enough to fill the chip many times
// over, never more than the grid allows.
inline unsigned grid_for(int64_t items, int per_block, int64_t cap = 1 << 20) {
  int64_t blocks = ceil_div(items, per_block);
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (unsigned)blocks;
}

}  // namespace drift
