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

// Float to BF16 bits as CpuOps.toBfloat16 rounds (ops/CpuOps.scala:426-431):
// nearest even on the bit pattern; a NaN keeps its top half, quiet bit set.
__device__ __forceinline__ uint32_t bf16_bits(float v) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t rounded = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
  return (v != v) ? ((b >> 16) | 0x40u) : rounded;
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) { return bf16_bits(lo) | (bf16_bits(hi) << 16); }

// ---------------------------------------------------------------- element types

// A 16-byte chunk of a row: 4 floats or 8 bf16, unpacked to float.
template <typename T>
struct Chunk;

template <>
struct Chunk<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void load(const float* p, float (&v)[4]) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  }
  __device__ __forceinline__ static void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

template <>
struct Chunk<uint16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void load(const uint16_t* p, float (&v)[8]) {
    const uint4 q = *reinterpret_cast<const uint4*>(p);
    v[0] = bf16_lo(q.x);
    v[1] = bf16_hi(q.x);
    v[2] = bf16_lo(q.y);
    v[3] = bf16_hi(q.y);
    v[4] = bf16_lo(q.z);
    v[5] = bf16_hi(q.z);
    v[6] = bf16_lo(q.w);
    v[7] = bf16_hi(q.w);
  }
  __device__ __forceinline__ static void store(uint16_t* p, const float (&v)[8]) {
    *reinterpret_cast<uint4*>(p) =
        make_uint4(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7]));
  }
};

// Scalar element access for the awkward-shape paths.
__device__ __forceinline__ float load_one(const float* p) { return *p; }
__device__ __forceinline__ float load_one(const uint16_t* p) { return __uint_as_float((uint32_t)*p << 16); }
__device__ __forceinline__ void store_one(float* p, float v) { *p = v; }
__device__ __forceinline__ void store_one(uint16_t* p, float v) { *p = (uint16_t)bf16_bits(v); }

// ---------------------------------------------------------------- reductions

// Sum over aligned groups of `width` lanes (a power of two up to 64); every
// lane of a group gets the group's total. The butterfly order is fixed, so a
// row's sum does not depend on how many rows share the launch.
template <int width>
__device__ __forceinline__ double group_sum(double v) {
#pragma unroll
  for (int mask = 1; mask < width; mask <<= 1) v += __shfl_xor(v, mask, width);
  return v;
}

// ---------------------------------------------------------------- host side

// Records why an entry point refused its arguments (thread-local), returns
// hipErrorInvalidValue.
int refuse(const char* format, ...);
// The result of a launch: the runtime's error, if any, recorded too.
int launched(const char* entry);
void clear_error();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workgroups for a grid-stride launch: enough to fill the chip many times
// over, never more than the grid allows.
inline unsigned grid_for(int64_t items, int per_block, int64_t cap = 1 << 20) {
  int64_t blocks = ceil_div(items, per_block);
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (unsigned)blocks;
}

}  // namespace drift
