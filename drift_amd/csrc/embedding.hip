// Quantized token-embedding gather for gfx950: rows of a Q8_0 table decoded
// to F32 or BF16.
//
// Q8_0 (tensor/GgmlQuants.scala:104-118): every 32 values are a 34-byte
// block, an fp16 scale d then 32 int8 codes; value j = float(code j) * d,
// which is exact in float (11-bit by 8-bit significands), so the BF16 output
// is bit-exact against the reference's F32 gather rounded to BF16.
//
// One wave per id. A row is walked in segments of 128 blocks (4352 bytes,
// 4096 values): the wave stages the segment in its slice of LDS with 16-byte
// loads (34-byte blocks are only 2-byte aligned), then each lane decodes
// 8 consecutive values per step from LDS and stores them as one 16-byte
// (BF16) or two 16-byte (F32) writes; a store instruction of the wave covers
// a contiguous 1 or 2 KiB of the output row.
#include "common.hpp"

namespace drift {
namespace {

constexpr int kSegmentBlocks = 128;
constexpr int kSegmentBytes = kSegmentBlocks * 34;  // 4352, a multiple of 16

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// float(code) * d as the reference computes it on x86: exact for finite d; an
// infinite d times code 0 is the x86 default NaN; a NaN d comes back as the
// float NaN Float.float16ToFloat makes of it (its significand shifted up),
// quieted by the multiply. nan_bits is that quiet NaN.
__device__ __forceinline__ float decode(int code, float d, bool special, uint32_t nan_bits) {
  const float v = (float)code * d;
  if (!special) return v;
  if (d != d) return __uint_as_float(nan_bits);
  return code == 0 ? __uint_as_float(0xffc00000u) : v;
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]);

template <>
__device__ __forceinline__ void store8<uint16_t>(uint16_t* p, const float (&v)[8]) {
  Chunk<uint16_t>::store(p, v);
}

template <>
__device__ __forceinline__ void store8<float>(float* p, const float (&v)[8]) {
  Chunk<float>::store(p, *reinterpret_cast<const float(*)[4]>(v));
  Chunk<float>::store(p + 4, *reinterpret_cast<const float(*)[4]>(v + 4));
}

// Work items are (id, segment of up to 128 blocks). A wave stages an item's
// bytes with loads issued back to back (indices clamped, not branched, so no
// load waits on the one before), writes them to its LDS slice, starts the
// loads of its next item, then decodes and stores this one.
template <bool ALIGNED>
struct Stage;

template <>
struct Stage<true> {  // 16-byte loads: a segment is at most 272 of them
  static constexpr int kLoads = (kSegmentBytes / 16 + kWave - 1) / kWave;
  uint4 q[kLoads];
  __device__ __forceinline__ void load(const uint8_t* source, int bytes, int lane) {
    const int n = bytes / 16;
#pragma unroll
    for (int k = 0; k < kLoads; ++k) q[k] = reinterpret_cast<const uint4*>(source)[min(k * kWave + lane, n - 1)];
  }
  __device__ __forceinline__ void store(uint4* slice, const uint8_t* source, int bytes, int lane) const {
    const int n = bytes / 16;
#pragma unroll
    for (int k = 0; k < kLoads; ++k)
      if (k * kWave + lane < n) slice[k * kWave + lane] = q[k];
    // a partial segment's last bytes (fewer than 16, an even count)
    const int tail = (bytes - n * 16) / 2;
    if (lane < tail)
      reinterpret_cast<uint16_t*>(slice)[n * 8 + lane] = reinterpret_cast<const uint16_t*>(source)[n * 8 + lane];
  }
};

template <>
struct Stage<false> {  // 2-byte loads for rows that are not 16-byte aligned
  static constexpr int kLoads = (kSegmentBytes / 2 + kWave - 1) / kWave;
  uint16_t h[kLoads];
  __device__ __forceinline__ void load(const uint8_t* source, int bytes, int lane) {
    const int n = bytes / 2;
#pragma unroll
    for (int k = 0; k < kLoads; ++k) h[k] = reinterpret_cast<const uint16_t*>(source)[min(k * kWave + lane, n - 1)];
  }
  __device__ __forceinline__ void store(uint4* slice, const uint8_t*, int bytes, int lane) const {
    const int n = bytes / 2;
#pragma unroll
    for (int k = 0; k < kLoads; ++k)
      if (k * kWave + lane < n) reinterpret_cast<uint16_t*>(slice)[k * kWave + lane] = h[k];
  }
};

template <typename T, bool ALIGNED>
__global__ void __launch_bounds__(256) q8_0_gather(const uint8_t* table, const int32_t* ids, T* out, int64_t count,
                                                   int64_t vocab, int cols, int32_t* bad_id) {
  __shared__ uint4 stage[4][kSegmentBytes / 16];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint4* slice = stage[wave];
  const uint16_t* halves = reinterpret_cast<const uint16_t*>(slice);
  const int blocks = cols / 32;
  const int segments = (blocks + kSegmentBlocks - 1) / kSegmentBlocks;
  const int64_t row_bytes = (int64_t)blocks * 34;
  const int64_t items = count * segments;
  const int64_t stride = (int64_t)gridDim.x * 4;
  Stage<ALIGNED> st;
  // an item: its id (negative when outside the table), first block, block count
  auto locate = [&](int64_t item, int64_t& id, int& first, int& nb) {
    const int64_t t = item / segments;
    first = (int)(item % segments) * kSegmentBlocks;
    nb = min(kSegmentBlocks, blocks - first);
    id = ids[t];
    if (id >= vocab) id = -1;
  };
  int64_t item = (int64_t)blockIdx.x * 4 + wave;
  int64_t id = -1;
  int first = 0, nb = 0;
  if (item < items) {
    locate(item, id, first, nb);
    if (id >= 0) st.load(table + id * row_bytes + (int64_t)first * 34, nb * 34, lane);
  }
  for (; item < items; item += stride) {
    const int64_t t = item / segments;
    T* target = out + t * cols + (int64_t)first * 32;
    const int64_t this_id = id;
    const int this_nb = nb;
    if (this_id >= 0) {
      wave_sync();  // the previous item has been read from the slice
      st.store(slice, table + this_id * row_bytes + (int64_t)first * 34, this_nb * 34, lane);
      wave_sync();
    }
    // the next item's bytes load while this one decodes
    if (item + stride < items) {
      locate(item + stride, id, first, nb);
      if (id >= 0) st.load(table + id * row_bytes + (int64_t)first * 34, nb * 34, lane);
    }
    if (this_id < 0) {
      const float zeros[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int q = lane; q < this_nb * 4; q += kWave) store8<T>(target + q * 8, zeros);
      if (bad_id && lane == 0) *bad_id = 1;
      continue;
    }
    // 8 values per step: block b = q / 4, its quarter q % 4. Infinite and
    // NaN scales take the slow path only in a wave that holds one.
    for (int q = lane; q < this_nb * 4; q += kWave) {
      const int b = q >> 2, part = q & 3;
      const uint32_t h = halves[b * 17];
      const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
      const bool special = (h & 0x7c00u) == 0x7c00u;
      uint32_t pairs[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pairs[i] = halves[b * 17 + 1 + part * 4 + i];
      float v[8];
      if (__builtin_expect(__any(special), 0)) {
        const uint32_t nan_bits = ((h & 0x8000u) << 16) | 0x7fc00000u | ((h & 0x3ffu) << 13);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[2 * i] = decode((int)(int8_t)(pairs[i] & 0xffu), d, special, nan_bits);
          v[2 * i + 1] = decode((int)(int8_t)(pairs[i] >> 8), d, special, nan_bits);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[2 * i] = (float)(int8_t)(pairs[i] & 0xffu) * d;
          v[2 * i + 1] = (float)(int8_t)(pairs[i] >> 8) * d;
        }
      }
      store8<T>(target + q * 8, v);
    }
  }
}

template <typename T>
int embedding_q8_0(const char* entry, const uint8_t* table, const int32_t* ids, T* out, int64_t count,
                   int64_t vocab, int32_t cols, int32_t* bad_id, void* stream) {
  clear_error();
  if (count < 0 || vocab < 0) return refuse("%s: %lld ids into %lld rows", entry, (long long)count, (long long)vocab);
  if (cols <= 0 || cols % 32 != 0) return refuse("%s: %d values are not whole Q8_0 blocks of 32", entry, cols);
  if (count == 0) return 0;
  if (!table || !ids || !out) return refuse("%s: null table, ids or out", entry);
  if (!aligned16(out)) return refuse("%s: out is not 16-byte aligned", entry);
  const int64_t row_bytes = (int64_t)cols / 32 * 34;
  const bool aligned = aligned16(table) && row_bytes % 16 == 0;
  const dim3 grid(grid_for(count, 4, 1 << 16));
  const hipStream_t s = (hipStream_t)stream;
  if (aligned)
    hipLaunchKernelGGL((q8_0_gather<T, true>), grid, dim3(256), 0, s, table, ids, out, count, vocab, cols, bad_id);
  else
    hipLaunchKernelGGL((q8_0_gather<T, false>), grid, dim3(256), 0, s, table, ids, out, count, vocab, cols, bad_id);
  return launched(entry);
}

}  // namespace
}  // namespace drift

using namespace drift;

extern "C" int drift_embedding_q8_0_f32(const uint8_t* table, const int32_t* ids, float* out, int64_t count,
                                        int64_t vocab, int32_t cols, int32_t* bad_id, void* stream) {
  return embedding_q8_0<float>("drift_embedding_q8_0_f32", table, ids, out, count, vocab, cols, bad_id, stream);
}

extern "C" int drift_embedding_q8_0_bf16(const uint8_t* table, const int32_t* ids, uint16_t* out, int64_t count,
                                         int64_t vocab, int32_t cols, int32_t* bad_id, void* stream) {
  return embedding_q8_0<uint16_t>("drift_embedding_q8_0_bf16", table, ids, out, count, vocab, cols, bad_id, stream);
}
