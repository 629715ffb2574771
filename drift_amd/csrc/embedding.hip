// Quantized token-embedding gather for gfx950: rows of a Q8_0 table decoded
// to F32 or BF16.
//
// Q8_0 (tensor/GgmlQuants.scala:104-118): every 32 values are a 34-byte
// block, an fp16 scale d then 32 int8 codes; value j = float(code j) * d,
// which is exact in float (11-bit by 8-bit significands), so the BF16 output
// is bit-exact against the reference's F32 gather rounded to BF16.
//
// One wave per slice of 128 chunks of a row (4 slices of a 4096-value row),
// the grid covering every slice in one pass. A lane owns chunks of 8
// consecutive values (a quarter of a block): it loads the chunk's 8 codes and
// the block's scale straight from the table row, decodes them and stores them
// as one 16-byte (BF16) or two 16-byte (F32) writes, so a store instruction
// of the wave covers a contiguous 1 or 2 KiB of the output row. A lane's two
// chunks are loaded back to back (indices clamped, not branched, so no load
// waits on another) before either is decoded. Measured on MI355X at 8192 rows
// of 4096: 2 chunks per lane 18.4 us, 4 19.1 us, 8 (a wave per row) 20.2 us,
// 1 27.4 us.
//
// What bounds it is where the rows lie, not the wait for the id: drawn at
// random from a [151936, 4096] table (661 MB, past the 256 MB MALL) the rows
// come from scattered DRAM pages, 19.7 us a launch (per-dispatch median),
// where contiguous ids take 17.5 us, the contiguous 1:2 read/write stream's
// figure. A plain copy of the same random rows with no decode (a block per
// row, every load in flight at once) takes the same 19.7 us. Waves that
// take two to four rows each, loading every id before any row (20.4 to
// 26.2 us), and one-wave blocks (20.4 us) were slower.
//
// Rows of whole 256-value runs in a 16-byte aligned table (the runner's
// embeddings) take q8_0_gather_slices, which stages each wave's slice of
// the row in LDS first.
//
// Codes sit at 2-byte offsets (34-byte blocks). When rows start on 4-byte
// boundaries (an even number of blocks per row and a 4-byte aligned table) a
// chunk's 8 codes are read as one 12-byte window from the 4-byte boundary at
// or below them, clamped to end at the row's end, and shifted into place;
// otherwise they are read as four 2-byte loads.
#include "common.hpp"

namespace drift {
namespace {

constexpr int kChunksPerLane = 2;

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

// The 8 codes of chunk q (block q / 4, quarter q % 4) of a row, as raw bytes
// in two words, little-endian.
template <bool WORDS>
struct Codes;

template <>
struct Codes<true> {  // rows on 4-byte boundaries: one 12-byte window
  uint3 w;
  uint32_t offset;  // 0, 2 or 4: where the codes start in the window
  __device__ __forceinline__ void load(const uint8_t* row, int64_t row_bytes, int q) {
    const int64_t at = (int64_t)(q >> 2) * 34 + 2 + (q & 3) * 8;
    const int64_t base = min(at & ~(int64_t)3, row_bytes - 12);
    offset = (uint32_t)(at - base);
    w = *reinterpret_cast<const uint3*>(row + base);
  }
  __device__ __forceinline__ void words(uint32_t& lo, uint32_t& hi) const {
    lo = offset == 4 ? w.y : __builtin_amdgcn_alignbyte(w.y, w.x, offset);
    hi = offset == 4 ? w.z : __builtin_amdgcn_alignbyte(w.z, w.y, offset);
  }
};

template <>
struct Codes<false> {  // rows on 2-byte boundaries: four 2-byte loads
  uint16_t h[4];
  __device__ __forceinline__ void load(const uint8_t* row, int64_t, int q) {
    const uint16_t* codes = reinterpret_cast<const uint16_t*>(row + (int64_t)(q >> 2) * 34 + 2 + (q & 3) * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = codes[i];
  }
  __device__ __forceinline__ void words(uint32_t& lo, uint32_t& hi) const {
    lo = h[0] | ((uint32_t)h[1] << 16);
    hi = h[2] | ((uint32_t)h[3] << 16);
  }
};

template <typename T, bool WORDS>
__global__ void __launch_bounds__(256) q8_0_gather(const uint8_t* table, const int32_t* ids, T* out, int64_t count,
                                                   int64_t vocab, int cols, int32_t* bad_id, int slices) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blocks = cols / 32;
  const int chunks = blocks * 4;
  const int64_t row_bytes = (int64_t)blocks * 34;
  const int64_t item = (int64_t)blockIdx.x * 4 + wave;
  const int64_t t = item / slices;
  if (t >= count) return;
  const int first = (int)(item - t * slices) * kChunksPerLane * kWave;
  const int64_t id = ids[t];
  T* target = out + t * cols;
  if (id < 0 || id >= vocab) {
    const float zeros[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int end = min(chunks, first + kChunksPerLane * kWave);
    for (int q = first + lane; q < end; q += kWave) store8<T>(target + q * 8, zeros);
    if (bad_id && lane == 0) *bad_id = 1;
    return;
  }
  const uint8_t* row = table + id * row_bytes;
  Codes<WORDS> codes[kChunksPerLane];
  uint32_t scale[kChunksPerLane];
#pragma unroll
  for (int k = 0; k < kChunksPerLane; ++k) {
    const int q = min(first + k * kWave + lane, chunks - 1);
    codes[k].load(row, row_bytes, q);
    scale[k] = *reinterpret_cast<const uint16_t*>(row + (int64_t)(q >> 2) * 34);
  }
#pragma unroll
  for (int k = 0; k < kChunksPerLane; ++k) {
    const int q = first + k * kWave + lane;
    if (q >= chunks) break;
    uint32_t lo, hi;
    codes[k].words(lo, hi);
    const uint32_t h = scale[k];
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    const bool special = (h & 0x7c00u) == 0x7c00u;
    const uint32_t pairs[4] = {lo & 0xffffu, lo >> 16, hi & 0xffffu, hi >> 16};
    float v[8];
    // infinite and NaN scales take the slow path only in a wave that holds one
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

// Rows of whole 256-value runs from a 16-byte aligned table (a wave's slice
// of CPL * 64 chunks then starts on a 16-byte boundary, 1,088 bytes for 2
// chunks a lane): the wave copies its slice into its own LDS with 16-byte
// loads (68 a wave, all in flight together), then each lane reads its
// chunks' code windows and scales from there; no barrier, the slice is the
// wave's alone. Half the load instructions of the direct gather below, each
// one aligned: 19.1-19.3 us against 19.6-19.7 at 8192 random rows of
// [151936, 4096] (a block per id copying its row to LDS behind a barrier took
// 20.2-20.3).
template <typename T, int CPL>
__global__ void __launch_bounds__(256) q8_0_gather_slices(const uint8_t* table, const int32_t* ids, T* out,
                                                          int64_t count, int64_t vocab, int cols, int32_t* bad_id,
                                                          int slices) {
  constexpr int kSliceBytes = CPL * kWave / 4 * 34;  // 1,088 for 2 chunks a lane
  constexpr int kSlicePieces = kSliceBytes / 16;
  constexpr int kLoads = (kSlicePieces + kWave - 1) / kWave;
  __shared__ __align__(16) uint32_t staged[4][kSliceBytes / 4 + 4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int chunks = cols / 8;
  const int64_t row_bytes = (int64_t)cols / 32 * 34;
  const int64_t item = (int64_t)blockIdx.x * 4 + wave;
  const int64_t t = item / slices;
  if (t >= count) return;
  const int slice = (int)(item - t * slices);
  const int first = slice * CPL * kWave;
  const int64_t id = ids[t];
  T* target = out + t * cols;
  if (id < 0 || id >= vocab) {
    const float zeros[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int end = min(chunks, first + CPL * kWave);
    for (int q = first + lane; q < end; q += kWave) store8<T>(target + q * 8, zeros);
    if (bad_id && lane == 0) *bad_id = 1;
    return;
  }
  // the slice's pieces, the last slice's cut at the row's end
  const int pieces = (int)min((int64_t)kSlicePieces, (row_bytes - (int64_t)slice * kSliceBytes) / 16);
  const uint4* from = reinterpret_cast<const uint4*>(table + id * row_bytes + (int64_t)slice * kSliceBytes);
  uint4* into = reinterpret_cast<uint4*>(staged[wave]);
  uint4 piece[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) piece[i] = stream_load(from + min(lane + i * kWave, pieces - 1));
#pragma unroll
  for (int i = 0; i < kLoads; ++i)
    if (lane + i * kWave < pieces) into[lane + i * kWave] = piece[i];
  wave_sync();
  const uint16_t* halves = reinterpret_cast<const uint16_t*>(staged[wave]);
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int q = first + k * kWave + lane;
    if (q >= chunks) break;
    const int local = q - first;  // the chunk within the slice
    const int at = (local >> 2) * 34 + 2 + (local & 3) * 8;
    const int word = at >> 2;
    const uint32_t offset = (uint32_t)(at & 3);
    const uint32_t w0 = staged[wave][word], w1 = staged[wave][word + 1], w2 = staged[wave][word + 2];
    const uint32_t lo = __builtin_amdgcn_alignbyte(w1, w0, offset), hi = __builtin_amdgcn_alignbyte(w2, w1, offset);
    const uint32_t h = halves[(local >> 2) * 17];
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    const bool special = (h & 0x7c00u) == 0x7c00u;
    const uint32_t pairs[4] = {lo & 0xffffu, lo >> 16, hi & 0xffffu, hi >> 16};
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

template <typename T>
int embedding_q8_0(const char* entry, const uint8_t* table, const int32_t* ids, T* out, int64_t count,
                   int64_t vocab, int32_t cols, int32_t* bad_id, void* stream) {
  clear_error();
  if (count < 0 || vocab < 0) return refuse("%s: %lld ids into %lld rows", entry, (long long)count, (long long)vocab);
  if (cols <= 0 || cols % 32 != 0) return refuse("%s: %d values are not whole Q8_0 blocks of 32", entry, cols);
  if (count == 0) return 0;
  if (!table || !ids || !out) return refuse("%s: null table, ids or out", entry);
  if (!aligned16(out)) return refuse("%s: out is not 16-byte aligned", entry);
  if (reinterpret_cast<uintptr_t>(table) & 1u) return refuse("%s: table is not 2-byte aligned", entry);
  const int64_t row_bytes = (int64_t)cols / 32 * 34;
  const bool words = (reinterpret_cast<uintptr_t>(table) & 3u) == 0 && row_bytes % 4 == 0;
  // a wave per slice of kChunksPerLane * 64 chunks of a row
  const int slices = (int)ceil_div(cols / 8, kChunksPerLane * kWave);
  const int64_t blocks = ceil_div(count * slices, 4);
  if (blocks > kOneShotBlocks) return refuse("%s: %lld ids", entry, (long long)count);
  const dim3 grid((unsigned)blocks);
  const hipStream_t s = (hipStream_t)stream;
  if (cols % 256 == 0 && aligned16(table)) {
    // 2 chunks a lane, as the direct gather (1: 24.1 us, 4: 21.1 us, 2: 19.2 us
    // at 8192 random rows of [151936, 4096])
    hipLaunchKernelGGL((q8_0_gather_slices<T, kChunksPerLane>), grid, dim3(256), 0, s, table, ids, out, count, vocab,
                       cols, bad_id, slices);
    return launched(entry);
  }
  if (words)
    hipLaunchKernelGGL((q8_0_gather<T, true>), grid, dim3(256), 0, s, table, ids, out, count, vocab, cols, bad_id,
                       slices);
  else
    hipLaunchKernelGGL((q8_0_gather<T, false>), grid, dim3(256), 0, s, table, ids, out, count, vocab, cols, bad_id,
                       slices);
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
