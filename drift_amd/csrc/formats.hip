// Rows of tables in the runner's other storage types, decoded on gfx950: the
// embedding gather of any GGUF quant the runner reads (Q4_0, Q4_1, Q5_0,
// Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS, ROCmFP4 dual and fast) or
// dense type (F32, F16, BF16), to F32 or BF16; and whole tables decoded to
// BF16 or F16 for the runner's GEMM path (kernels/matvec.hip:814-839,
// 891-897, the gather_<q> and dequantize_bf16_<q> instances at :942-954).
//
// A thread decodes one chunk of 8 consecutive values of a row (blocks of 32
// values are 4 chunks, blocks of 256 are 32) and stores it as one 16-byte
// (BF16, F16) or two 16-byte (F32) writes, so consecutive threads write
// consecutive output; the grid covers every chunk in one pass. Each format
// reads its fields with the widest loads its block alignment allows (2, 4 or
// 8 bytes; ROCmFP4's 17-byte fast blocks byte by byte).
//
// Arithmetic is each decoder's in the reference (tensor/GgmlQuants.scala,
// tensor/KQuants.scala, tensor/IQuants.scala, tensor/RocmFp4.scala), in
// float, operation by operation (-ffp-contract=off): the outputs are
// bit-exact, BF16 being the F32 result rounded to nearest even.
#include "common.hpp"

namespace drift {
namespace {

// ---------------------------------------------------------------- field loads

__device__ __forceinline__ uint32_t ld8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ __forceinline__ float f16_value(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// 8 bytes as two little-endian words, read with loads of `align` bytes.
template <int align>
__device__ __forceinline__ uint2 bytes8(const uint8_t* p) {
  if constexpr (align >= 8) return *reinterpret_cast<const uint2*>(p);
  if constexpr (align == 4) return make_uint2(ld32(p), ld32(p + 4));
  if constexpr (align == 2) return make_uint2(ld16(p) | (ld16(p + 2) << 16), ld16(p + 4) | (ld16(p + 6) << 16));
  uint32_t w[2] = {0, 0};
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i / 4] |= ld8(p + i) << (8 * (i % 4));
  return make_uint2(w[0], w[1]);
}

__device__ __forceinline__ uint32_t byte_of(uint2 w, int k) { return ((k < 4 ? w.x : w.y) >> (8 * (k % 4))) & 0xffu; }
__device__ __forceinline__ int nibble_of(uint2 w, int k, int shift) { return (int)((byte_of(w, k) >> shift) & 0xfu); }

// IQuants.Values (tensor/IQuants.scala:14-16) and RocmFp4.Codebook
// (tensor/RocmFp4.scala:21-22). A kernel copies its format's table into LDS
// (`lut`) once: read per value with a lane's own index, a table in global
// memory costs a vector load per value.
__device__ __forceinline__ float lut_entry(int id, int i) {
  constexpr float kIq4Values[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
  constexpr float kRocmCodebook[16] = {0, 1, 2, 3, 4, 6, 8, 10, 0, -1, -2, -3, -4, -6, -8, -10};
  return id == 1 ? kIq4Values[i] : kRocmCodebook[i];
}

// RocmFp4.halfScale (tensor/RocmFp4.scala:27-39): half an unsigned E4M3 byte,
// 0 past 0x7e.
__device__ __forceinline__ float rocm_half_scale(uint32_t byte) {
  if (byte > 0x7eu) return 0.0f;
  const int exponent = (int)(byte >> 3), mantissa = (int)(byte & 7u);
  if (exponent == 0) return ldexpf((float)mantissa, -10);
  return (float)(8 + mantissa) * ldexpf(1.0f, exponent - 11);
}

// ---------------------------------------------------------------- decoders
// decode(block, c, v): chunk c of the block (values 8c .. 8c + 7) into v.

struct Q4_0 {  // GgmlQuants.scala:13-29: d * (q - 8)
  static constexpr int kValues = 32, kBytes = 18, kAlign = 2;
  static constexpr int kLut = 0;
  template <int A = kAlign>
  __device__ static void decode(const uint8_t* b, int c, float (&v)[8], const float* lut) {
    const float d = f16_value(ld16(b));
    const uint2 w = bytes8<A>(b + 2 + 8 * (c & 1));
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = d * (float)(nibble_of(w, k, 4 * (c >> 1)) - 8);
  }
};

struct Q4_1 {  // :31-49: d * q + m
  static constexpr int kValues = 32, kBytes = 20, kAlign = 4;
  static constexpr int kLut = 0;
  template <int A = kAlign>
  __device__ static void decode(const uint8_t* b, int c, float (&v)[8], const float* lut) {
    const uint32_t dm = ld32(b);
    const float d = f16_value(dm & 0xffffu), m = f16_value(dm >> 16);
    const uint2 w = bytes8<A>(b + 4 + 8 * (c & 1));
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = d * (float)nibble_of(w, k, 4 * (c >> 1)) + m;
  }
};

// GgmlQuants.fiveBit (:53-64): bit j of qh is value j's fifth bit.
template <bool MIN>
struct Q5 {  // Q5_0 (:66-81) d * (q - 16); Q5_1 (:83-99) d * q + m
  static constexpr int kValues = 32, kBytes = MIN ? 24 : 22, kAlign = MIN ? 4 : 2;
  static constexpr int kLut = 0;
  template <int A = kAlign>
  __device__ static void decode(const uint8_t* b, int c, float (&v)[8], const float* lut) {
    float d, m = 0.0f;
    uint32_t qh;
    if constexpr (MIN) {
      const uint32_t dm = ld32(b);
      d = f16_value(dm & 0xffffu);
      m = f16_value(dm >> 16);
      qh = ld32(b + 4);
    } else {
      d = f16_value(ld16(b));
      qh = ld16(b + 2) | (ld16(b + 4) << 16);
    }
    const uint2 w = bytes8<A>(b + (MIN ? 8 : 6) + 8 * (c & 1));
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int j = 8 * c + k;
      const int q = nibble_of(w, k, 4 * (c >> 1)) | (int)(((qh >> j) & 1u) << 4);
      if constexpr (MIN)
        v[k] = d * (float)q + m;
      else
        v[k] = d * (float)(q - 16);
    }
  }
};

struct Q8_0 {  // :101-117: q * d (plain IEEE products; the Q8_0 gather kernel also matches x86's NaNs)
  static constexpr int kValues = 32, kBytes = 34, kAlign = 2;
  static constexpr int kLut = 0;
  template <int A = kAlign>
  __device__ static void decode(const uint8_t* b, int c, float (&v)[8], const float* lut) {
    const float d = f16_value(ld16(b));
    const uint2 w = bytes8<A>(b + 2 + 8 * c);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = (float)(int8_t)byte_of(w, k) * d;
  }
};

// KQuants.scaleAndMin (tensor/KQuants.scala:55-70): sub-block j's 6-bit scale
// and min from the 12 bytes s (three words).
__device__ __forceinline__ void scale_and_min(const uint32_t (&s)[3], int j, int& scale, int& min) {
  auto byte = [&](int i) { return (int)((s[i / 4] >> (8 * (i % 4))) & 0xffu); };
  if (j < 4) {
    scale = byte(j) & 63;
    min = byte(j + 4) & 63;
  } else {
    scale = (byte(j + 4) & 0xf) | ((byte(j - 4) >> 2) & 0x30);
    min = (byte(j + 4) >> 4) | ((byte(j) >> 2) & 0x30);
  }
}

template <bool FIVE>
struct QK45 {  // Q4_K (KQuants.scala:102-110), Q5_K (:112-121): d * sc * q - dmin * m, per 32
  static constexpr int kValues = 256, kBytes = FIVE ? 176 : 144, kAlign = 8;
  static constexpr int kLut = 0;
  template <int A = kAlign>
  __device__ static void decode(const uint8_t* b, int c, float (&v)[8], const float* lut) {
    const uint32_t dd = ld32(b);
    const uint32_t s[3] = {ld32(b + 4), ld32(b + 8), ld32(b + 12)};
    const int j = c / 4;  // the 32-value sub-block
    int scale, min;
    scale_and_min(s, j, scale, min);
    const float d = f16_value(dd & 0xffffu) * (float)scale;
    const float m = f16_value(dd >> 16) * (float)min;
    // KQuants.nibble (:47-53): chunk j's values are the low (even j) or high
    // nibbles of the 32 bytes at (j / 2) * 32
    const uint2 w = bytes8<A>(b + (FIVE ? 48 : 16) + (j / 2) * 32 + 8 * (c % 4));
    uint2 h = make_uint2(0, 0);
    if constexpr (FIVE) h = bytes8<A>(b + 16 + 8 * (c % 4));  // the fifth bits, bit j of byte e % 32
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      int q = nibble_of(w, k, 4 * (j % 2));
      if constexpr (FIVE) q |= (int)((byte_of(h, k) >> j) & 1u) << 4;
      v[k] = d * (float)q - m;
    }
  }
};

struct Q6_K {  // KQuants.scala:123-134: d * sc * (q - 32), q of six bits
  static constexpr int kValues = 256, kBytes = 210, kAlign = 2;
  static constexpr int kLut = 0;
  template <int A = kAlign>
  __device__ static void decode(const uint8_t* b, int c, float (&v)[8], const float* lut) {
    const int half = c / 16, r = c % 16;  // values 128 half + 8 r ..
    const uint2 low = bytes8<A>(b + half * 64 + 8 * (r % 8));  // nibble 4 (r / 8) of ql[half 64 + r' % 64]
    const uint2 high = bytes8<A>(b + 128 + half * 32 + 8 * (r % 4));  // KQuants.twoBits (:38-45)
    const float d = f16_value(ld16(b + 208)) * (float)(int8_t)ld8(b + 192 + c / 2);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int q = (nibble_of(low, k, 4 * (r / 8)) | ((int)((byte_of(high, k) >> (2 * (r / 4))) & 3u) << 4)) - 32;
      v[k] = d * (float)q;
    }
  }
};

struct IQ4_NL {  // IQuants.scala:18-47: d * Values(q)
  static constexpr int kValues = 32, kBytes = 18, kAlign = 2;
  static constexpr int kLut = 1;
  template <int A = kAlign>
  __device__ static void decode(const uint8_t* b, int c, float (&v)[8], const float* lut) {
    const float d = f16_value(ld16(b));
    const uint2 w = bytes8<A>(b + 2 + 8 * (c & 1));
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = d * lut[nibble_of(w, k, 4 * (c >> 1))];
  }
};

struct IQ4_XS {  // IQuants.scala:49-80: run i scaled by d * (ls - 32)
  static constexpr int kValues = 256, kBytes = 136, kAlign = 8;
  static constexpr int kLut = 1;
  template <int A = kAlign>
  __device__ static void decode(const uint8_t* b, int c, float (&v)[8], const float* lut) {
    const int i = c / 4, r = c % 4;  // run i, chunk r of its 4
    const float d = f16_value(ld16(b));
    const uint32_t high = ld16(b + 2);
    const uint32_t low = (ld8(b + 4 + i / 2) >> (4 * (i % 2))) & 0xfu;
    const int ls = (int)(low | (((high >> (2 * i)) & 3u) << 4));
    const float scale = d * (float)(ls - 32);
    const uint2 w = bytes8<A>(b + 8 + 16 * i + 8 * (r & 1));
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = scale * lut[nibble_of(w, k, 4 * (r >> 1))];
  }
};

template <bool FAST>
struct RocmFp4 {  // RocmFp4.scala:45-62: Codebook(q) * halfScale, a scale per half (one for FAST)
  static constexpr int kValues = 32, kBytes = FAST ? 17 : 18, kAlign = FAST ? 1 : 2;
  static constexpr int kLut = 2;
  template <int A = kAlign>
  __device__ static void decode(const uint8_t* b, int c, float (&v)[8], const float* lut) {
    const uint2 w = bytes8<A>(b + 8 * (c & 1));
    const float scale = rocm_half_scale(ld8(b + (FAST ? 16 : 16 + (c >> 1))));
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = lut[nibble_of(w, k, 4 * (c >> 1))] * scale;
  }
};

// Dense rows: 8 values from 16 or 32 bytes (16-byte aligned rows).
template <int FORMAT>
struct Dense {
  static constexpr int kValues = 1, kBytes = FORMAT == DRIFT_F32 ? 4 : 2, kAlign = 16;
  static constexpr int kLut = 0;
  template <int A = kAlign>
  __device__ static void decode(const uint8_t* b, int c, float (&v)[8], const float* lut) {
    if constexpr (FORMAT == DRIFT_F32) {
      float4 a = *reinterpret_cast<const float4*>(b + 32 * c), z = *reinterpret_cast<const float4*>(b + 32 * c + 16);
      v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = z.x, v[5] = z.y, v[6] = z.z, v[7] = z.w;
    } else {
      const uint4 q = *reinterpret_cast<const uint4*>(b + 16 * c);
      const uint32_t words[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t h = (words[k / 2] >> (16 * (k % 2))) & 0xffffu;
        v[k] = FORMAT == DRIFT_F16 ? f16_value(h) : __uint_as_float(h << 16);
      }
    }
  }
};

// ---------------------------------------------------------------- kernels

template <typename T>
__device__ __forceinline__ void store_chunk(T* p, const float (&v)[8]);

template <>
__device__ __forceinline__ void store_chunk<float>(float* p, const float (&v)[8]) {
  Chunk<float>::store(p, *reinterpret_cast<const float(*)[4]>(v));
  Chunk<float>::store(p + 4, *reinterpret_cast<const float(*)[4]>(v + 4));
}

template <>
__device__ __forceinline__ void store_chunk<uint16_t>(uint16_t* p, const float (&v)[8]) {
  Chunk<uint16_t>::store(p, v);
}

// F16 out (the GEMM path's dequantize): to nearest even.
struct Half {
  uint16_t bits;
};

template <>
__device__ __forceinline__ void store_chunk<Half>(Half* p, const float (&v)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    w[k] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * k]) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * k + 1]) << 16);
  __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]}, reinterpret_cast<u32x4*>(p));
}

// Rows ids[t] (row t with no ids) of a table of format F into out [count,
// cols], a thread per chunk of 8 values. An id outside [0, vocab) gets a row
// of zeros and sets *bad_id. BY_ROW: the grid's y is the row (at most 65535
// rows) and its x the row's blocks of 256 chunks, so no thread divides; else
// a one-dimensional grid over every chunk, the row by a reciprocal quotient.
template <typename T, typename F, bool BY_ROW = false>
__global__ void __launch_bounds__(256) decode_rows(const uint8_t* table, const int32_t* ids, T* out, int64_t count,
                                                   int64_t vocab, int cols, int64_t row_bytes, int32_t* bad_id,
                                                   double row_inverse) {
  constexpr int kChunks = F::kValues / 8 > 0 ? F::kValues / 8 : 1;  // chunks per block
  __shared__ float lut[16];
  if constexpr (F::kLut != 0) {
    if (threadIdx.x < 16) lut[threadIdx.x] = lut_entry(F::kLut, (int)threadIdx.x);
    __syncthreads();
  }
  const int per_row = cols / 8;
  auto chunk = [&](int64_t t, int q) {
    const int64_t id = ids ? ids[t] : t;
    float v[8];
    if (id < 0 || id >= vocab) {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = 0.0f;
      if (bad_id) *bad_id = 1;
    } else if constexpr (F::kValues == 1) {
      F::decode(table + id * row_bytes, q, v, lut);
    } else {
      F::decode(table + id * row_bytes + (int64_t)(q / kChunks) * F::kBytes, q % kChunks, v, lut);
    }
    store_chunk<T>(out + t * cols + (int64_t)q * 8, v);
  };
  if constexpr (BY_ROW) {
    const int q = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (q < per_row) chunk((int64_t)blockIdx.y, q);
  } else {
    const int64_t total = count * per_row;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      const int64_t t = quotient(i, per_row, row_inverse);  // not a 64-bit division a chunk
      chunk(t, (int)(i - t * per_row));
    }
  }
}

// Dense tables of any width and alignment (the reference's gather_rows_f32,
// kernels/elementwise.hip:89-93, takes any width): a thread per value.
__device__ __forceinline__ void store_value(float* p, float v) { *p = v; }
__device__ __forceinline__ void store_value(uint16_t* p, float v) { *p = (uint16_t)bf16_bits(v); }
__device__ __forceinline__ void store_value(Half* p, float v) { p->bits = __builtin_bit_cast(uint16_t, (_Float16)v); }

template <typename T, int FORMAT>
__global__ void __launch_bounds__(256) dense_values(const uint8_t* table, const int32_t* ids, T* out, int64_t count,
                                                    int64_t vocab, int cols, int32_t* bad_id, double col_inverse) {
  const int64_t total = count * cols;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t t = quotient(i, cols, col_inverse);
    const int64_t id = ids ? ids[t] : t;
    float v = 0.0f;
    if (id < 0 || id >= vocab) {
      if (bad_id) *bad_id = 1;
    } else {
      const int64_t at = id * cols + (i - t * cols);
      if constexpr (FORMAT == DRIFT_F32)
        v = reinterpret_cast<const float*>(table)[at];
      else if constexpr (FORMAT == DRIFT_F16)
        v = f16_value(reinterpret_cast<const uint16_t*>(table)[at]);
      else
        v = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(table)[at] << 16);
    }
    store_value(out + i, v);
  }
}

// The 256-value formats (the K-quants, IQ4_XS) through LDS, for more rows
// than decode_rows' two-dimensional grid holds: each half wave copies one
// block (144 to 210 bytes) into LDS with a few coalesced 4- or 2-byte loads a
// lane, then its 32 lanes decode their chunks from there, so the block's
// scales and fields are read from HBM once, not by every lane with its own
// small loads. Two blocks a wave, waves independent. (At [14336, 4096] the
// two-dimensional decode_rows beat it for every 256-value format: Q4_K 25.3
// against 27.3 us, Q6_K 26.8 against 32.3, IQ4_XS 23.2 against 29.1.)
template <typename T, typename F>
__global__ void __launch_bounds__(256) decode_staged(const uint8_t* table, const int32_t* ids, T* out, int64_t count,
                                                     int64_t vocab, int cols, int64_t row_bytes, int32_t* bad_id) {
  static_assert(F::kValues == 256, "a block is 32 chunks");
  constexpr int kPad = (F::kBytes + 7) / 8 * 8;  // blocks on 8-byte boundaries: 8-byte field reads
  constexpr int kPiece = F::kAlign >= 4 && F::kBytes % 4 == 0 ? 4 : 2;
  constexpr int kPieces = F::kBytes / kPiece;
  __shared__ __align__(16) uint8_t staged[8][kPad];
  __shared__ float lut[16];
  if constexpr (F::kLut != 0) {
    if (threadIdx.x < 16) lut[threadIdx.x] = lut_entry(F::kLut, (int)threadIdx.x);
    __syncthreads();
  }
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6, half = lane >> 5, c = lane & 31;
  uint8_t* mine = staged[wave * 2 + half];
  const int per_row = cols / 256;
  const int64_t blocks = count * per_row;
  for (int64_t first = (int64_t)blockIdx.x * 8 + wave * 2; first < blocks; first += (int64_t)gridDim.x * 8) {
    const int64_t block = min(first + half, blocks - 1);  // a half past the last block mirrors it
    const int64_t t = block / per_row;
    const int b = (int)(block - t * per_row);
    const int64_t id = ids ? ids[t] : t;
    const bool bad = id < 0 || id >= vocab;
    const uint8_t* src = table + (bad ? 0 : id) * row_bytes + (int64_t)b * F::kBytes;
#pragma unroll
    for (int k = 0; k < (kPieces + 31) / 32; ++k) {
      const int piece = c + 32 * k;
      if (piece < kPieces) {
        if constexpr (kPiece == 4)
          *reinterpret_cast<uint32_t*>(mine + 4 * piece) = ld32(src + 4 * piece);
        else
          *reinterpret_cast<uint16_t*>(mine + 2 * piece) = (uint16_t)ld16(src + 2 * piece);
      }
    }
    wave_sync();
    float v[8];
    if (bad) {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = 0.0f;
      if (bad_id) *bad_id = 1;
    } else {
      F::template decode<8>(mine, c, v, lut);
    }
    if (first + half < blocks) store_chunk<T>(out + t * cols + (int64_t)b * 256 + c * 8, v);
    wave_sync();  // the block's reads are done before the next copy
  }
}

// Block formats a run of 2048 values at a time (8 blocks of 256 or 64 of 32),
// for rows of whole runs on 16-byte boundaries: a one-wave block copies the
// run's bytes (1,152 to 1,408 for the formats that take it, a multiple of 16)
// into LDS with 16-byte loads, all in flight together, then each lane decodes
// 4 chunks (chunk k * 64 + lane of the run's 256) from there, so each store
// instruction writes 64 consecutive 16-byte pieces and a block's scales are
// read from LDS by the lanes that share them.
constexpr int kRunValues = 2048;

// rows a grid's y dimension holds (decode_rows' BY_ROW form)
constexpr int64_t kMaxGridRows = 65535;

template <typename F>
constexpr int run_pieces() {
  return kRunValues / F::kValues * F::kBytes / 16;
}

// a run's blocks start every kBytes from a 16-byte boundary: the largest
// power of two dividing kBytes, at most 8, is each one's alignment
template <typename F>
constexpr int run_field_align() {
  return (F::kBytes & -F::kBytes) < 8 ? (F::kBytes & -F::kBytes) : 8;
}

// Whether a format's rows of whole runs take decode_runs rather than
// decode_rows by row (its two-dimensional grid). Timed on a [14336, 4096]
// weight decoded to bf16, the two decoders' graph replays alternating with
// the format's stream probe, both orders (us, runs / by row): Q4_K 25.0 /
// 28.1, Q5_K 26.4 / 32.9, IQ4_NL 25.3 / 25.7 and ROCmFP4 25.4 / 26.9 take
// runs; Q5_1 26.6 / 25.7, Q6_K 30.8 / 29.7, IQ4_XS 27.3 / 26.3 and ROCmFP4
// fast 27.4 / 27.0 decode by row, as do Q4_0, Q4_1, Q5_0 and Q8_0.
template <typename F>
struct TakesRuns {
  static constexpr bool value = false;
};
template <bool FIVE>
struct TakesRuns<QK45<FIVE>> {
  static constexpr bool value = true;
};
template <>
struct TakesRuns<IQ4_NL> {
  static constexpr bool value = true;
};
template <>
struct TakesRuns<RocmFp4<false>> {
  static constexpr bool value = true;
};

template <typename T, typename F>
__global__ void __launch_bounds__(kWave) decode_runs(const uint8_t* table, const int32_t* ids, T* out, int64_t count,
                                                     int64_t vocab, int cols, int64_t row_bytes, int32_t* bad_id) {
  static_assert(F::kValues >= 8 && (kRunValues / F::kValues * F::kBytes) % 16 == 0, "runs of whole 16-byte pieces");
  constexpr int kPieces = run_pieces<F>();
  constexpr int kLoads = (kPieces + kWave - 1) / kWave;
  constexpr int kFieldAlign = run_field_align<F>();
  constexpr int kBlockChunks = F::kValues / 8;
  static_assert(kFieldAlign >= F::kAlign, "the run keeps each block's alignment");
  __shared__ __align__(16) uint8_t staged[kPieces * 16];
  __shared__ float lut[16];
  const int lane = (int)threadIdx.x;
  if constexpr (F::kLut != 0) {
    if (lane < 16) lut[lane] = lut_entry(F::kLut, lane);
  }
  const int runs_per_row = cols / kRunValues;
  const int64_t run = blockIdx.x;
  const int64_t t = run / runs_per_row;
  const int r = (int)(run - t * runs_per_row);
  const int64_t id = ids ? ids[t] : t;
  const bool bad = id < 0 || id >= vocab;
  const uint4* src = reinterpret_cast<const uint4*>(table + (bad ? 0 : id) * row_bytes +
                                                    (int64_t)r * (kRunValues / F::kValues) * F::kBytes);
  uint4 piece[kLoads];
#pragma unroll
  for (int k = 0; k < kLoads; ++k) piece[k] = stream_load(src + min(lane + k * kWave, kPieces - 1));
#pragma unroll
  for (int k = 0; k < kLoads; ++k)
    if (lane + k * kWave < kPieces) reinterpret_cast<uint4*>(staged)[lane + k * kWave] = piece[k];
  wave_sync();
  if (bad && bad_id && lane == 0) *bad_id = 1;
  T* target = out + t * cols + (int64_t)r * kRunValues;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int chunk = k * kWave + lane;
    float v[8];
    if (bad) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    } else {
      F::template decode<kFieldAlign>(staged + (chunk / kBlockChunks) * F::kBytes, chunk % kBlockChunks, v, lut);
    }
    store_chunk<T>(target + chunk * 8, v);
  }
}

// ---------------------------------------------------------------- launch layer

// A format's block and alignment, for the checks: values, bytes, alignment.
struct Layout {
  int values = 0, bytes = 0, align = 0;
};

Layout layout(int32_t format) {
  switch (format) {
#define DRIFT_LAYOUT(CODE, F) \
  case CODE:                  \
    return Layout{F::kValues, F::kBytes, F::kAlign};
    DRIFT_LAYOUT(DRIFT_F32, Dense<DRIFT_F32>)
    DRIFT_LAYOUT(DRIFT_F16, Dense<DRIFT_F16>)
    DRIFT_LAYOUT(DRIFT_BF16, Dense<DRIFT_BF16>)
    DRIFT_LAYOUT(DRIFT_Q4_0, Q4_0)
    DRIFT_LAYOUT(DRIFT_Q4_1, Q4_1)
    DRIFT_LAYOUT(DRIFT_Q5_0, Q5<false>)
    DRIFT_LAYOUT(DRIFT_Q5_1, Q5<true>)
    DRIFT_LAYOUT(DRIFT_Q8_0, Q8_0)
    DRIFT_LAYOUT(DRIFT_Q4_K, QK45<false>)
    DRIFT_LAYOUT(DRIFT_Q5_K, QK45<true>)
    DRIFT_LAYOUT(DRIFT_Q6_K, Q6_K)
    DRIFT_LAYOUT(DRIFT_IQ4_NL, IQ4_NL)
    DRIFT_LAYOUT(DRIFT_IQ4_XS, IQ4_XS)
    DRIFT_LAYOUT(DRIFT_Q4_0_ROCMFP4, RocmFp4<false>)
    DRIFT_LAYOUT(DRIFT_Q4_0_ROCMFP4_FAST, RocmFp4<true>)
#undef DRIFT_LAYOUT
    default:
      return Layout{};
  }
}

template <typename T>
int decode_launch(const char* entry, const void* table, int32_t format, const int32_t* ids, T* out, int64_t count,
                  int64_t vocab, int32_t cols, int32_t* bad_id, void* stream) {
  clear_error();
  const Layout l = layout(format);
  if (l.values == 0) return refuse("%s: no storage type %d", entry, format);
  if (count < 0 || vocab < 0) return refuse("%s: %lld rows of %lld", entry, (long long)count, (long long)vocab);
  const bool dense = l.values == 1;
  if (cols <= 0 || cols % l.values != 0 || (!dense && cols % 8 != 0))
    return refuse("%s: rows of %d values are not whole blocks of %d (and chunks of 8)", entry, cols, l.values);
  if (count == 0) return 0;
  if (!table || !out) return refuse("%s: null table or out", entry);
  const hipStream_t s = (hipStream_t)stream;
  if (dense && (cols % 8 != 0 || !aligned16(out) || !aligned16(table))) {
    // any width: element alignment only
    if (reinterpret_cast<uintptr_t>(table) % (uintptr_t)l.bytes != 0 ||
        reinterpret_cast<uintptr_t>(out) % sizeof(T) != 0)
      return refuse("%s: the table or out is not aligned to its elements", entry);
    const dim3 grid(grid_for(count * cols, 256, kOneShotBlocks));
    const auto* bytes = static_cast<const uint8_t*>(table);
    if (format == DRIFT_F32)
      hipLaunchKernelGGL((dense_values<T, DRIFT_F32>), grid, dim3(256), 0, s, bytes, ids, out, count, vocab, cols,
                         bad_id, 1.0 / (double)cols);
    else if (format == DRIFT_F16)
      hipLaunchKernelGGL((dense_values<T, DRIFT_F16>), grid, dim3(256), 0, s, bytes, ids, out, count, vocab, cols,
                         bad_id, 1.0 / (double)cols);
    else
      hipLaunchKernelGGL((dense_values<T, DRIFT_BF16>), grid, dim3(256), 0, s, bytes, ids, out, count, vocab, cols,
                         bad_id, 1.0 / (double)cols);
    return launched(entry);
  }
  if (!aligned16(out)) return refuse("%s: out is not 16-byte aligned", entry);
  if (reinterpret_cast<uintptr_t>(table) % (uintptr_t)l.align != 0)
    return refuse("%s: the table is not %d-byte aligned", entry, l.align);
  const int64_t row_bytes = (int64_t)cols / l.values * l.bytes;
  const int64_t chunks = count * (cols / 8);
  const dim3 grid(grid_for(chunks, 256, kOneShotBlocks));
  const auto* bytes = static_cast<const uint8_t*>(table);
  switch (format) {
#define DRIFT_DECODE(CODE, F)                                                                                     \
  case CODE:                                                                                                     \
    if constexpr (TakesRuns<F>::value) {                                                                        \
      const int64_t runs = count * (cols / kRunValues);                                                          \
      if (vocab > 0 && cols % kRunValues == 0 && aligned16(table) && runs <= kOneShotBlocks) {                   \
        hipLaunchKernelGGL((decode_runs<T, F>), dim3((unsigned)runs), dim3(kWave), 0, s, bytes, ids, out, count,  \
                           vocab, cols, row_bytes, bad_id);                                                      \
        break;                                                                                                   \
      }                                                                                                          \
    }                                                                                                            \
    if (count <= kMaxGridRows) {                                                                                 \
      hipLaunchKernelGGL((decode_rows<T, F, true>), dim3((unsigned)ceil_div(cols / 8, 256), (unsigned)count),      \
                         dim3(256), 0, s, bytes, ids, out, count, vocab, cols, row_bytes, bad_id, 0.0);           \
      break;                                                                                                       \
    }                                                                                                              \
    if constexpr (F::kValues == 256) {                                                                           \
      if (vocab > 0) {                                                                                           \
        const dim3 staged(grid_for(count * (cols / 256), 8, kOneShotBlocks));                                    \
        hipLaunchKernelGGL((decode_staged<T, F>), staged, dim3(256), 0, s, bytes, ids, out, count, vocab, cols,    \
                           row_bytes, bad_id);                                                                   \
        break;                                                                                                   \
      }                                                                                                          \
    }                                                                                                            \
    hipLaunchKernelGGL((decode_rows<T, F>), grid, dim3(256), 0, s, bytes, ids, out, count, vocab, cols, row_bytes, \
                       bad_id, 1.0 / (double)(cols / 8));                                                        \
    break;
    DRIFT_DECODE(DRIFT_F32, Dense<DRIFT_F32>)
    DRIFT_DECODE(DRIFT_F16, Dense<DRIFT_F16>)
    DRIFT_DECODE(DRIFT_BF16, Dense<DRIFT_BF16>)
    DRIFT_DECODE(DRIFT_Q4_0, Q4_0)
    DRIFT_DECODE(DRIFT_Q4_1, Q4_1)
    DRIFT_DECODE(DRIFT_Q5_0, Q5<false>)
    DRIFT_DECODE(DRIFT_Q5_1, Q5<true>)
    DRIFT_DECODE(DRIFT_Q8_0, Q8_0)
    DRIFT_DECODE(DRIFT_Q4_K, QK45<false>)
    DRIFT_DECODE(DRIFT_Q5_K, QK45<true>)
    DRIFT_DECODE(DRIFT_Q6_K, Q6_K)
    DRIFT_DECODE(DRIFT_IQ4_NL, IQ4_NL)
    DRIFT_DECODE(DRIFT_IQ4_XS, IQ4_XS)
    DRIFT_DECODE(DRIFT_Q4_0_ROCMFP4, RocmFp4<false>)
    DRIFT_DECODE(DRIFT_Q4_0_ROCMFP4_FAST, RocmFp4<true>)
#undef DRIFT_DECODE
  }
  return launched(entry);
}

}  // namespace
}  // namespace drift

using namespace drift;

extern "C" int drift_embedding_f32(const void* table, int32_t format, const int32_t* ids, float* out, int64_t count,
                                   int64_t vocab, int32_t cols, int32_t* bad_id, void* stream) {
  // Q8_0 rows take the gather kernel tuned for them (and matching x86's NaNs)
  if (format == DRIFT_Q8_0)
    return drift_embedding_q8_0_f32(static_cast<const uint8_t*>(table), ids, out, count, vocab, cols, bad_id, stream);
  if (!ids && count > 0) {
    clear_error();
    return refuse("drift_embedding_f32: null ids");
  }
  return decode_launch<float>("drift_embedding_f32", table, format, ids, out, count, vocab, cols, bad_id, stream);
}

extern "C" int drift_embedding_bf16(const void* table, int32_t format, const int32_t* ids, uint16_t* out,
                                    int64_t count, int64_t vocab, int32_t cols, int32_t* bad_id, void* stream) {
  if (format == DRIFT_Q8_0)
    return drift_embedding_q8_0_bf16(static_cast<const uint8_t*>(table), ids, out, count, vocab, cols, bad_id,
                                     stream);
  if (!ids && count > 0) {
    clear_error();
    return refuse("drift_embedding_bf16: null ids");
  }
  return decode_launch<uint16_t>("drift_embedding_bf16", table, format, ids, out, count, vocab, cols, bad_id, stream);
}

extern "C" int drift_dequantize_bf16(const void* table, int32_t format, uint16_t* out, int64_t rows, int32_t cols,
                                     void* stream) {
  return decode_launch<uint16_t>("drift_dequantize_bf16", table, format, nullptr, out, rows, rows, cols, nullptr,
                                 stream);
}

extern "C" int drift_dequantize_f16(const void* table, int32_t format, uint16_t* out, int64_t rows, int32_t cols,
                                    void* stream) {
  return decode_launch<Half>("drift_dequantize_f16", table, format, nullptr, reinterpret_cast<Half*>(out), rows,
                             rows, cols, nullptr, stream);
}
