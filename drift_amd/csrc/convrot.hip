// ConvRot's rotated linears, decoded on gfx950 where the file holds their
// codes: ComfyUI's int8_tensorwise (one int8 a value, a scale a row or one for
// all) and asym_w4a8_int8 (two 4-bit codes a byte, each a level of a 16-entry
// codebook times its group's fp8 relative scale, rounded and clamped to int8,
// times a scale a row), every 256 columns times the normalized regular
// Hadamard matrix (tensor/ConvRot.scala:20-50). Rows `ids` of one gathered as
// F32 or BF16 (the embedding, ops/HipLinear.scala:54-92), or the whole weight
// as BF16 for the GEMM path (ops/HipBase.scala:276-311, the convert of
// ops/HipMemory.scala:127-130); the reference's kernels are
// kernels/convrot.hip:84-121.
//
// The 256 x 256 matrix is the Kronecker fourth power of a 4 x 4 one, so the
// rotation is four rounds of 4-point butterflies over the base-4 digits of
// the column (strides 1, 4, 16, 64), each `half = (a + b + c + d) / 2` summed
// left to right, then `half - d, half - c, half - b, half - a`: float, in the
// CPU's order, no contraction, so outputs are the CPU's bit for bit.
//
// Layout on the wave: four lanes a group of 256 values, a lane a quarter of it
// (64 consecutive values, digits 0-2 in its registers, digit 3 its lane in the
// quad), 16 groups a wave. A lane loads its codes with 16-byte loads (64 B of
// int8, 32 B of nibbles; the int8 weight's decode loads the wave's 4 KiB whole
// and passes it through the wave's LDS), decodes, and runs the rounds of
// digits 0, 1 and 2 in registers. The quad then trades values through the
// wave's own LDS (4 KiB, a quarter of the values at a time), so that a lane
// holds digit 3 and digits 0-1 for one digit 2; it runs the last round in
// registers and passes its outputs back through the LDS so that every store
// instruction writes whole 128-byte lines (half-line stores had the L2 write
// 1.5 times the output to HBM). The trade's LDS slots are laid out so that
// neither the writes nor the reads of a 16-lane phase share a bank.
#include "common.hpp"

namespace drift {
namespace {

constexpr int kGroup = 256;       // ConvRot.Group
constexpr int kLaneValues = 64;   // a quarter group
constexpr int kWaveGroups = 16;   // 64 lanes, 4 a group
constexpr int kBlockWaves = 1;  // one-wave blocks: the finest dispatch (measured 1-5% faster than 4)

// fp8 E4M3 "fn" (tensor/DType.scala:105-115): bias 7, no infinities, NaN at
// S.1111.111.
__device__ __forceinline__ float e4m3(uint32_t code) {
  const int exponent = (int)((code >> 3) & 0xfu), mantissa = (int)(code & 7u);
  float magnitude;
  if (exponent == 0xf && mantissa == 7)
    magnitude = __builtin_nanf("");
  else if (exponent == 0)
    magnitude = ldexpf((float)mantissa, -9);
  else
    magnitude = ldexpf((float)(8 + mantissa), exponent - 10);
  return (code & 0x80u) ? -magnitude : magnitude;
}

// One butterfly of ConvRot.rotate (tensor/ConvRot.scala:33-42) on v[i],
// v[i + S], v[i + 2S], v[i + 3S].
template <int S>
__device__ __forceinline__ void butterfly(float* v, int i) {
  const float a = v[i], b = v[i + S], c = v[i + 2 * S], d = v[i + 3 * S];
  const float half = (((a + b) + c) + d) * 0.5f;
  v[i] = half - d;
  v[i + S] = half - c;
  v[i + 2 * S] = half - b;
  v[i + 3 * S] = half - a;
}

// A round over the 64 values of a lane: every butterfly of stride S.
template <int S>
__device__ __forceinline__ void round_of(float (&v)[kLaneValues]) {
#pragma unroll
  for (int block = 0; block < kLaneValues; block += 4 * S)
#pragma unroll
    for (int i = block; i < block + S; ++i) butterfly<S>(v, i);
}

// The codes of a lane's 64 values: `Bytes` bytes from p, in 16-byte loads
// where p allows, byte loads where it does not. Plain loads: a load
// instruction here reads 16 bytes of every lane's 64 or 32, a part of each
// line, and the non-temporal form measured 12-20% slower.
template <int Bytes, bool ALIGNED>
__device__ __forceinline__ void load_codes(const uint8_t* p, uint32_t (&w)[Bytes / 4]) {
  if constexpr (ALIGNED) {
#pragma unroll
    for (int k = 0; k < Bytes / 16; ++k) {
      const uint4 q = *reinterpret_cast<const uint4*>(p + 16 * k);
      w[4 * k] = q.x;
      w[4 * k + 1] = q.y;
      w[4 * k + 2] = q.z;
      w[4 * k + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < Bytes / 4; ++k)
      w[k] = (uint32_t)p[4 * k] | ((uint32_t)p[4 * k + 1] << 8) | ((uint32_t)p[4 * k + 2] << 16) |
             ((uint32_t)p[4 * k + 3] << 24);
  }
}

// A wave's int8 codes when its 16 groups lie back to back (no ids): 4 KiB
// from base in four loads of 1 KiB, lane j the j-th 16 bytes of each,
// non-temporal (read once), then through the wave's LDS into each lane's own
// 64 bytes. Every load instruction reads whole 128-byte lines, where a lane
// loading its own run reads a sixteenth of 32 lines (3.5-4% faster on a
// [13824, 5120] weight; the 4-bit codes, 2 KiB a wave, measured 2-12%
// slower so). `last` is the offset of the wave's last 16 bytes: the loads
// past the weight's end read it again. The four pieces of a lane are
// permuted among its slots so that the 16 lanes of a read phase cover all 64
// banks (and the 8 of a 32-bank phase, its 32), while a phase's writes stay
// 256 consecutive bytes.
__device__ __forceinline__ void staged_codes(const uint8_t* base, int64_t last, uint4* slots, int lane,
                                             uint32_t (&w)[16]) {
  const auto slot = [](int p) {
    const int l = p >> 2;
    return 4 * l + ((p & 3) ^ (((l >> 1) ^ (l >> 3)) & 3));
  };
  uint4 piece[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) piece[i] = stream_load(base + min((int64_t)(kWave * i + lane) * 16, last));
#pragma unroll
  for (int i = 0; i < 4; ++i) slots[slot(kWave * i + lane)] = piece[i];
  wave_sync();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint4 c = slots[slot(4 * lane + k)];
    w[4 * k] = c.x;
    w[4 * k + 1] = c.y;
    w[4 * k + 2] = c.z;
    w[4 * k + 3] = c.w;
  }
  wave_sync();  // the codes' reads are done before the trade writes over them
}

// 16 consecutive outputs as out holds them, into LDS: BF16 (32 bytes), or
// F32 holding the BF16 value (ops/CpuLinear.scala:24-29; 64 bytes).
__device__ __forceinline__ void stage_run(uint8_t* p, const float* v, uint16_t) {
  uint4* q = reinterpret_cast<uint4*>(p);
  q[0] = make_uint4(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7]));
  q[1] = make_uint4(pack_bf16(v[8], v[9]), pack_bf16(v[10], v[11]), pack_bf16(v[12], v[13]),
                    pack_bf16(v[14], v[15]));
}

__device__ __forceinline__ void stage_run(uint8_t* p, const float* v, float) {
  uint4* q = reinterpret_cast<uint4*>(p);
#pragma unroll
  for (int k = 0; k < 4; ++k)
    q[k] = make_uint4(bf16_bits(v[4 * k]) << 16, bf16_bits(v[4 * k + 1]) << 16, bf16_bits(v[4 * k + 2]) << 16,
                      bf16_bits(v[4 * k + 3]) << 16);
}

// A lane's 64 4-bit values from the words of its codes: lane l holds
// codebook[l % 16] in `entry`, and a value's entry comes from lane `code`
// (ds_bpermute, no LDS).
//
// ds_bpermute takes its lane from bits 7:2 of the address, and every lane
// holds the entry of its lane modulo 16, so the address need only have the
// code in bits 5:2: what lies above them (the next codes' bits) picks a lane
// holding the same entry, and no mask is needed (0.8% of the 4-bit decode).
__device__ __forceinline__ int nibble_address(const uint32_t (&w)[8], int j) {
  const int shift = 4 * (j % 8) - 2;  // the code times 4 in bits 5:2
  const uint32_t word = w[j / 8];
  return (int)(shift < 0 ? word << 2 : word >> shift);
}

__device__ __forceinline__ int nibble_code(const uint32_t (&w)[8], int j) {
  return (int)((w[j / 8] >> (4 * (j % 8))) & 0xfu);
}

__device__ __forceinline__ float codebook_times(const uint32_t (&w)[8], float entry, const float (&rel)[4], int j) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(nibble_address(w, j), __float_as_int(entry))) * rel[j / 16];
}

__device__ __forceinline__ void decode_nibbles(const uint32_t (&w)[8], float entry, const float (&rel)[4], float scale,
                                               float (&v)[kLaneValues]) {
#pragma unroll
  for (int j = 0; j < kLaneValues; ++j)
    v[j] = fminf(fmaxf(__builtin_rintf(codebook_times(w, entry, rel, j)), -127.0f), 127.0f) * scale;
}

// Where codebook * relative is NaN the level is NaN, which the clamp above
// dropped (Java's min and max keep it). That is where the entry is NaN, the
// relative scale is NaN, or an infinite entry meets a zero scale (E4M3 has
// no infinities): `bad[r]` has bit c set when code c is NaN with run r's
// scale. A wave with any such bit puts the NaNs back.
__device__ __forceinline__ void keep_nans(const uint32_t (&w)[8], const uint32_t (&bad)[4], float (&v)[kLaneValues]) {
#pragma unroll
  for (int j = 0; j < kLaneValues; ++j)
    if ((bad[j / 16] >> nibble_code(w, j)) & 1u) v[j] = __builtin_nanf("");
}

// A lane's 64 4-bit values by a table, where the relative scales cover 64
// columns or more: the lane's 64 values then share one relative scale and
// one row scale, so a value is the lane's own function of its code. The lane
// makes its 16 (the level as above, a NaN product kept as NaN, times the
// scale) once and reads each value's from the wave's LDS, at word code * 64 +
// lane: the 64 lanes of a read fall on distinct banks, and a lane reads only
// what it wrote. Per value an LDS read replaces the multiply, rounding, clamp
// and multiply; the NaN cases need no pass of their own.
__device__ __forceinline__ void decode_by_table(const uint32_t (&w)[8], const float* codebook, float rel, float scale,
                                                float* table, float (&v)[kLaneValues]) {
  const int lane = (int)threadIdx.x % kWave;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const float x = codebook[c] * rel;
    const float level = x != x ? x : fminf(fmaxf(__builtin_rintf(x), -127.0f), 127.0f);
    table[c * kWave + lane] = level * scale;
  }
#pragma unroll
  for (int j = 0; j < kLaneValues; ++j) v[j] = table[nibble_code(w, j) * kWave + lane];
}

// What decodes a rotated weight (ops/ConvRotParts.scala): scales F32, one a
// row or one for all; with a codebook, the 4-bit levels' codebook (F32
// [16]), relative scales (fp8 [rows, cols / group_size]) and group_size.
struct Parts {
  const uint8_t* codes;
  const float* scales;
  int64_t scale_count;
  const float* codebook;
  const uint8_t* relative;
  int group_size;
};

// Rows ids[t] (row t with no ids) of a rotated weight [rows, cols] into out
// [count, cols]; T float (the BF16 value widened, as the reference gathers)
// or uint16_t (BF16). An id outside [0, rows) gets zeros and sets *bad_id.
// TABLE (4-bit, relative scales a group of 64 columns or more): the values
// by decode_by_table. Registers held to five waves a SIMD (90-96 in place
// of 98-104): the 4-bit table decode of a [13824, 5120] weight 3% faster,
// the int8 even; the 4-bit permute decode stays free (held, it spills).
template <typename T, bool FOUR_BIT, bool ALIGNED, bool TABLE = false, bool STAGED = false>
__global__ void __launch_bounds__(kBlockWaves * kWave)
    __attribute__((amdgpu_waves_per_eu(FOUR_BIT && !TABLE ? 1 : 5)))
    rotated_rows(Parts parts, const int32_t* ids, T* out, int64_t count, int64_t rows, int cols, int32_t* bad_id) {
  static_assert(!TABLE || FOUR_BIT, "the table is the 4-bit codes'");
  static_assert(!STAGED || (ALIGNED && !FOUR_BIT), "staged codes are int8 on 16-byte boundaries");
  __shared__ float4 trade[kBlockWaves][kWaveGroups * 16];  // 4 KiB a wave
  const int lane = (int)threadIdx.x % kWave, wave = (int)threadIdx.x / kWave;
  const int g = lane >> 2, q = lane & 3;  // group in the wave, quarter in the group
  const int per_row = cols / kGroup;
  const int64_t groups = count * per_row;
  const int64_t wanted = ((int64_t)blockIdx.x * kBlockWaves + wave) * kWaveGroups + g;
  const bool live = wanted < groups;
  const int64_t group = live ? wanted : groups - 1;  // loads stay in bounds, stores are skipped
  const int64_t t = group / per_row;
  const int column = (int)(group - t * per_row) * kGroup;
  int64_t row = ids ? (int64_t)ids[t] : t;
  const bool bad = row < 0 || row >= rows;
  if (bad) row = 0;
  const int first = column + q * kLaneValues;  // this lane's first column

  float v[kLaneValues];
  const float scale = parts.scales[parts.scale_count == 1 ? 0 : row];
  const int64_t wave_first = ((int64_t)blockIdx.x * kBlockWaves + wave) * kWaveGroups;
  if constexpr (!FOUR_BIT) {
    // ops/CpuBase.scala:47-49: the code as float times the row's scale
    uint32_t w[16];
    if constexpr (STAGED)  // the wave's 16 groups back to back in codes
      staged_codes(parts.codes + wave_first * kGroup, (groups - wave_first) * kGroup - 16,
                   reinterpret_cast<uint4*>(trade[wave]), lane, w);
    else
      load_codes<64, ALIGNED>(parts.codes + row * cols + first, w);
#pragma unroll
    for (int j = 0; j < kLaneValues; ++j) v[j] = (float)(int8_t)(w[j / 4] >> (8 * (j % 4))) * scale;
  } else if constexpr (TABLE) {
    uint32_t w[8];
    load_codes<32, ALIGNED>(parts.codes + row * (cols / 2) + first / 2, w);
    const float rel = e4m3(parts.relative[row * (cols / parts.group_size) + first / parts.group_size]);
    decode_by_table(w, parts.codebook, rel, scale, reinterpret_cast<float*>(trade[wave]), v);
    wave_sync();  // the table's reads are done before the trade writes over it
  } else {
    // ops/CpuBase.scala:50-66: the low nibble the even column; level =
    // clamp(rint(codebook(code) * relative), -127, 127), a NaN kept (Java's
    // min and max), times the row's scale.
    const float entry = parts.codebook[lane & 15];
    uint32_t w[8];
    load_codes<32, ALIGNED>(parts.codes + row * (cols / 2) + first / 2, w);
    const int64_t rel_row = row * (cols / parts.group_size);
    uint32_t rel_code[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rel_code[r] = parts.relative[rel_row + (first + 16 * r) / parts.group_size];
    float rel[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rel[r] = e4m3(rel_code[r]);
    // codes whose entry is NaN, or infinite (lanes 0-15 hold the 16 entries)
    const uint32_t nan_codes = (uint32_t)__ballot(lane < 16 && entry != entry) & 0xffffu;
    const uint32_t inf_codes = (uint32_t)__ballot(lane < 16 && __builtin_isinf(entry)) & 0xffffu;
    uint32_t bad[4];
    bool any = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      bad[r] = rel[r] != rel[r] ? 0xffffu : nan_codes | (rel[r] == 0.0f ? inf_codes : 0u);
      any |= bad[r] != 0;
    }
    decode_nibbles(w, entry, rel, scale, v);
    if (__any(any)) keep_nans(w, bad, v);
  }

  // digits 0, 1, 2 (strides 1, 4, 16) in registers
  round_of<1>(v);
  round_of<4>(v);
  round_of<16>(v);

  // Trade within the quad, a value of digit 1 at a time: lane q writes its
  // four runs of digit 2 (4 values of digit 0 each) and reads back, from the
  // quad's four lanes (digit 3), the runs of digit 2 = q, into the registers
  // it wrote from. After it, v[16 * d3 + 4 * d1 + d0] is the value of digits
  // (d0, d1, q, d3). Slot of (g, d3, d2) in the wave's 256: (g / 4) * 64 +
  // d2 * 16 + 4 * ((d3 + d2) % 4) + g % 4, so the 16 lanes of a phase write,
  // and read, 16 different slots.
  float4* slots = trade[wave] + (g >> 2) * 64 + (g & 3);
#pragma unroll
  for (int d1 = 0; d1 < 4; ++d1) {
#pragma unroll
    for (int d2 = 0; d2 < 4; ++d2) {
      const int at = 16 * d2 + 4 * d1;
      slots[d2 * 16 + 4 * ((q + d2) & 3)] = make_float4(v[at], v[at + 1], v[at + 2], v[at + 3]);
    }
    wave_sync();
#pragma unroll
    for (int d3 = 0; d3 < 4; ++d3) {
      const float4 r = slots[q * 16 + 4 * ((d3 + q) & 3)];
      const int at = 16 * d3 + 4 * d1;
      v[at] = r.x;
      v[at + 1] = r.y;
      v[at + 2] = r.z;
      v[at + 3] = r.w;
    }
    wave_sync();  // every lane's reads are done before the next writes
  }

  // digit 3 (stride 64 in the group, 16 here)
  round_of<16>(v);

  if (bad) {
#pragma unroll
    for (int j = 0; j < kLaneValues; ++j) v[j] = 0.0f;
    if (bad_id && live) *bad_id = 1;
  }

  // Out through the wave's LDS, a part at a time (4 KiB: a quarter or half
  // of each of its 16 groups): the lanes write their runs of the part, then
  // read it back so that each store instruction's 64 lanes write 16
  // consecutive 16-byte pieces of four groups, whole 128-byte lines. The
  // wave's groups are consecutive in out.
  constexpr int kRunsPerPart = 256 / (4 * 16 * (int)sizeof(T));  // a lane's digit-3 runs in a part: 2 BF16, 1 F32
  static_assert(kRunsPerPart >= 1 && 4 % kRunsPerPart == 0, "a part is whole runs");
  uint8_t* part = reinterpret_cast<uint8_t*>(trade[wave]);
#pragma unroll
  for (int first3 = 0; first3 < 4; first3 += kRunsPerPart) {
#pragma unroll
    for (int r = 0; r < kRunsPerPart; ++r)
      stage_run(part + g * 256 + (r * 64 + q * 16) * (int)sizeof(T), v + 16 * (first3 + r), T{});
    wave_sync();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int piece = lane + 64 * i;  // 16-byte piece of the part
      const int pg = piece / 16;        // its group in the wave
      const uint4 w = reinterpret_cast<const uint4*>(part)[piece];
      if (wave_first + pg < groups) {
        T* at = out + (wave_first + pg) * kGroup + first3 * 64 + (piece % 16) * (16 / (int)sizeof(T));
        __builtin_nontemporal_store(u32x4{w.x, w.y, w.z, w.w}, reinterpret_cast<u32x4*>(at));
      }
    }
    wave_sync();  // the part's reads are done before the next part's writes
  }
}

// ---------------------------------------------------------------- launch layer

// rotated_rows for the codes' alignment and layout: staged (int8, aligned,
// no ids), 16-byte loads a lane (aligned), or byte loads.
template <typename T, bool FOUR_BIT, bool TABLE>
void launch_rows(bool aligned, bool staged, dim3 grid, hipStream_t s, const Parts& parts, const int32_t* ids, T* out,
                 int64_t count, int64_t rows, int32_t cols, int32_t* bad_id) {
  const dim3 block(kBlockWaves * kWave);
  if constexpr (!FOUR_BIT) {
    if (staged) {
      hipLaunchKernelGGL((rotated_rows<T, false, true, false, true>), grid, block, 0, s, parts, ids, out, count, rows,
                         cols, bad_id);
      return;
    }
  }
  if (aligned)
    hipLaunchKernelGGL((rotated_rows<T, FOUR_BIT, true, TABLE>), grid, block, 0, s, parts, ids, out, count, rows,
                       cols, bad_id);
  else
    hipLaunchKernelGGL((rotated_rows<T, FOUR_BIT, false, TABLE>), grid, block, 0, s, parts, ids, out, count, rows,
                       cols, bad_id);
}

// Ops.checkRotated (ops/LinearOps.scala:121-157) on the raw arguments, then
// the launch: a wave per 16 groups of 256 values, one pass.
template <typename T>
int rotated_launch(const char* entry, const Parts& parts, const int32_t* ids, T* out, int64_t count, int64_t rows,
                   int32_t cols, int32_t* bad_id, void* stream) {
  clear_error();
  const bool four_bit = parts.codebook != nullptr;
  if (count < 0 || rows < 0) return refuse("%s: %lld rows of %lld", entry, (long long)count, (long long)rows);
  if (cols <= 0 || cols % kGroup != 0) return refuse("%s: rows of %d columns", entry, cols);
  if (!(parts.scale_count == rows || (parts.scale_count == 1 && !four_bit)))
    return refuse("%s: %lld scales for %lld rows", entry, (long long)parts.scale_count, (long long)rows);
  if (four_bit && (parts.group_size <= 0 || parts.group_size % 16 != 0 || cols % parts.group_size != 0))
    return refuse("%s: %d columns in groups of %d", entry, cols, parts.group_size);
  if (count == 0) return 0;
  // an id outside the weight reads row 0 (and writes zeros): there must be one
  if (rows == 0) return refuse("%s: %lld rows of an empty weight", entry, (long long)count);
  if (!parts.codes || !parts.scales || !out || (four_bit && !parts.relative))
    return refuse("%s: null codes, scales, relative scales or out", entry);
  if (!aligned16(out)) return refuse("%s: out is not 16-byte aligned", entry);
  if (reinterpret_cast<uintptr_t>(parts.scales) % 4 != 0 || reinterpret_cast<uintptr_t>(parts.codebook) % 4 != 0)
    return refuse("%s: scales or codebook not 4-byte aligned", entry);
  const int64_t groups = count * (cols / kGroup);
  const int64_t waves = (groups + kWaveGroups - 1) / kWaveGroups;
  const int64_t blocks = (waves + kBlockWaves - 1) / kBlockWaves;
  if (blocks > kOneShotBlocks) return refuse("%s: %lld groups is too many for one launch", entry, (long long)groups);
  // 16-byte code loads need every lane's run (64 B, or 32 B of nibbles) on a
  // 16-byte boundary: the weight's start, and its rows (cols is a multiple of
  // 256, so they are).
  const bool aligned = aligned16(parts.codes);
  // Without ids a wave's 16 groups lie back to back and it loads them whole.
  const bool staged = aligned && !ids && !four_bit;
  const hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks);
  if (four_bit && parts.group_size % 64 == 0)
    launch_rows<T, true, true>(aligned, staged, grid, st, parts, ids, out, count, rows, cols, bad_id);
  else if (four_bit)
    launch_rows<T, true, false>(aligned, staged, grid, st, parts, ids, out, count, rows, cols, bad_id);
  else
    launch_rows<T, false, false>(aligned, staged, grid, st, parts, ids, out, count, rows, cols, bad_id);
  return launched(entry);
}

}  // namespace
}  // namespace drift

using namespace drift;

extern "C" int drift_rotated_embedding_f32(const void* codes, const float* scales, int64_t scale_count,
                                           const float* codebook, const uint8_t* relative, int32_t group_size,
                                           const int32_t* ids, float* out, int64_t count, int64_t rows, int32_t cols,
                                           int32_t* bad_id, void* stream) {
  if (!ids && count > 0) {
    clear_error();
    return refuse("drift_rotated_embedding_f32: null ids");
  }
  const Parts parts{static_cast<const uint8_t*>(codes), scales, scale_count, codebook, relative, group_size};
  return rotated_launch<float>("drift_rotated_embedding_f32", parts, ids, out, count, rows, cols, bad_id, stream);
}

extern "C" int drift_rotated_embedding_bf16(const void* codes, const float* scales, int64_t scale_count,
                                            const float* codebook, const uint8_t* relative, int32_t group_size,
                                            const int32_t* ids, uint16_t* out, int64_t count, int64_t rows,
                                            int32_t cols, int32_t* bad_id, void* stream) {
  if (!ids && count > 0) {
    clear_error();
    return refuse("drift_rotated_embedding_bf16: null ids");
  }
  const Parts parts{static_cast<const uint8_t*>(codes), scales, scale_count, codebook, relative, group_size};
  return rotated_launch<uint16_t>("drift_rotated_embedding_bf16", parts, ids, out, count, rows, cols, bad_id, stream);
}

extern "C" int drift_rotated_dequantize_bf16(const void* codes, const float* scales, int64_t scale_count,
                                             const float* codebook, const uint8_t* relative, int32_t group_size,
                                             uint16_t* out, int64_t rows, int32_t cols, void* stream) {
  const Parts parts{static_cast<const uint8_t*>(codes), scales, scale_count, codebook, relative, group_size};
  return rotated_launch<uint16_t>("drift_rotated_dequantize_bf16", parts, nullptr, out, rows, rows, cols, nullptr,
                                  stream);
}
