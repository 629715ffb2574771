// Attention inputs for gfx950: per-head query/key RMSNorm fused with rope,
// the same with a gated query's split and the keys' and values' write into
// the runner's paged F16 KV cache (attention_inputs), the cache write alone,
// and the split of a row's halves.
//
// Layouts: queries and keys [tokens, heads, head_dim] row-major (a gated
// query projection [tokens, heads, 2 head_dim]: the query, then its output
// gate). The cache (ops/KvCache.scala:5-22): keys F16 [pages, page_size,
// kv_heads, head_dim], values F16 [pages, kv_heads, head_dim, page_size]
// (transposed within a page); a sequence's page table (int32) maps
// position / page_size to a page.
//
// Arithmetic is the CPU reference's: the norm in double rounded once to F32
// (rmsNorm writes F32), the rope of those F32 values (ops/CpuAttention.scala:
// 89-146, as rope.hpp), and F32 -> F16 rounding to nearest even for the
// cache (Float.floatToFloat16 in ops/CpuAttention.scala:181-210).
#include "rope.hpp"
#include "sincos.hpp"

#include <algorithm>
#include <climits>

namespace drift {
namespace {

// ------------------------------------------------------------------ per-head RMSNorm + rope

struct QkArgs {
  RopeArgs rope;
  int32_t q_heads, kv_heads;
  float eps, offset;
  int64_t q_stride;  // values from one query head's row to the next: head_dim, or 2 head_dim with a gate
};

// What attention_inputs writes beyond the rotated queries: the gate half of
// each query head's row (when `gate` is set) and, when `keys` is set, the
// rotated keys and the values `v` into the paged cache instead of k_out.
template <typename T>
struct Extras {
  T* gate;
  const T* v;
  uint16_t* keys;    // F16 [pages, page_size, kv_heads, head_dim]
  uint16_t* values;  // F16 [pages, kv_heads, head_dim, page_size]
  const int32_t* page_table;
  int32_t pages, page_size, start;
  int32_t* bad_page;
  int64_t tiles;  // value tiles the launch's extra blocks write (0: the token blocks write the values)
};

// Token t's place in the cache for key head kv: keys[key + d] and
// values[value + d * page_size] (ops/CpuAttention.scala:163-179). False
// when the page table names a page outside the cache: then nothing is
// written and *bad_page is set.
template <typename T>
__device__ __forceinline__ bool cache_place(const Extras<T>& e, int64_t t, int kv_heads, int dim, int kv,
                                            int64_t& key, int64_t& value) {
  const int64_t position = e.start + t;
  const int64_t page = e.page_table[position / e.page_size];
  const int64_t offset = position % e.page_size;
  if (page < 0 || page >= e.pages) {
    if (e.bad_page) *e.bad_page = 1;
    return false;
  }
  key = ((page * e.page_size + offset) * kv_heads + kv) * dim;
  value = (page * kv_heads + kv) * (int64_t)dim * e.page_size + offset;
  return true;
}

// The key row alone, the token's page and its place in the page already
// known (as cache_place, without the division).
template <typename T>
__device__ __forceinline__ bool key_place(const Extras<T>& e, int32_t page, uint32_t in_page, int kv_heads, int dim,
                                          int kv, int64_t& key) {
  if (page < 0 || page >= e.pages) {
    if (e.bad_page) *e.bad_page = 1;
    return false;
  }
  key = (((int64_t)page * e.page_size + in_page) * kv_heads + kv) * dim;
  return true;
}

// F32 -> F16 bits, to nearest even (v_cvt_f16_f32): Float.floatToFloat16's
// rounding; NaN payloads are the hardware's.
__device__ __forceinline__ uint32_t f16_bits(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }

// N consecutive values as F16, one 8- or 16-byte store.
template <int N>
__device__ __forceinline__ void store_f16(uint16_t* p, const float (&v)[N]) {
  uint32_t w[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i) w[i] = f16_bits(v[2 * i]) | (f16_bits(v[2 * i + 1]) << 16);
  // non-temporal, as the other streamed outputs (plain stores measured slower)
  if constexpr (N == 8)
    __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]}, reinterpret_cast<u32x4*>(p));
  else
    __builtin_nontemporal_store(w[0] | ((uint64_t)w[1] << 32), reinterpret_cast<uint64_t*>(p));
}

// Any head size: each wave norms one head row at a time into LDS (the F32
// values rmsNorm writes), then turns its pairs from there. With EXTRAS, the
// gate half of a query row is copied out, and a key head's turned row and
// its values go to the cache as F16.
template <typename T, bool EXTRAS>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(const T* q, const T* k, T* q_out, T* k_out,
                                                           const float* q_weight, const float* k_weight,
                                                           const int32_t* positions, QkArgs a, Extras<T> e) {
  __shared__ double2 cs[kMaxPairs];
  __shared__ float normed[4][2 * kMaxPairs];
  const RopeArgs& p = a.rope;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = a.q_heads + a.kv_heads;
  const int slots = (p.dim + 1) / 2;
  for (int64_t t = blockIdx.x; t < p.tokens; t += gridDim.x) {
    token_angles(p, positions, t, cs);
    for (int round = 0; round < rows; round += 4) {
      const int h = round + wave;
      const bool query = h < a.q_heads;
      const int kv = h - a.q_heads;
      const T* xh = query ? q + (t * a.q_heads + h) * a.q_stride : k + (t * a.kv_heads + kv) * p.dim;
      const float* w = query ? q_weight : k_weight;
      if (h < rows) {
        float v[2 * kMaxPairs / kWave];
        double squares = 0.0;
#pragma unroll
        for (int i = 0; i < 2 * kMaxPairs / kWave; ++i) {
          const int d = i * kWave + lane;
          v[i] = d < p.dim ? load_one(xh + d) : 0.0f;
          squares = fma((double)v[i], (double)v[i], squares);
        }
        if (EXTRAS && query && e.gate)
          for (int d = lane; d < p.dim; d += kWave)
            store_one(e.gate + (t * a.q_heads + h) * p.dim + d, load_one(xh + p.dim + d));
        const double factor = 1.0 / sqrt(group_sum<64>(squares) / (double)p.dim + (double)a.eps);
#pragma unroll
        for (int i = 0; i < 2 * kMaxPairs / kWave; ++i) {
          const int d = i * kWave + lane;
          if (d < p.dim) normed[wave][d] = (float)((double)v[i] * factor * ((double)w[d] + (double)a.offset));
        }
      }
      __syncthreads();  // normed rows and (first round) cs are ready
      if (h < rows) {
        auto load = [&](int d) { return (double)normed[wave][d]; };
        if (!EXTRAS || query || !e.keys) {
          T* oh = query ? q_out + (t * a.q_heads + h) * p.dim : k_out + (t * a.kv_heads + kv) * p.dim;
          for (int j = lane; j < slots; j += kWave) turn_slot<T>(j, p.dim, p.rotary, p.layout, cs, load, oh);
        } else {
          int64_t key, value;
          if (cache_place(e, t, a.kv_heads, p.dim, kv, key, value)) {
            for (int j = lane; j < slots; j += kWave)
              turn_slot(j, p.dim, p.rotary, p.layout, cs, load,
                        [&](int d, float r) { e.keys[key + d] = (uint16_t)f16_bits(r); });
            const T* vh = e.v + (t * a.kv_heads + kv) * p.dim;
            for (int d = lane; d < p.dim; d += kWave)
              e.values[value + (int64_t)d * e.page_size] = (uint16_t)f16_bits(load_one(vh + d));
          }
        }
      }
      __syncthreads();  // normed is reused next round, cs next token
    }
  }
}

// The fast path for whole-chunk heads with every value turning: one wave per
// (token, group of 64 / G heads), each in a one-wave block, G lanes per head,
// each lane holding two chunks of its head (NeoX: a chunk and its partner;
// otherwise chunks i and i + G). The waves are independent: no block barrier.
// A wave issues its loads first; while they land it makes its token's cos and
// sin (a pair a lane, the double sin and cos of sincos.hpp) in its own LDS.
// Heads with mRoPE sections (a position per section) take the general kernel.
//
// Measured on MI355X at Q [4096,32,128], K [4096,8,128] bf16 (kernel-trace
// medians), against the designs it replaced: a block of five waves per token
// sharing the angles through a barrier 17.5 us, a wave per token (all 40
// heads) 19.3 us, two tokens a wave 17.5 us, 16 lanes a head (one chunk a
// lane, partners by DPP) 21.5 us; this one 16.0 us, at 64 registers (eight
// waves a SIMD). One-wave blocks stream faster than larger ones at this size:
// a plain copy of the same bytes takes 14.3 us in one-wave blocks and 15.5 us
// in 256-thread blocks.
//
// The angles' LDS is laid out so the G lanes of a head read consecutive
// entries: for NeoX the pair of lane i0's value i sits at i * G + i0 (the
// natural index would put the G lanes N entries apart, on the same banks).
template <bool NEOX, int G, int N>
__device__ __forceinline__ int qk_pair_slot(int pair) {
  if constexpr (NEOX) return (pair % N) * G + pair / N;
  return pair;
}

// Values into the cache by tiles, one tile a one-wave block: a tile is 16
// consecutive positions of one page (16 divides the page size) for H key
// heads. In the value layout ([page][head][value][position]) a whole tile of
// a 16-token page is one contiguous run, 32 bytes per value.
//
// Lane l takes position l % 16 of chunks (l / 16) + 4 r: each load covers 64
// bytes of 16 positions. The chunk's values go to F16; lanes 2i and 2i + 1
// (positions p, p + 1) trade them by DPP, so that each LDS write is one dword
// holding positions p and p + 1 of one value, the even lane writing the
// chunk's first half of values, the odd lane the second. A row (value) of
// the staged tile is 8 dwords, and every 8 rows are followed by 8 dwords of
// padding: then the 64 lanes of a write land on 64 distinct banks. The tile
// leaves as 16-byte stores, 8 positions of one value each. A tile that
// positions outside the tokens cut (the sequence's first or last page) is
// written value by value instead; a tile of a page outside the cache writes
// nothing and sets *bad_page.
//
// Key heads per value tile: as many as keep the staged tile within 4 KiB of
// values (one head of 128).
constexpr int kTileHeads(int dim) { return dim * 32 >= 4096 ? 1 : 4096 / (dim * 32); }

__device__ __forceinline__ int tile_dword(int value, int position) { return value * 8 + (value / 8) * 8 + position / 2; }

// LDS words the staged tile takes
constexpr int kTileWords(int dim) { return kTileHeads(dim) * dim * 9; }

template <typename T, int DIM, int H = kTileHeads(DIM)>
__device__ __forceinline__ void cache_values_tile(const Extras<T>& e, int64_t tokens, int kv_heads, int64_t tile,
                                                  uint32_t* staged) {
  constexpr int N = Chunk<T>::N;
  constexpr int kTile = 16;
  constexpr int kRows = H * DIM;
  constexpr int kChunks = kTile * kRows / N;
  const int lane = threadIdx.x;
  const int head_blocks = (kv_heads + H - 1) / H;
  const int kv0 = (int)(tile % head_blocks) * H;
  const int heads = min(H, kv_heads - kv0);
  const int64_t first = (e.start / kTile + tile / head_blocks) * kTile;  // the tile's first position
  const int64_t lo = max(first, (int64_t)e.start), hi = min(first + kTile, e.start + tokens);
  const int64_t page = e.page_table[first / e.page_size];
  const int p = lane % kTile;
  const bool odd = p & 1;
  // positions the tokens do not cover, and heads past the last, are clamped
  // to ones they do (loads are never branched around)
  const int64_t position = min(max(first + p, lo), hi - 1);
  const T* row = e.v + (position - e.start) * kv_heads * DIM;
  for (int base = 0; base < kChunks; base += 4 * kWave) {
    typename Chunk<T>::Raw raw[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rest = min((base + r * kWave + lane) / kTile, kChunks / kTile - 1);  // (head, chunk) of the tile
      const int hh = min(rest / (DIM / N), heads - 1), q = rest % (DIM / N);
      raw[r] = Chunk<T>::load_raw(row + (kv0 + hh) * DIM + q * N);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rest = (base + r * kWave + lane) / kTile;
      if (base + r * kWave >= kChunks) break;
      float v[N];
      Chunk<T>::unpack(raw[r], v);
      uint32_t own[N / 2], other[N / 2];
#pragma unroll
      for (int j = 0; j < N / 2; ++j) {
        own[j] = f16_bits(v[2 * j]) | (f16_bits(v[2 * j + 1]) << 16);
        other[j] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)own[j], 0xb1, 0xf, 0xf, true);  // lane ^ 1
      }
      // the even lane writes values 0 .. N/2 - 1 of the chunk, the odd lane
      // the rest, each dword (position p, p + 1) of one value
#pragma unroll
      for (int j = 0; j < N / 2; ++j) {
        const int w = odd ? N / 4 + j / 2 : j / 2;  // the word holding value (odd ? N/2 : 0) + j
        const bool high = j & 1;
        const uint32_t mine = high ? own[w] >> 16 : own[w] & 0xffffu;
        const uint32_t theirs = high ? other[w] >> 16 : other[w] & 0xffffu;
        const uint32_t word = odd ? theirs | (mine << 16) : mine | (theirs << 16);
        staged[tile_dword(rest * N + (odd ? N / 2 : 0) + j, p)] = word;
      }
    }
  }
  wave_sync();
  if (page < 0 || page >= e.pages) {
    if (e.bad_page && lane == 0) *e.bad_page = 1;
    return;
  }
  // rows (head, value) of the tile: kv0's row 0, then on, page_size apart
  uint16_t* row0 = e.values + (page * kv_heads + kv0) * (int64_t)DIM * e.page_size + first % e.page_size;
  if (lo == first && hi == first + kTile) {
    for (int c = lane; c < heads * DIM * 2; c += kWave) {
      const int value = c / 2, half = c % 2;
      const uint4 w = *reinterpret_cast<const uint4*>(&staged[tile_dword(value, half * 8)]);
      __builtin_nontemporal_store(u32x4{w.x, w.y, w.z, w.w},
                                  reinterpret_cast<u32x4*>(row0 + (int64_t)value * e.page_size + half * 8));
    }
  } else {
    const uint16_t* halves = reinterpret_cast<const uint16_t*>(staged);
    for (int c = lane; c < heads * DIM * kTile; c += kWave) {
      const int value = c / kTile, i = c % kTile;
      if (first + i >= lo && first + i < hi)
        row0[(int64_t)value * e.page_size + i] = halves[2 * tile_dword(value, i) + (i & 1)];
    }
  }
}

// cos and sin of an angle of 2^20 or more by the library, out of line: its
// registers are not the kernel's while the heads and weights wait in theirs
__device__ __attribute__((noinline)) double2 sincos_far(float angle) {
  double sn, cn;
  sincos((double)angle, &sn, &cn);
  return make_double2(cn, sn);
}

// FAST: every wave's heads are all queries or all keys (so the choice of
// tensor, and its addresses' base, is the wave's, not each lane's) and the
// weight offset is 0 (the identity addition is left out: the two forms of
// the weight multiply in one kernel cost 20 registers, and waves).
// P = 2 (FAST, no cache): the wave takes two groups of 64 / G heads of its
// token, one after the other, both loaded first; the angles, the weights
// (widened once) and the wave's set-up serve both. Measured at the C3 shape:
// 2% faster than one group a wave, at 95 registers against 64; a pass loop
// loading one group ahead was 5% slower, four groups a wave 30% slower, and
// with the cache two groups were slower than one.
template <typename T, int G, bool NEOX, bool EXTRAS, bool GATE, bool FAST, int P>
__device__ __forceinline__ void qk_wave_heads(const T* q, const T* k, T* q_out, T* k_out, const float* q_weight,
                                              const float* k_weight, const int32_t* positions, const QkArgs& a,
                                              const Extras<T>& e, int64_t t, int group, double2* cs) {
  static_assert(P == 1 || (P == 2 && FAST && !EXTRAS), "two groups a wave: the fast body, no cache");
  constexpr int N = Chunk<T>::N;
  using Raw = typename Chunk<T>::Raw;
  constexpr int kHeadsPerPass = kWave / G;
  constexpr int dim = 2 * N * G, half = N * G;  // a head's pairs: half (rotary == dim)
  const RopeArgs& p = a.rope;
  const int lane = threadIdx.x;
  const int rows = a.q_heads + a.kv_heads;
  const int i0 = lane % G;
  const int d0 = i0 * N, d1 = (NEOX ? half : G * N) + i0 * N;
  const int first = group * kHeadsPerPass * P;  // the wave's first head
  const int h = first + lane / G;
  const bool live = h < rows;
  const bool query = FAST ? first < a.q_heads : h < a.q_heads;
  // the small operands load first (the token's position, the pairs'
  // frequencies, the lane's norm weights), then the heads: loads complete in
  // order, so waiting for the small ones never waits for the heads, and the
  // angles are made while the heads land. A head past the last is clamped to
  // it (loads are never branched around). Measured at the C3 shape, against
  // weights staged as doubles in LDS, a position read per lane and a branch
  // for irregular sums: each of those cost about 1 us.
  constexpr int kPairsPerLane = (half + kWave - 1) / kWave;
  const int32_t position = positions[t];  // single-section rope: one position a token
  float inverse[kPairsPerLane];
#pragma unroll
  for (int u = 0; u < kPairsPerLane; ++u) inverse[u] = p.inverse[min(lane + u * kWave, half - 1)];
  const int hc = min(h, rows - 1);
  const bool query_c = FAST ? query : hc < a.q_heads;
  const float* ws = query_c ? q_weight : k_weight;
  float w0[N], w1[N];
#pragma unroll
  for (int i = 0; i < N; i += 4) {
    const float4 x0 = *reinterpret_cast<const float4*>(ws + d0 + i), x1 = *reinterpret_cast<const float4*>(ws + d1 + i);
    w0[i] = x0.x, w0[i + 1] = x0.y, w0[i + 2] = x0.z, w0[i + 3] = x0.w;
    w1[i] = x1.x, w1[i + 1] = x1.y, w1[i + 2] = x1.z, w1[i + 3] = x1.w;
  }
  const T* xh = query_c ? q + (t * a.q_heads + hc) * a.q_stride : k + (t * a.kv_heads + (hc - a.q_heads)) * dim;
  const Raw r0 = Chunk<T>::load_raw(xh + d0);
  const Raw r1 = Chunk<T>::load_raw(xh + d1);
  // the second group's heads (P = 2; FAST: the same tensor as the first's)
  Raw s0, s1;
  if constexpr (P == 2) {
    const int hc2 = min(h + kHeadsPerPass, rows - 1);
    const T* xh2 = query ? q + (t * a.q_heads + hc2) * a.q_stride : k + (t * a.kv_heads + (hc2 - a.q_heads)) * dim;
    s0 = Chunk<T>::load_raw(xh2 + d0);
    s1 = Chunk<T>::load_raw(xh2 + d1);
  }
  // the gate half of a query head's row (key heads clamped to the last query head)
  Raw g0, g1;
  if constexpr (GATE) {
    if (a.q_heads > 0) {
      const T* gh = q + (t * a.q_heads + min(hc, a.q_heads - 1)) * a.q_stride + dim;
      g0 = Chunk<T>::load_raw(gh + d0);
      g1 = Chunk<T>::load_raw(gh + d1);
    }
  }
  // with the cache, a key wave's page and the token's place in it, divided
  // and read once the heads' loads are issued and before the turn, where the
  // keys' stores would wait for them (cache positions are below 2^32: start
  // and the tokens are int32 and not negative, so the quotient is 32-bit)
  int32_t page = 0;  // widened only where the keys' stores use it, so nothing waits for it before
  uint32_t in_page = 0;
  if constexpr (EXTRAS) {
    if (e.keys && (!FAST || !query)) {
      const uint32_t cached = (uint32_t)e.start + (uint32_t)t;
      const uint32_t slot = cached / (uint32_t)e.page_size;
      in_page = cached - slot * (uint32_t)e.page_size;
      page = e.page_table[slot];
    }
  }
  // the token's cos and sin, a pair a lane, into the wave's LDS
#pragma unroll
  for (int u = 0; u < kPairsPerLane; ++u) {
    const int j = lane + u * kWave;
    if (j < half) {
      const float angle = (float)position * inverse[u];
      double sn, cn;
      if (!sincos_reduced(angle, &sn, &cn)) {
        const double2 far = sincos_far(angle);
        cn = far.x;
        sn = far.y;
      }
      cs[qk_pair_slot<NEOX, G, N>(j)] = make_double2(cn, sn);
    }
  }
  wave_sync();
  // a lane past the last head is past it in the second group too
  if (!live) return;
  // one group's heads: norm, turn and store
  auto turn_heads = [&](const Raw& x0, const Raw& x1, int hh) {
    float v0[N], v1[N];
    Chunk<T>::unpack(x0, v0);
    Chunk<T>::unpack(x1, v1);
    double squares = 0.0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      squares = fma((double)v0[i], (double)v0[i], squares);
      squares = fma((double)v1[i], (double)v1[i], squares);
    }
    squares = group_sum<G>(squares);
    // a positive epsilon (every caller's) keeps the mean above 2^-1000: the
    // branch is the wave's, on a kernel argument
    const double mean = squares / (double)dim + (double)a.eps;
    const double factor = a.eps > 0.0f ? inverse_sqrt<true>(mean) : inverse_sqrt(mean);
    // (double) weight + offset, as the reference adds them
    if constexpr (FAST) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        v0[i] = (float)((double)v0[i] * factor * (double)w0[i]);
        v1[i] = (float)((double)v1[i] * factor * (double)w1[i]);
      }
    } else {
      const double offset = (double)a.offset;
#pragma unroll
      for (int i = 0; i < N; ++i) {
        v0[i] = (float)((double)v0[i] * factor * ((double)w0[i] + offset));
        v1[i] = (float)((double)v1[i] * factor * ((double)w1[i] + offset));
      }
    }
    if constexpr (NEOX) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const double2 c = cs[qk_pair_slot<NEOX, G, N>(d0 + i)];
        turn_fused(v0[i], v1[i], c.x, c.y, v0[i], v1[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; i += 2) {
        const double2 c0 = cs[(d0 + i) / 2], c1 = cs[(d1 + i) / 2];
        turn_fused(v0[i], v0[i + 1], c0.x, c0.y, v0[i], v0[i + 1]);
        turn_fused(v1[i], v1[i + 1], c1.x, c1.y, v1[i], v1[i + 1]);
      }
    }
    if (!EXTRAS || query || !e.keys) {
      T* oh = query ? q_out + (t * a.q_heads + hh) * dim : k_out + (t * a.kv_heads + (hh - a.q_heads)) * dim;
      Chunk<T>::store(oh + d0, v0);
      Chunk<T>::store(oh + d1, v1);
    }
    if constexpr (EXTRAS) {
      if (GATE && query) {
        T* gh = e.gate + (t * a.q_heads + hh) * dim;
        *reinterpret_cast<uint4*>(gh + d0) = g0;
        *reinterpret_cast<uint4*>(gh + d1) = g1;
      }
      int64_t key;
      if (!query && e.keys && key_place(e, page, in_page, a.kv_heads, dim, hh - a.q_heads, key)) {
        store_f16<N>(e.keys + key + d0, v0);
        store_f16<N>(e.keys + key + d1, v1);
      }
    }
  };
  turn_heads(r0, r1, h);
  if constexpr (P == 2) {
    // the second group past the last head: the wave's (a uniform branch), or
    // this lane's
    if (first + kHeadsPerPass >= rows || h + kHeadsPerPass >= rows) return;
    // the first group's registers free before the second's are used
    __builtin_amdgcn_sched_barrier(0);
    turn_heads(s0, s1, h + kHeadsPerPass);
  }
}

template <typename T, int G, bool NEOX, bool EXTRAS, bool GATE, bool FAST, int P>
__global__ void __launch_bounds__(kWave) qk_norm_rope_wave(const T* q, const T* k, T* q_out, T* k_out,
                                                          const float* q_weight, const float* k_weight,
                                                          const int32_t* positions, QkArgs a, Extras<T> e,
                                                          int waves_per_token, int query_waves, bool keys_first) {
  constexpr int N = Chunk<T>::N;
  constexpr int dim = 2 * N * G;
  const RopeArgs& p = a.rope;
  // one LDS buffer for the token's angles or, in a tile block, the staged
  // tile (a block uses one of them; two buffers would hold fewer blocks)
  constexpr int kAngleWords = N * G * 4;  // double2 per pair
  constexpr int kWords = EXTRAS && kTileWords(dim) > kAngleWords ? kTileWords(dim) : kAngleWords;
  __shared__ __align__(16) uint32_t lds[kWords];
  int64_t item = blockIdx.x;
  if constexpr (EXTRAS) {
    // with the cache, the first e.tiles blocks write the values by tiles.
    // Measured at the C3 shape with the cache (4,096 tokens, 2,048 tiles):
    // tiles first 20.6 us, interleaved evenly 21.8 us, last 21.6 us.
    if (item < e.tiles) {
      cache_values_tile<T, dim>(e, p.tokens, a.kv_heads, item, lds);
      return;
    }
    item -= e.tiles;
  }
  // the grid's waves in two runs, the heavier first, so that the launch ends
  // on its shortest waves: every token's query waves (its first query_waves
  // groups), then its key waves, or with keys_first the other way round.
  // Without the cache C3's key wave takes 8 heads and a query wave 16, so the
  // keys go last (QK 16.05-16.15 -> 15.72-15.80 us; keys first 16.48-16.54);
  // with it a key wave also places and writes the cache, and goes first
  // (19.45-19.61 against 19.78-19.90 token by token). Blocks number fewer
  // than 2^31 (the launcher checks): 32-bit division.
  const uint32_t tokens = (uint32_t)p.tokens, qw = (uint32_t)query_waves;
  const uint32_t kw = (uint32_t)waves_per_token - qw;  // 0: token by token (qw is every wave)
  const uint32_t first_run = tokens * (keys_first ? kw : qw), first_waves = keys_first ? kw : qw;
  uint32_t token, group_u;
  if ((uint32_t)item < first_run) {
    token = (uint32_t)item / first_waves;
    group_u = (uint32_t)item - token * first_waves + (keys_first ? qw : 0);
  } else {
    const uint32_t rest = (uint32_t)item - first_run, waves = keys_first ? qw : kw;
    token = rest / waves;
    group_u = rest - token * waves + (keys_first ? 0 : qw);
  }
  const int64_t t = token;
  const int group = (int)group_u;
  qk_wave_heads<T, G, NEOX, EXTRAS, GATE, FAST, P>(q, k, q_out, k_out, q_weight, k_weight, positions, a, e, t, group,
                                                reinterpret_cast<double2*>(lds));
}

// ------------------------------------------------------------------ cache write, split halves

// Keys and values [tokens, kv_heads, dim] into the cache at positions start
// .. start + tokens - 1 (kernels/attention.hip:480-493): a thread per chunk of
// N values of a head, its key chunk one F16 store, its values N stores a
// page apart (the value layout is transposed within a page).
template <typename T>
__global__ void __launch_bounds__(256) cache_write_chunks(const T* k, Extras<T> e, int64_t tokens, int kv_heads,
                                                          int dim) {
  constexpr int N = Chunk<T>::N;
  const int per_head = dim / N;
  const int64_t total = tokens * kv_heads * per_head;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int c = (int)(i % per_head);
    const int64_t row = i / per_head;  // token * kv_heads + head
    int64_t key, value;
    if (!cache_place(e, row / kv_heads, kv_heads, dim, (int)(row % kv_heads), key, value)) continue;
    float kx[N], vx[N];
    Chunk<T>::load(k + row * dim + c * N, kx);
    Chunk<T>::load(e.v + row * dim + c * N, vx);
    store_f16<N>(e.keys + key + c * N, kx);
#pragma unroll
    for (int j = 0; j < N; ++j) e.values[value + (int64_t)(c * N + j) * e.page_size] = (uint16_t)f16_bits(vx[j]);
  }
}

template <typename T>
__global__ void __launch_bounds__(256) cache_write_values(const T* k, Extras<T> e, int64_t tokens, int kv_heads,
                                                          int dim) {
  const int64_t total = tokens * kv_heads * dim;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int d = (int)(i % dim);
    const int64_t row = i / dim;
    int64_t key, value;
    if (!cache_place(e, row / kv_heads, kv_heads, dim, (int)(row % kv_heads), key, value)) continue;
    e.keys[key + d] = (uint16_t)f16_bits(load_one(k + i));
    e.values[value + (int64_t)d * e.page_size] = (uint16_t)f16_bits(load_one(e.v + i));
  }
}

// [rows, 2 d] into [rows, d] and [rows, d] (kernels/linear_attention.hip:
// 298-307): a thread per 16-byte chunk of the outputs, or per value.
template <typename T>
__global__ void __launch_bounds__(256) split_halves_chunks(const T* x, T* first, T* second, int64_t rows, int d) {
  constexpr int N = Chunk<T>::N;
  const int per_row = d / N;
  const int64_t total = rows * per_row;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / per_row;
    const int c = (int)(i % per_row) * N;
    const uint4 a = stream_load(x + r * 2 * d + c), b = stream_load(x + r * 2 * d + d + c);
    __builtin_nontemporal_store(u32x4{a.x, a.y, a.z, a.w}, reinterpret_cast<u32x4*>(first + r * d + c));
    __builtin_nontemporal_store(u32x4{b.x, b.y, b.z, b.w}, reinterpret_cast<u32x4*>(second + r * d + c));
  }
}

template <typename T>
__global__ void __launch_bounds__(256) split_halves_values(const T* x, T* first, T* second, int64_t rows, int d) {
  const int64_t total = rows * d;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / d;
    const int c = (int)(i % d);
    first[i] = x[r * 2 * d + c];
    second[i] = x[r * 2 * d + d + c];
  }
}

// ------------------------------------------------------------------ launch layer

// Picks the kernel for a checked call: the per-lane-chunk one where heads
// are whole 16-byte chunks with every value turning (and the tensors allow
// 16-byte access), else the LDS one.
template <typename T, bool EXTRAS>
int qk_launch(const char* entry, const T* q, const T* k, T* q_out, T* k_out, const float* q_weight,
              const float* k_weight, const int32_t* positions, const QkArgs& a, const Extras<T>& e, bool aligned,
              hipStream_t st) {
  const RopeArgs& p = a.rope;
  constexpr int N = Chunk<T>::N;
  const int dim = p.dim;
  const int lanes_per_head = dim / (2 * N);
  const bool whole = p.rotary == dim && dim % (2 * N) == 0 && (lanes_per_head & (lanes_per_head - 1)) == 0 &&
                     lanes_per_head <= kWave / 2 && aligned && p.sections == DRIFT_SECTIONS_SINGLE;
  if (!whole) {
    hipLaunchKernelGGL((qk_norm_rope_kernel<T, EXTRAS>), dim3(grid_for(p.tokens, 1, 1 << 16)), dim3(256), 0, st, q,
                       k, q_out, k_out, q_weight, k_weight, positions, a, e);
    return launched(entry);
  }
  // a one-wave block per (token, group of 64 / G heads); with the cache,
  // blocks before those write the values by tiles of 16 positions
  const int heads_per_wave = kWave / lanes_per_head;
  // the fast body: query heads fill whole waves and the weight offset is 0;
  // two passes a wave where the query heads fill whole pairs of waves
  const bool fast = a.q_heads % heads_per_wave == 0 && a.offset == 0.0f;
  const int passes = fast && !EXTRAS && a.q_heads % (2 * heads_per_wave) == 0 ? 2 : 1;
  const int waves_per_token = (int)ceil_div(a.q_heads + a.kv_heads, heads_per_wave * passes);
  // with the fast body a wave's heads are all queries or all keys, and the
  // grid runs the query waves and the key waves apart (the key waves first
  // when they write the cache, last otherwise); else token by token
  const int query_waves = fast && a.kv_heads > 0 ? a.q_heads / (heads_per_wave * passes) : waves_per_token;
  const bool keys_first = EXTRAS && e.keys != nullptr;
  Extras<T> ex = e;
  const int tile_heads = kTileHeads(dim);
  ex.tiles = EXTRAS && e.keys ? ((int64_t)(e.start + p.tokens - 1) / 16 - e.start / 16 + 1) *
                                    ((a.kv_heads + tile_heads - 1) / tile_heads)
                              : 0;
  const int64_t blocks = (int64_t)p.tokens * waves_per_token + ex.tiles;
  if (blocks > INT32_MAX) return refuse("%s: %d tokens of %d heads", entry, p.tokens, a.q_heads + a.kv_heads);
  const dim3 grid((unsigned)blocks), block(kWave);
  switch (lanes_per_head) {
#define DRIFT_QK_LAUNCH(G, NEOX, GATE)                                                                               \
  if (passes == 2)                                                                                                   \
    hipLaunchKernelGGL((qk_norm_rope_wave<T, G, NEOX, EXTRAS, GATE, true, EXTRAS ? 1 : 2>), grid, block, 0, st, q,  \
                       k, q_out, k_out, q_weight, k_weight, positions, a, ex, waves_per_token, query_waves, keys_first);\
  else if (fast)                                                                                                     \
    hipLaunchKernelGGL((qk_norm_rope_wave<T, G, NEOX, EXTRAS, GATE, true, 1>), grid, block, 0, st, q, k, q_out,     \
                       k_out, q_weight, k_weight, positions, a, ex, waves_per_token, query_waves, keys_first);      \
  else                                                                                                               \
    hipLaunchKernelGGL((qk_norm_rope_wave<T, G, NEOX, EXTRAS, GATE, false, 1>), grid, block, 0, st, q, k, q_out,    \
                       k_out, q_weight, k_weight, positions, a, ex, waves_per_token, query_waves, keys_first)
#define DRIFT_QK_CASE(G)                                                                                             \
  case G:                                                                                                            \
    if (EXTRAS && e.gate) {                                                                                          \
      if (p.layout == DRIFT_ROPE_NEOX)                                                                               \
        DRIFT_QK_LAUNCH(G, true, EXTRAS);                                                                            \
      else                                                                                                           \
        DRIFT_QK_LAUNCH(G, false, EXTRAS);                                                                           \
    } else if (p.layout == DRIFT_ROPE_NEOX) {                                                                        \
      DRIFT_QK_LAUNCH(G, true, false);                                                                               \
    } else {                                                                                                         \
      DRIFT_QK_LAUNCH(G, false, false);                                                                              \
    }                                                                                                                \
    break;
    DRIFT_QK_CASE(1)
    DRIFT_QK_CASE(2)
    DRIFT_QK_CASE(4)
    DRIFT_QK_CASE(8)
    DRIFT_QK_CASE(16)
    DRIFT_QK_CASE(32)
#undef DRIFT_QK_CASE
#undef DRIFT_QK_LAUNCH
    default:
      return refuse("%s: no kernel for heads of %d values", entry, dim);
  }
  return launched(entry);
}

template <typename T>
int qk_norm_rope(const char* entry, const T* q, const T* k, T* q_out, T* k_out, const float* q_weight,
                 const float* k_weight, const int32_t* positions, int32_t tokens, int32_t heads, int32_t kv_heads,
                 int32_t dim, float eps, float offset, int32_t rotary, float theta, int32_t layout,
                 int32_t sections, int32_t s0, int32_t s1, int32_t s2, int32_t s3, void* stream) {
  clear_error();
  const int32_t s[4] = {s0, s1, s2, s3};
  if (kv_heads < 0) return refuse("%s: %d key heads", entry, kv_heads);
  if (const int bad = check_rope(entry, tokens, heads, dim, rotary, layout, sections, s)) return bad;
  if ((int64_t)tokens * (heads + kv_heads) == 0) return 0;
  if (!positions || (heads > 0 && (!q || !q_out || !q_weight)) || (kv_heads > 0 && (!k || !k_out || !k_weight)))
    return refuse("%s: null tensor", entry);
  QkArgs a;
  fill_rope(a.rope, tokens, heads, dim, rotary, theta, layout, sections, s);
  a.q_heads = heads;
  a.kv_heads = kv_heads;
  a.eps = eps;
  a.offset = offset;
  a.q_stride = dim;
  // the fast body reads the norm weights as 16-byte loads too
  const bool aligned = (!q || (aligned16(q) && aligned16(q_out) && aligned16(q_weight))) &&
                       (!k || (aligned16(k) && aligned16(k_out) && aligned16(k_weight)));
  return qk_launch<T, false>(entry, q, k, q_out, k_out, q_weight, k_weight, positions, a, Extras<T>{}, aligned,
                             (hipStream_t)stream);
}

// attention_inputs: the checks of the reference's attentionInputs
// (ops/HipAttention.scala:144-215: checkSplitHalves, checkRope,
// checkCacheWrite and checkPageTable, ops/AttentionOps.scala:225-256), then
// one launch.
template <typename T>
int attention_inputs(const char* entry, const T* query_and_gate, const T* k, const T* v, const float* q_norm,
                     const float* k_norm, float eps, float offset, const int32_t* positions, int32_t tokens,
                     int32_t heads, int32_t kv_heads, int32_t dim, int32_t rotary, float theta, int32_t layout,
                     int32_t sections, int32_t s0, int32_t s1, int32_t s2, int32_t s3, T* queries, T* gate,
                     uint16_t* keys, uint16_t* values, const int32_t* page_table, int32_t table_pages,
                     int32_t cache_pages, int32_t page_size, int32_t start, int32_t* bad_page, void* stream) {
  clear_error();
  const int32_t s[4] = {s0, s1, s2, s3};
  if (kv_heads < 0) return refuse("%s: %d key heads", entry, kv_heads);
  if (const int bad = check_rope(entry, tokens, heads, dim, rotary, layout, sections, s)) return bad;
  if (page_size <= 0 || page_size % 16 != 0) return refuse("%s: pages of %d tokens: not a multiple of 16", entry, page_size);
  if (start < 0 || table_pages < 0 || cache_pages < 0)
    return refuse("%s: start %d, %d table pages, %d cache pages", entry, start, table_pages, cache_pages);
  if ((int64_t)table_pages * page_size < (int64_t)start + tokens)
    return refuse("%s: a page table of %d pages for %lld positions", entry, table_pages,
                  (long long)start + tokens);
  if ((int64_t)tokens * (heads + kv_heads) == 0) return 0;
  if (!positions || (heads > 0 && (!query_and_gate || !queries || !q_norm)) ||
      (kv_heads > 0 && (!k || !v || !k_norm || !keys || !values || !page_table)))
    return refuse("%s: null tensor", entry);
  QkArgs a;
  fill_rope(a.rope, tokens, heads, dim, rotary, theta, layout, sections, s);
  a.q_heads = heads;
  a.kv_heads = kv_heads;
  a.eps = eps;
  a.offset = offset;
  a.q_stride = gate ? 2 * (int64_t)dim : dim;
  const Extras<T> e{gate, v, keys, values, page_table, cache_pages, page_size, start, bad_page, 0};
  const bool aligned = (!query_and_gate || (aligned16(query_and_gate) && aligned16(queries) && aligned16(q_norm))) &&
                       (!gate || aligned16(gate)) && (!k || (aligned16(k) && aligned16(v) && aligned16(k_norm))) &&
                       (!keys || (aligned16(keys) && aligned16(values)));
  return qk_launch<T, true>(entry, query_and_gate, k, queries, nullptr, q_norm, k_norm, positions, a, e, aligned,
                            (hipStream_t)stream);
}

template <typename T>
int cache_write(const char* entry, const T* k, const T* v, uint16_t* keys, uint16_t* values,
                const int32_t* page_table, int32_t table_pages, int32_t cache_pages, int32_t tokens,
                int32_t kv_heads, int32_t dim, int32_t page_size, int32_t start, int32_t* bad_page, void* stream) {
  clear_error();
  if (tokens < 0 || kv_heads < 0 || dim <= 0)
    return refuse("%s: %d tokens of %d heads of %d values", entry, tokens, kv_heads, dim);
  if (page_size <= 0 || page_size % 16 != 0) return refuse("%s: pages of %d tokens: not a multiple of 16", entry, page_size);
  if (start < 0 || table_pages < 0 || cache_pages < 0)
    return refuse("%s: start %d, %d table pages, %d cache pages", entry, start, table_pages, cache_pages);
  if ((int64_t)table_pages * page_size < (int64_t)start + tokens)
    return refuse("%s: a page table of %d pages for %lld positions", entry, table_pages,
                  (long long)start + tokens);
  if ((int64_t)tokens * kv_heads == 0) return 0;
  if (!k || !v || !keys || !values || !page_table) return refuse("%s: null tensor", entry);
  const Extras<T> e{nullptr, v, keys, values, page_table, cache_pages, page_size, start, bad_page, 0};
  constexpr int N = Chunk<T>::N;
  const hipStream_t st = (hipStream_t)stream;
  const int64_t values_count = (int64_t)tokens * kv_heads * dim;
  if (dim % N == 0 && aligned16(k) && aligned16(v) && aligned16(keys))
    hipLaunchKernelGGL(cache_write_chunks<T>, dim3(grid_for(values_count / N, 256, kOneShotBlocks)), dim3(256), 0, st,
                       k, e, (int64_t)tokens, kv_heads, dim);
  else
    hipLaunchKernelGGL(cache_write_values<T>, dim3(grid_for(values_count, 256, kOneShotBlocks)), dim3(256), 0, st, k,
                       e, (int64_t)tokens, kv_heads, dim);
  return launched(entry);
}

template <typename T>
int split_halves(const char* entry, const T* x, T* first, T* second, int64_t rows, int32_t d, void* stream) {
  clear_error();
  if (rows < 0 || d <= 0) return refuse("%s: %lld rows of 2 x %d values", entry, (long long)rows, d);
  if (rows == 0) return 0;
  if (!x || !first || !second) return refuse("%s: null tensor", entry);
  constexpr int N = Chunk<T>::N;
  const hipStream_t st = (hipStream_t)stream;
  if (d % N == 0 && aligned16(x) && aligned16(first) && aligned16(second))
    hipLaunchKernelGGL(split_halves_chunks<T>, dim3(grid_for(rows * (d / N), 256, kOneShotBlocks)), dim3(256), 0, st,
                       x, first, second, rows, (int)d);
  else
    hipLaunchKernelGGL(split_halves_values<T>, dim3(grid_for(rows * d, 256, kOneShotBlocks)), dim3(256), 0, st, x,
                       first, second, rows, (int)d);
  return launched(entry);
}

}  // namespace
}  // namespace drift

using namespace drift;

extern "C" int drift_qk_norm_rope_f32(const float* q, const float* k, float* q_out, float* k_out,
                                      const float* q_weight, const float* k_weight, const int32_t* positions,
                                      int32_t tokens, int32_t heads, int32_t kv_heads, int32_t head_dim, float eps,
                                      float offset, int32_t rotary, float theta, int32_t layout, int32_t sections,
                                      int32_t s0, int32_t s1, int32_t s2, int32_t s3, void* stream) {
  return qk_norm_rope<float>("drift_qk_norm_rope_f32", q, k, q_out, k_out, q_weight, k_weight, positions, tokens,
                             heads, kv_heads, head_dim, eps, offset, rotary, theta, layout, sections, s0, s1, s2, s3,
                             stream);
}

extern "C" int drift_qk_norm_rope_bf16(const uint16_t* q, const uint16_t* k, uint16_t* q_out, uint16_t* k_out,
                                       const float* q_weight, const float* k_weight, const int32_t* positions,
                                       int32_t tokens, int32_t heads, int32_t kv_heads, int32_t head_dim, float eps,
                                       float offset, int32_t rotary, float theta, int32_t layout, int32_t sections,
                                       int32_t s0, int32_t s1, int32_t s2, int32_t s3, void* stream) {
  return qk_norm_rope<uint16_t>("drift_qk_norm_rope_bf16", q, k, q_out, k_out, q_weight, k_weight, positions, tokens,
                                heads, kv_heads, head_dim, eps, offset, rotary, theta, layout, sections, s0, s1, s2,
                                s3, stream);
}

extern "C" int drift_attention_inputs_f32(const float* query_and_gate, const float* k, const float* v,
                                          const float* q_norm, const float* k_norm, float eps, float offset,
                                          const int32_t* positions, int32_t tokens, int32_t heads, int32_t kv_heads,
                                          int32_t head_dim, int32_t rotary, float theta, int32_t layout,
                                          int32_t sections, int32_t s0, int32_t s1, int32_t s2, int32_t s3,
                                          float* queries, float* gate, uint16_t* keys, uint16_t* values,
                                          const int32_t* page_table, int32_t table_pages, int32_t cache_pages,
                                          int32_t page_size, int32_t start, int32_t* bad_page, void* stream) {
  return attention_inputs<float>("drift_attention_inputs_f32", query_and_gate, k, v, q_norm, k_norm, eps, offset,
                                 positions, tokens, heads, kv_heads, head_dim, rotary, theta, layout, sections, s0,
                                 s1, s2, s3, queries, gate, keys, values, page_table, table_pages, cache_pages,
                                 page_size, start, bad_page, stream);
}

extern "C" int drift_attention_inputs_bf16(const uint16_t* query_and_gate, const uint16_t* k, const uint16_t* v,
                                           const float* q_norm, const float* k_norm, float eps, float offset,
                                           const int32_t* positions, int32_t tokens, int32_t heads, int32_t kv_heads,
                                           int32_t head_dim, int32_t rotary, float theta, int32_t layout,
                                           int32_t sections, int32_t s0, int32_t s1, int32_t s2, int32_t s3,
                                           uint16_t* queries, uint16_t* gate, uint16_t* keys, uint16_t* values,
                                           const int32_t* page_table, int32_t table_pages, int32_t cache_pages,
                                           int32_t page_size, int32_t start, int32_t* bad_page, void* stream) {
  return attention_inputs<uint16_t>("drift_attention_inputs_bf16", query_and_gate, k, v, q_norm, k_norm, eps,
                                    offset, positions, tokens, heads, kv_heads, head_dim, rotary, theta, layout,
                                    sections, s0, s1, s2, s3, queries, gate, keys, values, page_table, table_pages,
                                    cache_pages, page_size, start, bad_page, stream);
}

extern "C" int drift_cache_write_f32(const float* k, const float* v, uint16_t* keys, uint16_t* values,
                                     const int32_t* page_table, int32_t table_pages, int32_t cache_pages,
                                     int32_t tokens, int32_t kv_heads, int32_t head_dim, int32_t page_size,
                                     int32_t start, int32_t* bad_page, void* stream) {
  return cache_write<float>("drift_cache_write_f32", k, v, keys, values, page_table, table_pages, cache_pages, tokens,
                            kv_heads, head_dim, page_size, start, bad_page, stream);
}

extern "C" int drift_cache_write_bf16(const uint16_t* k, const uint16_t* v, uint16_t* keys, uint16_t* values,
                                      const int32_t* page_table, int32_t table_pages, int32_t cache_pages,
                                      int32_t tokens, int32_t kv_heads, int32_t head_dim, int32_t page_size,
                                      int32_t start, int32_t* bad_page, void* stream) {
  return cache_write<uint16_t>("drift_cache_write_bf16", k, v, keys, values, page_table, table_pages, cache_pages,
                               tokens, kv_heads, head_dim, page_size, start, bad_page, stream);
}

extern "C" int drift_split_halves_f32(const float* x, float* first, float* second, int64_t rows, int32_t d,
                                      void* stream) {
  return split_halves<float>("drift_split_halves_f32", x, first, second, rows, d, stream);
}

extern "C" int drift_split_halves_bf16(const uint16_t* x, uint16_t* first, uint16_t* second, int64_t rows, int32_t d,
                                       void* stream) {
  return split_halves<uint16_t>("drift_split_halves_bf16", x, first, second, rows, d, stream);
}
