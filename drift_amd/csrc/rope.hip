// Rotary embeddings for gfx950: rope by positions (NeoX, interleaved, mRoPE
// sections, per-axis), rope from cos/sin tables, Wan's 3-D rope with its
// angles made in the kernel, and per-head query/key RMSNorm fused with rope.
//
// Layout: x, out [tokens, heads, head_dim], row-major. One workgroup takes a
// token at a time: it first makes the token's cos/sin for every pair (once,
// shared by all its heads: the reference recomputes them per value), then
// turns every head's pairs. Where a head is whole 16-byte chunks, each lane
// reads a pair's two chunks (NeoX: a chunk and its partner half a rotary
// away; interleaved: pairs sit inside a chunk), turns them in registers and
// writes them back, so out may be x.
//
// Arithmetic is the CPU reference's (ops/CpuAttention.scala:53-146):
// inverse frequency = 1f / float(pow(theta, 2i/rotary)) (host-side, double
// pow, as the CPU), angle = float(position) * inverse in float, cos and sin
// of it in double, the turn a*c - b*s, a*s + b*c in double, rounded once.
// Wan's tables (models/Wan.scala:324-361) are cos and sin of a double angle
// rounded to float; rope_3d makes exactly those values.
#include "common.hpp"

#include <algorithm>
#include <climits>

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
// the rest copy two tail values), scalar loads. Reads before it writes.
template <typename T, typename Load>
__device__ __forceinline__ void turn_slot(int j, int dim, int rotary, int layout, const double2* cs, Load load,
                                          T* head_out) {
  const int half = rotary / 2;
  if (j < half) {
    const int d0 = layout == DRIFT_ROPE_NEOX ? j : 2 * j;
    const int d1 = layout == DRIFT_ROPE_NEOX ? j + half : 2 * j + 1;
    const double a = load(d0), b = load(d1);
    float f, s;
    turn(a, b, cs[j].x, cs[j].y, f, s);
    store_one(head_out + d0, f);
    store_one(head_out + d1, s);
  } else {
    const int e = rotary + 2 * (j - half);
    const float v0 = load(e);
    const float v1 = e + 1 < dim ? (float)load(e + 1) : 0.0f;
    store_one(head_out + e, v0);
    if (e + 1 < dim) store_one(head_out + e + 1, v1);
  }
}

// ------------------------------------------------------------------ rope

// Chunked turn of a head: lane items are chunk pairs. NeoX: chunk i (< half/N)
// with chunk i + half/N; interleaved: one chunk, its N/2 pairs inside. Tail
// chunks (from rotary on) are copied.
template <typename T>
__device__ __forceinline__ void turn_chunks(const T* xh, T* oh, int item, int dim, int rotary, int layout,
                                            const double2* cs) {
  constexpr int N = Chunk<T>::N;
  const int half = rotary / 2;
  if (layout == DRIFT_ROPE_NEOX) {
    const int rotating = half / N;  // chunk pairs
    if (item < rotating) {
      float a[N], b[N];
      Chunk<T>::load(xh + item * N, a);
      Chunk<T>::load(xh + half + item * N, b);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const double2 q = cs[item * N + i];
        turn(a[i], b[i], q.x, q.y, a[i], b[i]);
      }
      Chunk<T>::store(oh + item * N, a);
      Chunk<T>::store(oh + half + item * N, b);
    } else {
      const int d = rotary + (item - rotating) * N;
      float v[N];
      Chunk<T>::load(xh + d, v);
      Chunk<T>::store(oh + d, v);
    }
  } else {
    const int d = item * N;
    float v[N];
    Chunk<T>::load(xh + d, v);
    if (d < rotary) {
#pragma unroll
      for (int i = 0; i < N; i += 2) {
        const double2 q = cs[d / 2 + i / 2];
        turn(v[i], v[i + 1], q.x, q.y, v[i], v[i + 1]);
      }
    }
    Chunk<T>::store(oh + d, v);
  }
}

template <typename T>
__device__ __forceinline__ int chunk_items(int dim, int rotary, int layout) {
  constexpr int N = Chunk<T>::N;
  return layout == DRIFT_ROPE_NEOX ? rotary / 2 / N + (dim - rotary) / N : dim / N;
}

template <typename T, bool CHUNKED>
__global__ void __launch_bounds__(256) rope_kernel(const T* x, const int32_t* positions, T* out, RopeArgs p) {
  __shared__ double2 cs[kMaxPairs];
  const int slots = CHUNKED ? chunk_items<T>(p.dim, p.rotary, p.layout) : (p.dim + 1) / 2;
  for (int64_t t = blockIdx.x; t < p.tokens; t += gridDim.x) {
    token_angles(p, positions, t, cs);
    __syncthreads();
    const T* xt = x + t * p.heads * p.dim;
    T* ot = out + t * p.heads * p.dim;
    for (int i = threadIdx.x; i < p.heads * slots; i += blockDim.x) {
      const int h = i / slots, j = i % slots;
      const T* xh = xt + (int64_t)h * p.dim;
      T* oh = ot + (int64_t)h * p.dim;
      if constexpr (CHUNKED)
        turn_chunks<T>(xh, oh, j, p.dim, p.rotary, p.layout, cs);
      else
        turn_slot<T>(j, p.dim, p.rotary, p.layout, cs, [&](int d) { return (double)load_one(xh + d); }, oh);
    }
    __syncthreads();  // cs is remade for the next token
  }
}

// ------------------------------------------------------------------ rope from tables

template <typename T>
__global__ void __launch_bounds__(256) rope_table_kernel(const T* x, const float* cosines, const float* sines, T* out,
                                                         int tokens, int heads, int dim, int pairs, int per_head,
                                                         int halves) {
  const int slots = (dim + 1) / 2;
  const int64_t items = (int64_t)tokens * heads * slots;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < items; i += stride) {
    const int j = (int)(i % slots);
    const int64_t head_row = i / slots;  // token * heads + head
    const int64_t row = per_head ? head_row : head_row / heads;
    const T* xh = x + head_row * dim;
    T* oh = out + head_row * dim;
    if (j < pairs) {
      const int d0 = halves ? j : 2 * j;
      const int d1 = halves ? j + pairs : 2 * j + 1;
      const double c = (double)cosines[row * pairs + j], s = (double)sines[row * pairs + j];
      const double a = (double)load_one(xh + d0), b = (double)load_one(xh + d1);
      float f, g;
      turn(a, b, c, s, f, g);
      store_one(oh + d0, f);
      store_one(oh + d1, g);
    } else {
      const int e = 2 * pairs + 2 * (j - pairs);
      const float v0 = load_one(xh + e);
      const float v1 = e + 1 < dim ? load_one(xh + e + 1) : 0.0f;
      store_one(oh + e, v0);
      if (e + 1 < dim) store_one(oh + e + 1, v1);
    }
  }
}

// ------------------------------------------------------------------ Wan 3-D rope

struct Rope3dArgs {
  double denominator[kMaxPairs];  // theta^(2 index / (2 pairs_axis)) per pair
  int64_t tokens, token_offset, grid;
  int32_t heads, dim, rows, cols, pairs0, pairs1;
};

template <typename T, bool CHUNKED>
__global__ void __launch_bounds__(256) rope_3d_kernel(const T* x, T* out, Rope3dArgs p) {
  __shared__ double2 cs[kMaxPairs];
  constexpr int N = Chunk<T>::N;
  const int half = p.dim / 2;
  const int slots = CHUNKED ? p.dim / N : half;
  for (int64_t t = blockIdx.x; t < p.tokens; t += gridDim.x) {
    const int64_t g = (p.token_offset + t) % p.grid;
    for (int j = threadIdx.x; j < half; j += blockDim.x) {
      const int64_t position = j < p.pairs0 ? g / ((int64_t)p.rows * p.cols)
                                            : (j < p.pairs0 + p.pairs1 ? g / p.cols % p.rows : g % p.cols);
      const double angle = (double)position / p.denominator[j];
      double sn, cn;
      sincos(angle, &sn, &cn);
      cs[j] = make_double2((double)(float)cn, (double)(float)sn);  // the F32 tables' values
    }
    __syncthreads();
    const T* xt = x + t * p.heads * p.dim;
    T* ot = out + t * p.heads * p.dim;
    for (int i = threadIdx.x; i < p.heads * slots; i += blockDim.x) {
      const int h = i / slots, j = i % slots;
      const T* xh = xt + (int64_t)h * p.dim;
      T* oh = ot + (int64_t)h * p.dim;
      if constexpr (CHUNKED)
        turn_chunks<T>(xh, oh, j, p.dim, p.dim, DRIFT_ROPE_INTERLEAVED, cs);
      else
        turn_slot<T>(j, p.dim, p.dim, DRIFT_ROPE_INTERLEAVED, cs, [&](int d) { return (double)load_one(xh + d); },
                     oh);
    }
    __syncthreads();
  }
}

// One wave per token, the grid covering the tokens in one pass. A wave issues
// its token's loads first; while they land, each lane makes one pair's angle
// (Wan's angle depends on one axis position: frame, row or column) and its
// cos and sin, exactly as the host tables hold them (cos and sin of the
// double angle, rounded to float), into the wave's LDS slice. Then each lane
// turns its chunks' pairs. With a, b bf16 or F32 and c, s floats, a*c and b*s
// are exact in double, so fma(a, c, -b*s) is the reference's a*c - b*s
// rounded once.
constexpr int kRope3dWaves = 8;

template <typename T, int K, bool FIXED>
__global__ void __launch_bounds__(kRope3dWaves * 64) rope_3d_waves(const T* x, T* out, Rope3dArgs p) {
  constexpr int N = Chunk<T>::N;
  using Raw = typename Chunk<T>::Raw;
  __shared__ float2 cs_all[kRope3dWaves][kMaxPairs];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = (int64_t)blockIdx.x * kRope3dWaves + wave;
  if (t >= p.tokens) return;  // no block-wide barrier follows
  const int per_token = p.heads * p.dim / N;  // chunks of a token, at most K * 64
  const int per_head = p.dim / N;
  const T* xt = x + t * p.heads * p.dim;
  // loads are never branched around (a branch makes each wait for the one
  // before): chunk indices past the token are clamped and their values unused
  Raw raw[K];
#pragma unroll
  for (int k = 0; k < K; ++k) raw[k] = Chunk<T>::load_raw(xt + min(k * kWave + lane, per_token - 1) * N);
  const int64_t g = (p.token_offset + t) % p.grid;
  const int plane = p.rows * p.cols;
  const int frame = (int)(g / plane), rem = (int)(g % plane);
  const int row = rem / p.cols, col = rem % p.cols;
  const int half = p.dim / 2;
  float2* cs = cs_all[wave];
  for (int m = lane; m < half; m += kWave) {
    const int position = m < p.pairs0 ? frame : (m < p.pairs0 + p.pairs1 ? row : col);
    double sn, cn;
    sincos((double)position / p.denominator[m], &sn, &cn);
    cs[m] = make_float2((float)cn, (float)sn);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // the lane's pairs' cos and sin, when they are the same in every chunk
  double fc[N / 2], fs[N / 2];
  if constexpr (FIXED) {
    const int m0 = (lane % per_head) * N / 2;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const float2 q = cs[m0 + i];
      fc[i] = q.x;
      fs[i] = q.y;
    }
  }
  T* ot = out + t * p.heads * p.dim;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int q = k * kWave + lane;
    if (q < per_token) {
      float v[N];
      Chunk<T>::unpack(raw[k], v);
      const int m0 = (q % per_head) * N / 2;
#pragma unroll
      for (int i = 0; i < N / 2; ++i) {
        double c, sn;
        if constexpr (FIXED) {
          c = fc[i];
          sn = fs[i];
        } else {
          const float2 e = cs[m0 + i];
          c = e.x;
          sn = e.y;
        }
        const double a = v[2 * i], b = v[2 * i + 1];
        v[2 * i] = (float)fma(a, c, -(b * sn));
        v[2 * i + 1] = (float)fma(a, sn, b * c);
      }
      Chunk<T>::store(ot + q * N, v);
    }
  }
}

// ------------------------------------------------------------------ per-head RMSNorm + rope

struct QkArgs {
  RopeArgs rope;
  int32_t q_heads, kv_heads;
  float eps, offset;
};

// Any head size: each wave norms one head row at a time into LDS (the F32
// values rmsNorm writes), then turns its pairs from there.
template <typename T>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(const T* q, const T* k, T* q_out, T* k_out,
                                                           const float* q_weight, const float* k_weight,
                                                           const int32_t* positions, QkArgs a) {
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
      const T* xh = query ? q + (t * a.q_heads + h) * p.dim : k + (t * a.kv_heads + (h - a.q_heads)) * p.dim;
      T* oh = query ? q_out + (t * a.q_heads + h) * p.dim : k_out + (t * a.kv_heads + (h - a.q_heads)) * p.dim;
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
        const double factor = 1.0 / sqrt(group_sum<64>(squares) / (double)p.dim + (double)a.eps);
#pragma unroll
        for (int i = 0; i < 2 * kMaxPairs / kWave; ++i) {
          const int d = i * kWave + lane;
          if (d < p.dim) normed[wave][d] = (float)((double)v[i] * factor * ((double)w[d] + (double)a.offset));
        }
      }
      __syncthreads();  // normed rows and (first round) cs are ready
      if (h < rows)
        for (int j = lane; j < slots; j += kWave)
          turn_slot<T>(j, p.dim, p.rotary, p.layout, cs, [&](int d) { return (double)normed[wave][d]; }, oh);
      __syncthreads();  // normed is reused next round, cs next token
    }
  }
}

// The fast path for whole-chunk heads with every value turning: one block per
// token, G lanes per head, each lane holding two chunks of its head (NeoX: a
// chunk and its partner; otherwise chunks i and i + G), 64 / G heads per
// wave. The grid covers the tokens in one pass. Each lane issues its loads
// first; while they land the block makes the token's cos and sin (one sincos
// per pair) and the norm weights (+ offset, in double) into LDS.
//
// LDS is laid out so the G lanes of a head read consecutive entries: for NeoX
// the pair (and weight) of lane i0's value i sits at i * G + i0 (the natural
// index would put the G lanes N entries apart, on the same banks).
template <bool NEOX, int G, int N>
__device__ __forceinline__ int qk_pair_slot(int pair) {
  if constexpr (NEOX) return (pair % N) * G + pair / N;
  return pair;
}

template <bool NEOX, int G, int N>
__device__ __forceinline__ int qk_weight_slot(int d) {
  if constexpr (NEOX) {
    const int half = N * G;
    const int h = d >= half ? 1 : 0, e = d - h * half;
    return h * half + (e % N) * G + e / N;
  }
  return d;
}

constexpr int kQkMaxWaves = 16;

template <typename T, int G, bool NEOX>
__global__ void __launch_bounds__(kQkMaxWaves * 64) qk_norm_rope_token(const T* q, const T* k, T* q_out, T* k_out,
                                                                     const float* q_weight, const float* k_weight,
                                                                     const int32_t* positions, QkArgs a) {
  constexpr int N = Chunk<T>::N;
  using Raw = typename Chunk<T>::Raw;
  constexpr int kHeadsPerWave = kWave / G;
  constexpr int kPairs = N * G;  // a head's pairs (rotary == dim == 2 N G)
  __shared__ double2 cs[kPairs];
  __shared__ double weights[2][2 * kPairs];
  const RopeArgs& p = a.rope;
  constexpr int dim = 2 * N * G, half = N * G;
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int rows = a.q_heads + a.kv_heads;
  const int i0 = lane % G;
  const int d0 = i0 * N, d1 = (NEOX ? half : G * N) + i0 * N;
  auto head_at = [&](auto* qs, auto* ks, int h) {
    return h < a.q_heads ? qs + (t * a.q_heads + h) * dim : ks + (t * a.kv_heads + (h - a.q_heads)) * dim;
  };
  // the angles' and weights' operands load first: a wave's loads complete in
  // issue order, so the tables are made while the heads are still loading
  const int j = threadIdx.x, jp = min(j, half - 1), jd = min(j, dim - 1);
  const int32_t position = positions[(int64_t)rope_section(jp, p) * p.tokens + t];
  const float inverse = p.inverse[jp];
  const float qw = q_weight[jd], kw = k_weight[jd];
  // loads are never branched around (the wait for the angles' operands would
  // then wait for them too): a head past the last is clamped to it
  int h = wave * kHeadsPerWave + lane / G;
  const T* xh = head_at(q, k, min(h, rows - 1));
  Raw r0 = Chunk<T>::load_raw(xh + d0);
  Raw r1 = Chunk<T>::load_raw(xh + d1);
  if (j < half) {
    double sn, cn;
    sincos((double)((float)position * inverse), &sn, &cn);
    cs[qk_pair_slot<NEOX, G, N>(j)] = make_double2(cn, sn);
  }
  if (j < dim) {
    const int slot = qk_weight_slot<NEOX, G, N>(j);
    weights[0][slot] = (double)qw + (double)a.offset;
    weights[1][slot] = (double)kw + (double)a.offset;
  }
  __syncthreads();
  for (;;) {
    const bool live = h < rows;
    float v0[N], v1[N];
    double squares = 0.0;
    if (live) {
      Chunk<T>::unpack(r0, v0);
      Chunk<T>::unpack(r1, v1);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        squares = fma((double)v0[i], (double)v0[i], squares);
        squares = fma((double)v1[i], (double)v1[i], squares);
      }
    }
    squares = group_sum<G>(squares);
    if (live) {
      const double factor = 1.0 / sqrt(squares / (double)dim + (double)a.eps);
      const double* w = weights[h < a.q_heads ? 0 : 1];
#pragma unroll
      for (int i = 0; i < N; ++i) {
        v0[i] = (float)((double)v0[i] * factor * w[qk_weight_slot<NEOX, G, N>(d0 + i)]);
        v1[i] = (float)((double)v1[i] * factor * w[qk_weight_slot<NEOX, G, N>(d1 + i)]);
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
      T* oh = head_at(q_out, k_out, h);
      Chunk<T>::store(oh + d0, v0);
      Chunk<T>::store(oh + d1, v1);
    }
    // more heads than the block has waves for: the next pass of this wave
    h += waves * kHeadsPerWave;
    if (h - lane / G >= rows) break;
    xh = head_at(q, k, min(h, rows - 1));
    r0 = Chunk<T>::load_raw(xh + d0);
    r1 = Chunk<T>::load_raw(xh + d1);
  }
}

// ------------------------------------------------------------------ launch layer

int check_rope(const char* entry, int32_t tokens, int32_t heads, int32_t dim, int32_t rotary, int32_t layout,
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
void fill_rope(RopeArgs& p, int32_t tokens, int32_t heads, int32_t dim, int32_t rotary, float theta, int32_t layout,
               int32_t sections, const int32_t (&s)[4]) {
  p.tokens = tokens;
  p.heads = heads;
  p.dim = dim;
  p.rotary = rotary;
  p.layout = layout;
  p.sections = sections;
  for (int a = 0; a < 4; ++a) p.s[a] = s[a];
  for (int pair = 0; pair < kMaxPairs; ++pair) {
    if (pair >= rotary / 2) {
      p.inverse[pair] = 0.0f;
      continue;
    }
    double exponent = 2.0 * pair / (double)rotary;
    if (sections == DRIFT_SECTIONS_AXES) {
      int start = 0, axis = 0;
      while (pair >= start + s[axis]) start += s[axis++];
      exponent = (double)(pair - start) / (double)s[axis];
    }
    p.inverse[pair] = 1.0f / (float)std::pow((double)theta, exponent);
  }
}

template <typename T>
int rope(const char* entry, const T* x, const int32_t* positions, T* out, int32_t tokens, int32_t heads,
         int32_t dim, int32_t rotary, float theta, int32_t layout, int32_t sections, int32_t s0, int32_t s1,
         int32_t s2, int32_t s3, void* stream) {
  clear_error();
  const int32_t s[4] = {s0, s1, s2, s3};
  if (const int bad = check_rope(entry, tokens, heads, dim, rotary, layout, sections, s)) return bad;
  if ((int64_t)tokens * heads == 0) return 0;
  if (!x || !positions || !out) return refuse("%s: null x, positions or out", entry);
  RopeArgs p;
  fill_rope(p, tokens, heads, dim, rotary, theta, layout, sections, s);
  constexpr int N = Chunk<T>::N;
  const bool chunked = aligned16(x) && aligned16(out) && dim % N == 0 &&
                       rotary % (layout == DRIFT_ROPE_NEOX ? 2 * N : N) == 0;
  const dim3 grid(grid_for(tokens, 1, 1 << 16));
  const hipStream_t st = (hipStream_t)stream;
  if (chunked)
    hipLaunchKernelGGL((rope_kernel<T, true>), grid, dim3(256), 0, st, x, positions, out, p);
  else
    hipLaunchKernelGGL((rope_kernel<T, false>), grid, dim3(256), 0, st, x, positions, out, p);
  return launched(entry);
}

template <typename T>
int rope_table(const char* entry, const T* x, const float* cosines, const float* sines, T* out, int32_t tokens,
               int32_t heads, int32_t dim, int32_t pairs, int32_t per_head, int32_t halves, void* stream) {
  clear_error();
  if (tokens < 0 || heads < 0 || dim <= 0) return refuse("%s: %d tokens of %d heads of %d", entry, tokens, heads, dim);
  if (pairs < 0 || 2 * pairs > dim) return refuse("%s: %d pairs in heads of %d", entry, pairs, dim);
  if ((int64_t)tokens * heads == 0) return 0;
  if (!x || !cosines || !sines || !out) return refuse("%s: null x, cosines, sines or out", entry);
  const int64_t items = (int64_t)tokens * heads * ((dim + 1) / 2);
  hipLaunchKernelGGL(rope_table_kernel<T>, dim3(grid_for(items, 256, 1 << 16)), dim3(256), 0, (hipStream_t)stream,
                     x, cosines, sines, out, tokens, heads, dim, pairs, per_head ? 1 : 0, halves ? 1 : 0);
  return launched(entry);
}

template <typename T>
int rope_3d(const char* entry, const T* x, T* out, int64_t tokens, int32_t heads, int32_t dim, int32_t frames,
            int32_t rows, int32_t cols, int64_t token_offset, double theta, void* stream) {
  clear_error();
  if (tokens < 0 || heads < 0) return refuse("%s: %lld tokens of %d heads", entry, (long long)tokens, heads);
  if (dim <= 0 || dim % 2 != 0 || dim > 2 * kMaxPairs) return refuse("%s: heads of %d values", entry, dim);
  if (frames <= 0 || rows <= 0 || cols <= 0 || (int64_t)frames * rows * cols > INT32_MAX)
    return refuse("%s: a %d x %d x %d grid", entry, frames, rows, cols);
  if (token_offset < 0) return refuse("%s: token offset %lld", entry, (long long)token_offset);
  if (tokens * heads == 0) return 0;
  if (!x || !out) return refuse("%s: null x or out", entry);
  // WanConfig.ropePairs (models/Wan.scala:35-41)
  const int side = 2 * (dim / 6);
  const int axes[3] = {(dim - 2 * side) / 2, side / 2, side / 2};
  if (axes[0] <= 0 || axes[1] <= 0) return refuse("%s: heads of %d values are too narrow for 3 axes", entry, dim);
  Rope3dArgs p;
  p.tokens = tokens;
  p.token_offset = token_offset;
  p.grid = (int64_t)frames * rows * cols;
  p.heads = heads;
  p.dim = dim;
  p.rows = rows;
  p.cols = cols;
  p.pairs0 = axes[0];
  p.pairs1 = axes[1];
  for (int pair = 0; pair < kMaxPairs; ++pair) {
    if (pair >= dim / 2) {
      p.denominator[pair] = 1.0;
      continue;
    }
    const int axis = pair < axes[0] ? 0 : (pair < axes[0] + axes[1] ? 1 : 2);
    const int index = pair - (axis > 0 ? axes[0] : 0) - (axis > 1 ? axes[1] : 0);
    p.denominator[pair] = std::pow(theta, 2.0 * index / (double)(2 * axes[axis]));
  }
  constexpr int N = Chunk<T>::N;
  const bool chunked = aligned16(x) && aligned16(out) && dim % N == 0;
  const hipStream_t st = (hipStream_t)stream;
  const int per_lane = (int)ceil_div((int64_t)heads * dim / N, kWave);
  const int64_t blocks = ceil_div(tokens, kRope3dWaves);
  if (chunked && blocks <= kOneShotBlocks) {
    const bool fixed = (64 % (dim / N)) == 0;
#define DRIFT_ROPE3D_CASE(K)                                                                                  \
  if (per_lane <= K) {                                                                                        \
    if (fixed)                                                                                                \
      hipLaunchKernelGGL((rope_3d_waves<T, K, true>), dim3((unsigned)blocks), dim3(64 * kRope3dWaves), 0, st, \
                         x, out, p);                                                                          \
    else                                                                                                      \
      hipLaunchKernelGGL((rope_3d_waves<T, K, false>), dim3((unsigned)blocks), dim3(64 * kRope3dWaves), 0,    \
                         st, x, out, p);                                                                      \
    return launched(entry);                                                                                   \
  }
    DRIFT_ROPE3D_CASE(1)
    DRIFT_ROPE3D_CASE(2)
    DRIFT_ROPE3D_CASE(4)
    DRIFT_ROPE3D_CASE(6)
    DRIFT_ROPE3D_CASE(8)
    DRIFT_ROPE3D_CASE(12)
    DRIFT_ROPE3D_CASE(16)
#undef DRIFT_ROPE3D_CASE
  }
  const dim3 grid(grid_for(tokens, 1, 1 << 16));
  if (chunked)
    hipLaunchKernelGGL((rope_3d_kernel<T, true>), grid, dim3(256), 0, st, x, out, p);
  else
    hipLaunchKernelGGL((rope_3d_kernel<T, false>), grid, dim3(256), 0, st, x, out, p);
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
  constexpr int N = Chunk<T>::N;
  const int lanes_per_head = dim / (2 * N);
  const bool whole = rotary == dim && dim % (2 * N) == 0 && (lanes_per_head & (lanes_per_head - 1)) == 0 &&
                     lanes_per_head <= kWave / 2 && (!q || (aligned16(q) && aligned16(q_out))) &&
                     (!k || (aligned16(k) && aligned16(k_out)));
  const dim3 grid(grid_for(tokens, 1, 1 << 16));
  const hipStream_t st = (hipStream_t)stream;
  if (whole) {
    const int heads_per_wave = kWave / lanes_per_head;
    // a wave per 64 / G heads, and a thread per weight of a head
    const int waves = (int)std::min<int64_t>(
        kQkMaxWaves, std::max<int64_t>(ceil_div(heads + kv_heads, heads_per_wave), ceil_div(dim, kWave)));
    const dim3 block(64 * waves);
    switch (lanes_per_head) {
#define DRIFT_QK_CASE(G)                                                                                         \
  case G:                                                                                                        \
    if (layout == DRIFT_ROPE_NEOX)                                                                               \
      hipLaunchKernelGGL((qk_norm_rope_token<T, G, true>), dim3(tokens), block, 0, st, q, k, q_out, k_out,       \
                         q_weight, k_weight, positions, a);                                                      \
    else                                                                                                         \
      hipLaunchKernelGGL((qk_norm_rope_token<T, G, false>), dim3(tokens), block, 0, st, q, k, q_out, k_out,      \
                         q_weight, k_weight, positions, a);                                                      \
    break;
      DRIFT_QK_CASE(1)
      DRIFT_QK_CASE(2)
      DRIFT_QK_CASE(4)
      DRIFT_QK_CASE(8)
      DRIFT_QK_CASE(16)
      DRIFT_QK_CASE(32)
#undef DRIFT_QK_CASE
      default:
        return refuse("%s: no kernel for heads of %d values", entry, dim);
    }
  } else {
    hipLaunchKernelGGL(qk_norm_rope_kernel<T>, grid, dim3(256), 0, st, q, k, q_out, k_out, q_weight, k_weight,
                       positions, a);
  }
  return launched(entry);
}

}  // namespace
}  // namespace drift

using namespace drift;

extern "C" int drift_rope_f32(const float* x, const int32_t* positions, float* out, int32_t tokens, int32_t heads,
                              int32_t head_dim, int32_t rotary, float theta, int32_t layout, int32_t sections,
                              int32_t s0, int32_t s1, int32_t s2, int32_t s3, void* stream) {
  return rope<float>("drift_rope_f32", x, positions, out, tokens, heads, head_dim, rotary, theta, layout, sections,
                     s0, s1, s2, s3, stream);
}

extern "C" int drift_rope_bf16(const uint16_t* x, const int32_t* positions, uint16_t* out, int32_t tokens,
                               int32_t heads, int32_t head_dim, int32_t rotary, float theta, int32_t layout,
                               int32_t sections, int32_t s0, int32_t s1, int32_t s2, int32_t s3, void* stream) {
  return rope<uint16_t>("drift_rope_bf16", x, positions, out, tokens, heads, head_dim, rotary, theta, layout,
                        sections, s0, s1, s2, s3, stream);
}

extern "C" int drift_rope_table_f32(const float* x, const float* cosines, const float* sines, float* out,
                                    int32_t tokens, int32_t heads, int32_t head_dim, int32_t pairs, int32_t per_head,
                                    int32_t halves, void* stream) {
  return rope_table<float>("drift_rope_table_f32", x, cosines, sines, out, tokens, heads, head_dim, pairs, per_head,
                           halves, stream);
}

extern "C" int drift_rope_table_bf16(const uint16_t* x, const float* cosines, const float* sines, uint16_t* out,
                                     int32_t tokens, int32_t heads, int32_t head_dim, int32_t pairs,
                                     int32_t per_head, int32_t halves, void* stream) {
  return rope_table<uint16_t>("drift_rope_table_bf16", x, cosines, sines, out, tokens, heads, head_dim, pairs,
                              per_head, halves, stream);
}

extern "C" int drift_rope_3d_f32(const float* x, float* out, int64_t tokens, int32_t heads, int32_t head_dim,
                                 int32_t frames, int32_t grid_rows, int32_t grid_cols, int64_t token_offset,
                                 double theta, void* stream) {
  return rope_3d<float>("drift_rope_3d_f32", x, out, tokens, heads, head_dim, frames, grid_rows, grid_cols,
                        token_offset, theta, stream);
}

extern "C" int drift_rope_3d_bf16(const uint16_t* x, uint16_t* out, int64_t tokens, int32_t heads,
                                  int32_t head_dim, int32_t frames, int32_t grid_rows, int32_t grid_cols,
                                  int64_t token_offset, double theta, void* stream) {
  return rope_3d<uint16_t>("drift_rope_3d_bf16", x, out, tokens, heads, head_dim, frames, grid_rows, grid_cols,
                           token_offset, theta, stream);
}

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
