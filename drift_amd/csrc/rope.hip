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
#include "rope.hpp"

#include <algorithm>
#include <climits>

namespace drift {
namespace {

// ------------------------------------------------------------------ rope

// Chunked turn of a head: lane items are chunk pairs. NeoX: chunk i (< half/N)
// with chunk i + half/N; interleaved: one chunk, its N/2 pairs inside. Tail
// chunks (from rotary on) are copied.
template <typename T>
__device__ __forceinline__ void turn_chunks(const T* xh, T* oh, int item, int rotary, int layout, const double2* cs) {
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
        turn_chunks<T>(xh, oh, j, p.rotary, p.layout, cs);
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
        turn_chunks<T>(xh, oh, j, p.dim, DRIFT_ROPE_INTERLEAVED, cs);
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

// ------------------------------------------------------------------ launch layer

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
