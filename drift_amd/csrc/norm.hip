// Row-wise norms for gfx950: RMSNorm (with the residual add), LayerNorm,
// AdaLN (LayerNorm then per-sample modulation, one pass) and modulate.
//
// Layout: row-major [rows, cols]. A row belongs to one wave (or to a group of
// four waves when it is long and rows are few), each lane holding K 16-byte
// chunks of it in registers, so the row crosses HBM once each way. Chunk k of
// lane l is chunk (k * W + wave) * 64 + l of the row: every load and store
// instruction of a wave covers 1 KiB of contiguous memory.
//
// Arithmetic is the runner's CPU reference's (ops/CpuNormalisation.scala:53-71,
// :128-151, ops/CpuElementwise.scala:33-38): sums, factor and every output in
// double, rounded once to float (then to bf16). CDNA4 runs double at the same
// vector rate as unpacked float, so this costs no more than float math and
// the results match the reference to the last bit but for sums taken in
// another order.
#include "common.hpp"

#include <algorithm>
#include <atomic>
#include <climits>

namespace drift {
namespace {

// The sum over a row's group of W waves (W = 1 or 4), the same in every lane.
template <int W>
__device__ __forceinline__ double row_sum(double v, double* partial) {
  v = group_sum<64>(v);
  if constexpr (W > 1) {
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) partial[wave] = v;
    __syncthreads();
    v = partial[0];
#pragma unroll
    for (int w = 1; w < W; ++w) v += partial[w];
    __syncthreads();  // partial is reused by the next sum
  }
  return v;
}

// Four or eight consecutive F32 weights, as the chunk of type T they pair with.
template <int N>
__device__ __forceinline__ void load_f32(const float* p, float (&v)[N]) {
#pragma unroll
  for (int j = 0; j < N; j += 4) {
    const float4 q = *reinterpret_cast<const float4*>(p + j);
    v[j] = q.x;
    v[j + 1] = q.y;
    v[j + 2] = q.z;
    v[j + 3] = q.w;
  }
}

// ------------------------------------------------------------------ RMSNorm

// A chunk's squares, summed in order in double. A row's sum of squares is
// taken as: per lane, its chunks' sums in increasing chunk order, then over
// the wave, then over the row's waves in order; with four waves a row, wave s
// holding the lane's chunks 64 * (4m + s) + lane. rms_norm_rows and
// rms_norm_wide keep that order, so a row norms the same in either.
template <int N>
__device__ __forceinline__ double chunk_squares(const float (&v)[N]) {
  double p = 0.0;
#pragma unroll
  for (int j = 0; j < N; ++j) p += (double)v[j] * (double)v[j];
  return p;
}

// With q.xq, out is quantized too as it is written (quantize_chunk; cols a
// multiple of 32, so a row holds whole blocks).
template <typename T, int K, int W>
__global__ void __launch_bounds__(256) rms_norm_rows(T* x, const T* y, const float* weight, T* out, int64_t rows,
                                                     int cols, float eps, float offset, int weight_rows,
                                                     Quantized q) {
  constexpr int N = Chunk<T>::N;
  constexpr int kRowsPerBlock = 4 / W;
  __shared__ double partial[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = wave % W;
  const int chunks = cols / N;
  for (int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + wave / W; row < rows;
       row += (int64_t)gridDim.x * kRowsPerBlock) {
    T* xr = x + row * cols;
    const float* w = weight + (row % weight_rows) * cols;
    // Short rows (decode) are latency-bound: their weights are loaded with x,
    // before the sum, so the two loads' latencies overlap.
    constexpr bool kEarlyWeights = K * N <= 16;
    float early[kEarlyWeights ? K : 1][N];
    if constexpr (kEarlyWeights) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int c = (k * W + sub) * kWave + lane;
        if (c < chunks) load_f32<N>(w + c * N, early[k]);
      }
    }
    float v[K][N];
    double squares = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int c = (k * W + sub) * kWave + lane;
      if (c < chunks) {
        Chunk<T>::load(xr + c * N, v[k]);
        if (y) {
          float u[N];
          Chunk<T>::load(y + row * cols + c * N, u);
#pragma unroll
          for (int j = 0; j < N; ++j) v[k][j] += u[j];  // the F32 sum, as add() rounds it
        }
        squares += chunk_squares(v[k]);
      }
    }
    squares = row_sum<W>(squares, partial);
    const double factor = 1.0 / sqrt(squares / (double)cols + (double)eps);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int c = (k * W + sub) * kWave + lane;
      if (c < chunks) {
        if (y) Chunk<T>::store(xr + c * N, v[k]);  // the residual stream, before out (which may be x)
        float wv[N], o[N];
        if constexpr (kEarlyWeights) {
#pragma unroll
          for (int j = 0; j < N; ++j) wv[j] = early[k][j];
        } else {
          load_f32<N>(w + c * N, wv);
        }
#pragma unroll
        for (int j = 0; j < N; ++j) o[j] = (float)((double)v[k][j] * factor * ((double)wv[j] + (double)offset));
        Chunk<T>::store(out + row * cols + c * N, o);
        if (q.xq) {
          as_written<T>(o);
          quantize_chunk<N>(o, (row * cols + c * N) / 32, q);
        }
      }
    }
  }
}

// Few rows (a decode step's tokens): a row's chunks spread over W = 8 or 16
// waves (512 or 1024 threads), so each lane's serial work is 2 or 4 times
// shorter than in the four-wave group. The chunks' sums of squares go through
// LDS to the first four waves, which add them in the four-wave group's order
// (chunk_squares), so the result is the same to the last bit.
template <typename T, int K, int W>
__global__ void __launch_bounds__(64 * W) rms_norm_wide(T* x, const T* y, const float* weight, T* out, int64_t rows,
                                                       int cols, float eps, float offset, int weight_rows,
                                                       Quantized q) {
  static_assert(W == 8 || W == 16, "the wide group is 8 or 16 waves");
  constexpr int N = Chunk<T>::N;
  constexpr int kSlots = K * W;  // 64-chunk slots a row can have
  __shared__ double sums[kSlots][kWave];
  __shared__ double partial[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int chunks = cols / N;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    T* xr = x + row * cols;
    const float* w = weight + (row % weight_rows) * cols;
    float wv[K][N];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int c = (k * W + wave) * kWave + lane;
      if (c < chunks) load_f32<N>(w + c * N, wv[k]);
    }
    float v[K][N];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int slot = k * W + wave, c = slot * kWave + lane;
      if (c < chunks) {
        Chunk<T>::load(xr + c * N, v[k]);
        if (y) {
          float u[N];
          Chunk<T>::load(y + row * cols + c * N, u);
#pragma unroll
          for (int j = 0; j < N; ++j) v[k][j] += u[j];
        }
        sums[slot][lane] = chunk_squares(v[k]);
      }
    }
    __syncthreads();
    if (wave < 4) {
      double squares = 0.0;
#pragma unroll
      for (int m = 0; m < kSlots / 4; ++m) {
        const int slot = 4 * m + wave;
        if (slot * kWave + lane < chunks) squares += sums[slot][lane];
      }
      squares = group_sum<64>(squares);
      if (lane == 0) partial[wave] = squares;
    }
    __syncthreads();
    const double total = ((partial[0] + partial[1]) + partial[2]) + partial[3];
    const double factor = 1.0 / sqrt(total / (double)cols + (double)eps);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int c = (k * W + wave) * kWave + lane;
      if (c < chunks) {
        if (y) Chunk<T>::store(xr + c * N, v[k]);
        float o[N];
#pragma unroll
        for (int j = 0; j < N; ++j) o[j] = (float)((double)v[k][j] * factor * ((double)wv[k][j] + (double)offset));
        Chunk<T>::store(out + row * cols + c * N, o);
        if (q.xq) {
          as_written<T>(o);
          quantize_chunk<N>(o, (row * cols + c * N) / 32, q);
        }
      }
    }
    __syncthreads();  // sums and partial are reused by the next row
  }
}

// Any width and alignment: a block of 256 per row, reading the row twice.
template <typename T>
__global__ void __launch_bounds__(256) rms_norm_rows_scalar(T* x, const T* y, const float* weight, T* out,
                                                            int64_t rows, int cols, float eps, float offset,
                                                            int weight_rows) {
  __shared__ double partial[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    T* xr = x + row * cols;
    const T* yr = y ? y + row * cols : nullptr;
    double squares = 0.0;
    for (int c = threadIdx.x; c < cols; c += 256) {
      float v = load_one(xr + c);
      if (yr) v += load_one(yr + c);
      squares += (double)v * (double)v;
    }
    squares = row_sum<4>(squares, partial);
    const double factor = 1.0 / sqrt(squares / (double)cols + (double)eps);
    const float* w = weight + (row % weight_rows) * cols;
    for (int c = threadIdx.x; c < cols; c += 256) {
      float v = load_one(xr + c);
      if (yr) {
        v += load_one(yr + c);
        store_one(xr + c, v);
      }
      store_one(out + row * cols + c, (float)((double)v * factor * ((double)w[c] + (double)offset)));
    }
  }
}

// Narrow rows (at most 32 values, a pixel's channels, often millions of
// rows): a thread per row, as the reference's rms_norm_narrow_f32
// (kernels/norm.hip:414-426). The sum runs over the row in order, as the
// CPU's left fold does, so the result is the CPU's to the last bit.
constexpr int kNarrowCols = 32;

template <typename T>
__global__ void __launch_bounds__(256) rms_norm_narrow(T* x, const T* y, const float* weight, T* out, int64_t rows,
                                                       int cols, float eps, float offset, int weight_rows) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; row < rows; row += stride) {
    T* xr = x + row * cols;
    const T* yr = y ? y + row * cols : nullptr;
    float v[kNarrowCols];
    double squares = 0.0;
#pragma unroll
    for (int c = 0; c < kNarrowCols; ++c) {
      if (c < cols) {
        v[c] = load_one(xr + c);
        if (yr) v[c] += load_one(yr + c);
        squares += (double)v[c] * (double)v[c];
      }
    }
    const double factor = 1.0 / sqrt(squares / (double)cols + (double)eps);
    const float* w = weight + (row % weight_rows) * cols;
#pragma unroll
    for (int c = 0; c < kNarrowCols; ++c) {
      if (c < cols) {
        if (yr) store_one(xr + c, v[c]);
        store_one(out + row * cols + c, (float)((double)v[c] * factor * ((double)w[c] + (double)offset)));
      }
    }
  }
}

// ------------------------------------------------------------------ LayerNorm / AdaLN

// MODULATE false: out = normal * (weight or 1) + (bias or 0).
// MODULATE true: n = float(normal + 0) (layerNorm's F32 result, no affine),
// out = n * (1 + scale[s, c]) + shift[s, c], s the row's sample.
template <typename T, int K, int W, bool MODULATE>
__global__ void __launch_bounds__(256) layer_norm_rows(const T* x, const float* weight, const float* bias, T* out,
                                                       int64_t rows, int cols, int64_t rows_per_sample, float eps) {
  constexpr int N = Chunk<T>::N;
  constexpr int kRowsPerBlock = 4 / W;
  __shared__ double partial[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = wave % W;
  const int chunks = cols / N;
  for (int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + wave / W; row < rows;
       row += (int64_t)gridDim.x * kRowsPerBlock) {
    float v[K][N];
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int c = (k * W + sub) * kWave + lane;
      if (c < chunks) {
        Chunk<T>::load(x + row * cols + c * N, v[k]);
#pragma unroll
        for (int j = 0; j < N; ++j) sum += (double)v[k][j];
      }
    }
    const double mean = row_sum<W>(sum, partial) / (double)cols;
    double squares = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int c = (k * W + sub) * kWave + lane;
      if (c < chunks) {
#pragma unroll
        for (int j = 0; j < N; ++j) {
          const double d = (double)v[k][j] - mean;
          squares += d * d;
        }
      }
    }
    const double factor = 1.0 / sqrt(row_sum<W>(squares, partial) / (double)cols + (double)eps);
    const float* s0 = weight;  // MODULATE: the sample's scale row
    const float* s1 = bias;    // MODULATE: the sample's shift row
    if constexpr (MODULATE) {
      const int64_t sample = row / rows_per_sample;
      s0 = weight + sample * cols;
      s1 = bias + sample * cols;
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int c = (k * W + sub) * kWave + lane;
      if (c < chunks) {
        float o[N];
        if constexpr (MODULATE) {
          float sc[N], sh[N];
          load_f32<N>(s0 + c * N, sc);
          load_f32<N>(s1 + c * N, sh);
#pragma unroll
          for (int j = 0; j < N; ++j) {
            const float n = (float)fma((double)v[k][j] - mean, factor, 0.0);
            o[j] = (float)fma((double)n, 1.0 + (double)sc[j], (double)sh[j]);
          }
        } else {
          float wv[N], bv[N];
          if (s0) load_f32<N>(s0 + c * N, wv);
          if (s1) load_f32<N>(s1 + c * N, bv);
#pragma unroll
          for (int j = 0; j < N; ++j) {
            const double normal = ((double)v[k][j] - mean) * factor;
            o[j] = (float)(normal * (s0 ? (double)wv[j] : 1.0) + (s1 ? (double)bv[j] : 0.0));
          }
        }
        Chunk<T>::store(out + row * cols + c * N, o);
      }
    }
  }
}

template <typename T, bool MODULATE>
__global__ void __launch_bounds__(256) layer_norm_rows_scalar(const T* x, const float* weight, const float* bias,
                                                              T* out, int64_t rows, int cols,
                                                              int64_t rows_per_sample, float eps) {
  __shared__ double partial[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const T* xr = x + row * cols;
    double sum = 0.0;
    for (int c = threadIdx.x; c < cols; c += 256) sum += (double)load_one(xr + c);
    const double mean = row_sum<4>(sum, partial) / (double)cols;
    double squares = 0.0;
    for (int c = threadIdx.x; c < cols; c += 256) {
      const double d = (double)load_one(xr + c) - mean;
      squares += d * d;
    }
    const double factor = 1.0 / sqrt(row_sum<4>(squares, partial) / (double)cols + (double)eps);
    const float* s0 = weight;
    const float* s1 = bias;
    if constexpr (MODULATE) {
      const int64_t sample = row / rows_per_sample;
      s0 = weight + sample * cols;
      s1 = bias + sample * cols;
    }
    for (int c = threadIdx.x; c < cols; c += 256) {
      const double d = (double)load_one(xr + c) - mean;
      float o;
      if constexpr (MODULATE) {
        const float n = (float)fma(d, factor, 0.0);
        o = (float)fma((double)n, 1.0 + (double)s0[c], (double)s1[c]);
      } else {
        o = (float)(d * factor * (s0 ? (double)s0[c] : 1.0) + (s1 ? (double)s1[c] : 0.0));
      }
      store_one(out + row * cols + c, o);
    }
  }
}

// F32 AdaLN, one wave per row, four rows of one sample per block (grid.y =
// sample), the grid covering the rows in one pass. Each lane reads its
// chunks' scale and shift from the sample's rows (cached: every row of the
// sample reads them).
//
// The mean and variance come from one pass over the row about its first
// value x0 (sums of d = x - x0 and d^2): the same as the reference's two
// passes to the last bits, since |mean - x0| is a few standard deviations at
// most. The arithmetic is the reference's, in double: n = float((x - mean) *
// factor) is layerNorm's F32 result, out = n * (1 + scale) + shift rounded
// once, as modulate.
constexpr int kAdalnMaxCols = 4096;

template <typename T, int K, bool FULL>
__global__ void __launch_bounds__(256) adaln_waves(const T* x, const float* scale, const float* shift, T* out,
                                                    int64_t rows, int cols, int64_t rows_per_sample, float eps) {
  constexpr int N = Chunk<T>::N;
  using Raw = typename Chunk<T>::Raw;
  const int chunks = FULL ? K * kWave : cols / N;
  const int64_t sample = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = sample * rows_per_sample + (int64_t)blockIdx.x * 4 + wave;
  if (row >= min(rows, (sample + 1) * rows_per_sample)) return;
  Raw raw[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int c = k * kWave + lane;
    if (FULL || c < chunks) raw[k] = Chunk<T>::load_raw(x + row * cols + c * N);
  }
  float first_value[N];
  Chunk<T>::unpack(raw[0], first_value);
  const double x0 = (double)__shfl(first_value[0], 0);
  double s1 = 0.0, s2 = 0.0;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    if (FULL || k * kWave + lane < chunks) {
      float v[N];
      Chunk<T>::unpack(raw[k], v);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const double d = (double)v[j] - x0;
        s1 += d;
        s2 = fma(d, d, s2);
      }
    }
  }
  s1 = group_sum<64>(s1);
  s2 = group_sum<64>(s2);
  const double m1 = s1 / (double)cols;  // mean - x0
  const double mean = x0 + m1;
  const double variance = fmax(s2 / (double)cols - m1 * m1, 0.0);
  const double factor = 1.0 / sqrt(variance + (double)eps);
  const double offset = -mean * factor;
  const float* sc = scale + sample * cols;
  const float* sh = shift + sample * cols;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int c = k * kWave + lane;
    if (FULL || c < chunks) {
      float v[N], o[N], a[N], b[N];
      Chunk<T>::unpack(raw[k], v);
      load_f32<N>(sc + c * N, a);
      load_f32<N>(sh + c * N, b);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const float n = (float)fma((double)v[j], factor, offset);
        o[j] = (float)fma((double)n, 1.0 + (double)a[j], (double)b[j]);
      }
      Chunk<T>::store(out + row * cols + c * N, o);
    }
  }
}

// BF16 AdaLN with each lane's (1 + scale, shift) held in registers across the
// rows it takes: re-reading them per row would move four times the row's own
// bytes through the L1. Wave w of a sample takes rows w, w + W, w + 2W, ... of
// it (W waves per sample, all resident at once), with the next row's loads in
// flight while it computes the current one.
//
// The arithmetic is adaln_waves', in double. It has to be: where the output
// nearly cancels (n * (1 + scale) ~ -shift) a float ulp of n or of 1 + scale
// is many bf16 ulps of the result. d = x - x0 is exact in float for bf16
// values within a factor 2^15 of each other, and d^2 exact in double.
template <int K, bool FULL>
__global__ void __launch_bounds__(256) adaln_resident(const uint16_t* x, const float* scale, const float* shift,
                                                      uint16_t* out, int64_t rows, int cols, int64_t rows_per_sample,
                                                      float eps, int64_t waves_per_sample) {
  constexpr int N = 8;
  using Raw = uint4;
  const int chunks = FULL ? K * kWave : cols / N;
  const int64_t sample = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t end = min(rows, (sample + 1) * rows_per_sample);
  int64_t row = sample * rows_per_sample + w;
  if (w >= waves_per_sample || row >= end) return;
  auto load_row = [&](int64_t r, Raw(&into)[K]) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int c = k * kWave + lane;
      if (FULL || c < chunks) into[k] = Chunk<uint16_t>::load_raw(x + r * cols + c * N);
    }
  };
  Raw raw[K];
  load_row(row, raw);
  double a[K][N];
  float b[K][N];
  const float* sc = scale + sample * cols;
  const float* sh = shift + sample * cols;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int c = k * kWave + lane;
    if (FULL || c < chunks) {
      float f[N];
      load_f32<N>(sc + c * N, f);
      load_f32<N>(sh + c * N, b[k]);
#pragma unroll
      for (int j = 0; j < N; ++j) a[k][j] = 1.0 + (double)f[j];
    }
  }
  const double inverse_cols = 1.0 / (double)cols;
  for (; row < end; row += waves_per_sample) {
    Raw next[K];
    if (row + waves_per_sample < end) load_row(row + waves_per_sample, next);
    float first_value[N];
    Chunk<uint16_t>::unpack(raw[0], first_value);
    const float x0 = __shfl(first_value[0], 0);
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (FULL || k * kWave + lane < chunks) {
        float v[N];
        Chunk<uint16_t>::unpack(raw[k], v);
#pragma unroll
        for (int j = 0; j < N; ++j) {
          const double d = (double)(v[j] - x0);
          s1 += d;
          s2 = fma(d, d, s2);
        }
      }
    }
    s1 = group_sum<64>(s1);
    s2 = group_sum<64>(s2);
    // the row's statistics are a chain the wave waits on, alone on its
    // SIMD: the width's reciprocal (made once) for the two divisions, and
    // 1/sqrt by the hardware's reciprocal root refined, not a root and a
    // division (each within a double ulp or two)
    const double m1 = s1 * inverse_cols;  // mean - x0
    const double mean = (double)x0 + m1;
    const double variance = fmax(fma(s2, inverse_cols, -(m1 * m1)), 0.0);
    const double factor = eps > 0.0f ? inverse_sqrt<true>(variance + (double)eps) : inverse_sqrt(variance + (double)eps);
    const double offset = -mean * factor;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int c = k * kWave + lane;
      if (FULL || c < chunks) {
        opaque(raw[k]);
        float v[N], o[N];
        Chunk<uint16_t>::unpack(raw[k], v);
#pragma unroll
        for (int j = 0; j < N; ++j) {
          const float n = (float)fma((double)v[j], factor, offset);
          o[j] = (float)fma((double)n, a[k][j], (double)b[k][j]);
        }
        Chunk<uint16_t>::store(out + row * cols + c * N, o);
      }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) raw[k] = next[k];
  }
}

// ------------------------------------------------------------------ modulate

template <typename T>
__global__ void __launch_bounds__(256) modulate_elements(const T* x, const float* scale, const float* shift, T* out,
                                                         int64_t n, int cols) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int c = (int)(i % cols);
    store_one(out + i, (float)fma((double)load_one(x + i), 1.0 + (double)scale[c], (double)shift[c]));
  }
}

template <typename T>
__global__ void __launch_bounds__(256) modulate_chunks(const T* x, const float* scale, const float* shift, T* out,
                                                       int64_t chunks, int cols) {
  constexpr int N = Chunk<T>::N;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < chunks; i += stride) {
    const int c = (int)((i * N) % cols);
    float v[N], sc[N], sh[N], o[N];
    Chunk<T>::load(x + i * N, v);
    load_f32<N>(scale + c, sc);
    load_f32<N>(shift + c, sh);
#pragma unroll
    for (int j = 0; j < N; ++j) o[j] = (float)fma((double)v[j], 1.0 + (double)sc[j], (double)sh[j]);
    Chunk<T>::store(out + i * N, o);
  }
}

// ------------------------------------------------------------------ launch layer

// How a row is split: W waves per row, K chunks per lane; K = 0 means the
// scalar path.
struct RowPlan {
  int waves = 1;
  int per_lane = 0;
};

template <typename T>
RowPlan plan_rows(int64_t rows, int cols, bool vector_ok) {
  constexpr int N = Chunk<T>::N;
  RowPlan plan;
  if (!vector_ok || cols % N != 0) return plan;
  const int chunks = cols / N;
  // long rows: a 4-wave group per row shortens each lane's chain. The split
  // depends on the row's width only, never on how many rows come with it, so
  // a row's sum is taken in the same order (and is the same to the last bit)
  // whether it is normed alone, as a decode step's token, or in a batch
  plan.waves = chunks >= 4 * kWave ? 4 : 1;
  (void)rows;
  const int per_lane = (int)ceil_div(chunks, kWave * plan.waves);
  static const int kSteps[] = {1, 2, 3, 4, 6, 8, 12, 16};
  for (int k : kSteps)
    if (per_lane <= k) {
      plan.per_lane = k;
      break;
    }
  return plan;
}

#define DRIFT_ROW_CASES(MACRO) \
  MACRO(1)                     \
  MACRO(2)                     \
  MACRO(3)                     \
  MACRO(4)                     \
  MACRO(6)                     \
  MACRO(8)                     \
  MACRO(12)                    \
  MACRO(16)

// Rows for rms_norm_wide: a few (at most one a CU) long rows, spread over 8
// waves (one or two chunks a lane) or 16 (one to four). 0: the four-wave
// group (or one wave) of plan_rows.
constexpr int64_t kWideRows = 256;

template <typename T>
int wide_waves(int64_t rows, int cols, const RowPlan& plan) {
  const int chunks = cols / Chunk<T>::N;
  if (plan.waves != 4 || rows > kWideRows || rows < 1) return 0;
  if (chunks >= 16 * kWave && chunks <= 4 * 16 * kWave) return 16;
  if (chunks >= 8 * kWave && chunks < 16 * kWave) return 8;
  return 0;
}

template <typename T>
int rms_norm(const char* entry, T* x, const T* y, const float* weight, T* out, int64_t rows, int32_t cols, float eps,
             float offset, int32_t weight_rows, Quantized q, void* stream) {
  clear_error();
  if (rows < 0) return refuse("%s: %lld rows", entry, (long long)rows);
  if (cols <= 0) return refuse("%s: rows of %d values", entry, cols);
  if (weight_rows <= 0) return refuse("%s: %d weight rows", entry, weight_rows);
  if (q.xq && cols % 32 != 0) return refuse("%s: rows of %d values are not whole blocks of 32 to quantize", entry, cols);
  if (const int bad = check_quantized(entry, q, rows * cols)) return bad;
  if (rows == 0) return 0;
  if (!x || !weight || !out) return refuse("%s: null x, weight or out", entry);
  const hipStream_t s = (hipStream_t)stream;
  const bool vector_ok = aligned16(x) && aligned16(out) && aligned16(weight) && (!y || aligned16(y));
  const RowPlan plan = plan_rows<T>(rows, cols, vector_ok);
  // the side output is written by the norm when its chunks can store the
  // codes, else by a quantize_x launch over out right after
  const bool fused = q.xq && plan.per_lane > 0 && codes_storable(q.xq, Chunk<T>::N);
  const Quantized in_kernel = fused ? q : Quantized{nullptr, nullptr, nullptr};
  if (cols <= kNarrowCols && !q.xq) {
    hipLaunchKernelGGL(rms_norm_narrow<T>, dim3(grid_for(rows, 256)), dim3(256), 0, s, x, y, weight, out, rows,
                       (int)cols, eps, offset, (int)weight_rows);
  } else if (plan.per_lane == 0) {
    hipLaunchKernelGGL(rms_norm_rows_scalar<T>, dim3(grid_for(rows, 1)), dim3(256), 0, s, x, y, weight, out, rows,
                       (int)cols, eps, offset, (int)weight_rows);
  } else if (const int wide = wide_waves<T>(rows, cols, plan)) {
    const int per_lane = (int)ceil_div(cols / Chunk<T>::N, kWave * wide);
    const dim3 grid((unsigned)rows), block(kWave * wide);
    if (wide == 8 && per_lane == 1)
      hipLaunchKernelGGL((rms_norm_wide<T, 1, 8>), grid, block, 0, s, x, y, weight, out, rows, cols, eps, offset,
                         weight_rows, in_kernel);
    else if (wide == 8)
      hipLaunchKernelGGL((rms_norm_wide<T, 2, 8>), grid, block, 0, s, x, y, weight, out, rows, cols, eps, offset,
                         weight_rows, in_kernel);
    else if (per_lane == 1)
      hipLaunchKernelGGL((rms_norm_wide<T, 1, 16>), grid, block, 0, s, x, y, weight, out, rows, cols, eps, offset,
                         weight_rows, in_kernel);
    else if (per_lane == 2)
      hipLaunchKernelGGL((rms_norm_wide<T, 2, 16>), grid, block, 0, s, x, y, weight, out, rows, cols, eps, offset,
                         weight_rows, in_kernel);
    else if (per_lane == 3)
      hipLaunchKernelGGL((rms_norm_wide<T, 3, 16>), grid, block, 0, s, x, y, weight, out, rows, cols, eps, offset,
                         weight_rows, in_kernel);
    else
      hipLaunchKernelGGL((rms_norm_wide<T, 4, 16>), grid, block, 0, s, x, y, weight, out, rows, cols, eps, offset,
                         weight_rows, in_kernel);
  } else {
    const unsigned grid = grid_for(rows, 4 / plan.waves);
#define DRIFT_RMS_CASE(K)                                                                                     \
  case K:                                                                                                     \
    if (plan.waves == 1)                                                                                      \
      hipLaunchKernelGGL((rms_norm_rows<T, K, 1>), dim3(grid), dim3(256), 0, s, x, y, weight, out, rows,     \
                         cols, eps, offset, weight_rows, in_kernel);                                          \
    else                                                                                                      \
      hipLaunchKernelGGL((rms_norm_rows<T, K, 4>), dim3(grid), dim3(256), 0, s, x, y, weight, out, rows,     \
                         cols, eps, offset, weight_rows, in_kernel);                                          \
    break;
    switch (plan.per_lane) { DRIFT_ROW_CASES(DRIFT_RMS_CASE) }
#undef DRIFT_RMS_CASE
  }
  if (q.xq && !fused) {
    if (const int status = launched(entry)) return status;
    launch_quantize(out, q, rows * cols / 32, s);
  }
  return launched(entry);
}

// Waves of `kernel` (256-thread blocks) the device holds at once.
template <typename Kernel>
int64_t resident_waves(Kernel kernel) {
  int device = 0, cus = 0, blocks = 0;
  if (hipGetDevice(&device) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, 256, 0) != hipSuccess)
    return 0;
  return (int64_t)cus * blocks * 4;
}

template <int K, bool FULL>
void adaln_resident_launch(const uint16_t* x, const float* scale, const float* shift, uint16_t* out, int64_t rows,
                           int cols, int64_t rows_per_sample, int64_t samples, float eps, hipStream_t s) {
  // every wave resident at once, rows shared out as evenly as they go; the
  // residency is the current device's, found once per device
  constexpr int kDevices = 64;
  static std::atomic<int64_t> budget[kDevices] = {};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kDevices) device = 0;
  int64_t waves = budget[device].load(std::memory_order_relaxed);
  if (waves == 0) {
    waves = std::max<int64_t>(resident_waves(adaln_resident<K, FULL>), 4);
    budget[device].store(waves, std::memory_order_relaxed);
  }
  int64_t per_sample = std::max<int64_t>(1, std::min(rows_per_sample, waves / samples));
  per_sample = ceil_div(rows_per_sample, ceil_div(rows_per_sample, per_sample));
  const dim3 grid((unsigned)ceil_div(per_sample, 4), (unsigned)samples);
  hipLaunchKernelGGL((adaln_resident<K, FULL>), grid, dim3(256), 0, s, x, scale, shift, out, rows, cols,
                     rows_per_sample, eps, per_sample);
}

// AdaLN: BF16 through adaln_resident, F32 through adaln_waves; rows of whole
// 16-byte chunks, at most 4096 values. Returns -1 when the shape does not
// qualify.
template <typename T>
int adaln_launch(const T* x, const float* scale, const float* shift, T* out, int64_t rows, int cols,
                 int64_t rows_per_sample, float eps, hipStream_t s) {
  constexpr int N = Chunk<T>::N;
  const int64_t samples = ceil_div(rows, rows_per_sample);
  if (cols % N != 0 || cols > kAdalnMaxCols || samples > 65535 || ceil_div(rows_per_sample, 4) >= INT32_MAX)
    return -1;
  const int chunks = cols / N;
  const int per_lane = (int)ceil_div(chunks, kWave);
  if constexpr (sizeof(T) == 2) {
#define DRIFT_ADALN_CASE(K)                                                                                   \
  if (per_lane <= K) {                                                                                        \
    if (chunks == K * kWave)                                                                                  \
      adaln_resident_launch<K, true>(x, scale, shift, out, rows, cols, rows_per_sample, samples, eps, s);     \
    else                                                                                                      \
      adaln_resident_launch<K, false>(x, scale, shift, out, rows, cols, rows_per_sample, samples, eps, s);    \
    return 0;                                                                                                 \
  }
    DRIFT_ADALN_CASE(1)
    DRIFT_ADALN_CASE(2)
    DRIFT_ADALN_CASE(3)
    DRIFT_ADALN_CASE(4)
    DRIFT_ADALN_CASE(6)
    DRIFT_ADALN_CASE(8)
#undef DRIFT_ADALN_CASE
  } else {
    const dim3 grid((unsigned)ceil_div(rows_per_sample, 4), (unsigned)samples);
#define DRIFT_ADALN_CASE(K)                                                                                  \
  if (per_lane <= K) {                                                                                       \
    if (chunks == K * kWave)                                                                                 \
      hipLaunchKernelGGL((adaln_waves<T, K, true>), grid, dim3(256), 0, s, x, scale, shift, out, rows, cols,  \
                         rows_per_sample, eps);                                                              \
    else                                                                                                     \
      hipLaunchKernelGGL((adaln_waves<T, K, false>), grid, dim3(256), 0, s, x, scale, shift, out, rows, cols, \
                         rows_per_sample, eps);                                                              \
    return 0;                                                                                                \
  }
    DRIFT_ADALN_CASE(1)
    DRIFT_ADALN_CASE(2)
    DRIFT_ADALN_CASE(3)
    DRIFT_ADALN_CASE(4)
    DRIFT_ADALN_CASE(6)
    DRIFT_ADALN_CASE(8)
    DRIFT_ADALN_CASE(12)
    DRIFT_ADALN_CASE(16)
#undef DRIFT_ADALN_CASE
  }
  return -1;
}

template <typename T, bool MODULATE>
int layer_norm(const char* entry, const T* x, const float* weight, const float* bias, T* out, int64_t rows,
               int32_t cols, int64_t rows_per_sample, float eps, void* stream) {
  clear_error();
  if (rows < 0) return refuse("%s: %lld rows", entry, (long long)rows);
  if (cols <= 0) return refuse("%s: rows of %d values", entry, cols);
  if (MODULATE && rows_per_sample <= 0) return refuse("%s: %lld rows per sample", entry, (long long)rows_per_sample);
  if (rows == 0) return 0;
  if (!x || !out) return refuse("%s: null x or out", entry);
  if (MODULATE && (!weight || !bias)) return refuse("%s: null scale or shift", entry);
  const hipStream_t s = (hipStream_t)stream;
  const bool vector_ok =
      aligned16(x) && aligned16(out) && (!weight || aligned16(weight)) && (!bias || aligned16(bias));
  if (MODULATE && vector_ok && adaln_launch<T>(x, weight, bias, out, rows, cols, rows_per_sample, eps, s) == 0)
    return launched(entry);
  const RowPlan plan = plan_rows<T>(rows, cols, vector_ok);
  if (plan.per_lane == 0) {
    hipLaunchKernelGGL((layer_norm_rows_scalar<T, MODULATE>), dim3(grid_for(rows, 1)), dim3(256), 0, s, x, weight,
                       bias, out, rows, (int)cols, rows_per_sample, eps);
    return launched(entry);
  }
  const unsigned grid = grid_for(rows, 4 / plan.waves);
#define DRIFT_LN_CASE(K)                                                                                     \
  case K:                                                                                                    \
    if (plan.waves == 1)                                                                                     \
      hipLaunchKernelGGL((layer_norm_rows<T, K, 1, MODULATE>), dim3(grid), dim3(256), 0, s, x, weight, bias, \
                         out, rows, cols, rows_per_sample, eps);                                             \
    else                                                                                                     \
      hipLaunchKernelGGL((layer_norm_rows<T, K, 4, MODULATE>), dim3(grid), dim3(256), 0, s, x, weight, bias, \
                         out, rows, cols, rows_per_sample, eps);                                             \
    break;
  switch (plan.per_lane) { DRIFT_ROW_CASES(DRIFT_LN_CASE) }
#undef DRIFT_LN_CASE
  return launched(entry);
}

}  // namespace
}  // namespace drift

using namespace drift;

extern "C" int drift_rms_norm_f32(float* x, const float* y, const float* weight, float* out, int64_t rows,
                                  int32_t cols, float eps, float offset, int32_t weight_rows, int8_t* xq, float* xd,
                                  float* xs, void* stream) {
  return rms_norm<float>("drift_rms_norm_f32", x, y, weight, out, rows, cols, eps, offset, weight_rows,
                         Quantized{xq, xd, xs}, stream);
}

extern "C" int drift_rms_norm_bf16(uint16_t* x, const uint16_t* y, const float* weight, uint16_t* out,
                                   int64_t rows, int32_t cols, float eps, float offset, int32_t weight_rows,
                                   int8_t* xq, float* xd, float* xs, void* stream) {
  return rms_norm<uint16_t>("drift_rms_norm_bf16", x, y, weight, out, rows, cols, eps, offset, weight_rows,
                            Quantized{xq, xd, xs}, stream);
}

extern "C" int drift_layer_norm_f32(const float* x, const float* weight, const float* bias, float* out,
                                    int64_t rows, int32_t cols, float eps, void* stream) {
  return layer_norm<float, false>("drift_layer_norm_f32", x, weight, bias, out, rows, cols, 1, eps, stream);
}

extern "C" int drift_layer_norm_modulate_f32(const float* x, const float* scale, const float* shift, float* out,
                                             int64_t rows, int32_t cols, int64_t rows_per_sample, float eps,
                                             void* stream) {
  return layer_norm<float, true>("drift_layer_norm_modulate_f32", x, scale, shift, out, rows, cols,
                                 rows_per_sample, eps, stream);
}

extern "C" int drift_layer_norm_modulate_bf16(const uint16_t* x, const float* scale, const float* shift,
                                              uint16_t* out, int64_t rows, int32_t cols, int64_t rows_per_sample,
                                              float eps, void* stream) {
  return layer_norm<uint16_t, true>("drift_layer_norm_modulate_bf16", x, scale, shift, out, rows, cols,
                                    rows_per_sample, eps, stream);
}

extern "C" int drift_modulate_f32(const float* x, const float* scale, const float* shift, float* out, int64_t rows,
                                  int32_t cols, void* stream) {
  const char* entry = "drift_modulate_f32";
  clear_error();
  if (rows < 0) return refuse("%s: %lld rows", entry, (long long)rows);
  if (cols <= 0) return refuse("%s: rows of %d values", entry, cols);
  if (rows == 0) return 0;
  if (!x || !scale || !shift || !out) return refuse("%s: null x, scale, shift or out", entry);
  const hipStream_t s = (hipStream_t)stream;
  const int64_t n = rows * cols;
  if (cols % 4 == 0 && aligned16(x) && aligned16(out) && aligned16(scale) && aligned16(shift)) {
    const int64_t chunks = n / 4;
    hipLaunchKernelGGL(modulate_chunks<float>, dim3(grid_for(chunks, 256)), dim3(256), 0, s, x, scale, shift, out,
                       chunks, (int)cols);
  } else {
    hipLaunchKernelGGL(modulate_elements<float>, dim3(grid_for(n, 256)), dim3(256), 0, s, x, scale, shift, out, n,
                       (int)cols);
  }
  return launched(entry);
}
