// The gated residuals and per-row modulations around a diffusion block's
// norms, for gfx950 (kernels/elementwise.hip:105-138; CPU forms
// ops/CpuElementwise.scala:40-86):
//   gatedAdd        x[r][c] += gate[r / rows_per_sample][c] * y[r][c]
//   modulateChunks  out[r][c] = x[r][c] * (1 + t[r][scale][c]) + t[r][shift][c]
//   gatedAddChunk   x[r][c] += t[r][gate][c] * y[r][c]
//   rowGatedAdd     x[r][c] += gate[r] * y[r][c]
// with t [rows][chunks][cols] F32. The reference's gatedAdd takes one gate
// vector for every row (rows_per_sample = rows here); a batch of samples
// passes [samples, cols] gates and runs as one launch.
//
// Arithmetic is the CPU reference's: every value in double, rounded once to
// float (then to bf16). g * y is exact in double, so x + g * y rounds once as
// the reference's double sum does; the modulation rounds 1 + s, the product
// and the sum in double in the reference's order (-ffp-contract=off).
//
// Layout: x, y, out row-major [rows, cols] of T; a lane takes one 16-byte
// chunk (4 F32 or 8 BF16) of the flat tensor and the grid covers it in one
// pass, in one-wave blocks or 512-thread blocks by the op. A chunk's row
// comes from a double multiply by 1 / chunks-per-row, corrected by one step,
// rather than a 64-bit division; gatedAdd takes its row and sample from the
// grid where they fit it.
#include "common.hpp"

#include <initializer_list>

namespace drift {
namespace {

enum Op { GATED_ADD = 0, MODULATE_CHUNKS = 1, GATED_ADD_CHUNK = 2, ROW_GATED_ADD = 3 };

struct RowMap {
  int64_t rows;
  int cols;
  int64_t per;       // gatedAdd: rows per sample
  int chunks;        // tables: chunks per row
  int first;         // gatedAddChunk: gate chunk; modulateChunks: shift chunk
  int second;        // modulateChunks: scale chunk
  int64_t row_chunks;  // 16-byte chunks per row
  double row_inverse;  // 1 / row_chunks
  double per_inverse;  // 1 / per
};

// N consecutive F32 factors. A row's table chunk is read once (streamed); a
// sample's gate row is read by every row of the sample (cached).
template <int N, bool STREAM>
__device__ __forceinline__ void load_floats(const float* p, float (&v)[N]) {
#pragma unroll
  for (int j = 0; j < N; j += 4) {
    const uint4 q = STREAM ? stream_load(p + j) : *reinterpret_cast<const uint4*>(p + j);
    v[j] = __uint_as_float(q.x);
    v[j + 1] = __uint_as_float(q.y);
    v[j + 2] = __uint_as_float(q.z);
    v[j + 3] = __uint_as_float(q.w);
  }
}

// One chunk's operands, loaded: x, y (gated ops), and the F32 factors.
template <typename T, int OP>
struct Operands {
  static constexpr int N = Chunk<T>::N;
  typename Chunk<T>::Raw x, y;
  float a[N], b[N];  // gate, or (scale, shift)

  __device__ __forceinline__ void load(const T* xs, const T* ys, const float* v, const RowMap& m, int64_t i) {
    const int64_t r = quotient(i, m.row_chunks, m.row_inverse);
    load_at(xs, ys, v, m, i, r, (int)(i - r * m.row_chunks) * N, OP == GATED_ADD ? quotient(r, m.per, m.per_inverse) : 0);
  }

  // chunk i, which is value c of row r (of sample `sample`, gatedAdd)
  __device__ __forceinline__ void load_at(const T* xs, const T* ys, const float* v, const RowMap& m, int64_t i,
                                          int64_t r, int c, int64_t sample) {
    x = Chunk<T>::load_raw(xs + i * N);
    if constexpr (OP != MODULATE_CHUNKS) y = Chunk<T>::load_raw(ys + i * N);
    if constexpr (OP == GATED_ADD) {
      load_floats<N, false>(v + sample * m.cols + c, a);
    } else if constexpr (OP == ROW_GATED_ADD) {
      const float g = v[r];
#pragma unroll
      for (int j = 0; j < N; ++j) a[j] = g;
    } else {
      const float* row = v + r * m.chunks * (int64_t)m.cols + c;
      if constexpr (OP == GATED_ADD_CHUNK) {
        load_floats<N, true>(row + (int64_t)m.first * m.cols, a);
      } else {
        load_floats<N, true>(row + (int64_t)m.second * m.cols, a);
        load_floats<N, true>(row + (int64_t)m.first * m.cols, b);
      }
    }
  }

  __device__ __forceinline__ void apply(T* out, int64_t i) const {
    float xv[N], o[N];
    Chunk<T>::unpack(x, xv);
    if constexpr (OP == MODULATE_CHUNKS) {
#pragma unroll
      for (int j = 0; j < N; ++j) o[j] = (float)((double)xv[j] * (1.0 + (double)a[j]) + (double)b[j]);
    } else {
      float yv[N];
      Chunk<T>::unpack(y, yv);
#pragma unroll
      for (int j = 0; j < N; ++j) o[j] = (float)((double)xv[j] + (double)a[j] * (double)yv[j]);
    }
    Chunk<T>::store(out + i * N, o);
  }
};

template <typename T, int OP>
__global__ void __launch_bounds__(512) row_map_chunks(const T* x, const T* y, const float* v, T* out, RowMap m,
                                                      int64_t total) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    Operands<T, OP> p;
    p.load(x, y, v, m, i);
    p.apply(out, i);
  }
}

// Any width and alignment: one value per thread.
// The row from the grid: blockIdx.x a wave's chunks of the row, blockIdx.y
// the row within sample blockIdx.z, so no lane divides. For rows of whole
// waves' chunks and at most 65,535 rows a sample.
template <typename T, int OP>
__global__ void __launch_bounds__(64) row_map_by_row(const T* x, const T* y, const float* v, T* out, RowMap m) {
  constexpr int N = Chunk<T>::N;
  const int64_t r = (int64_t)blockIdx.z * gridDim.y + blockIdx.y;
  const int c = (int)blockIdx.x * 64 + (int)threadIdx.x;
  const int64_t i = r * m.row_chunks + c;
  Operands<T, OP> p;
  p.load_at(x, y, v, m, i, r, c * N, blockIdx.z);
  p.apply(out, i);
}

template <typename T, int OP>
__global__ void __launch_bounds__(256) row_map_values(const T* x, const T* y, const float* v, T* out, RowMap m,
                                                      int64_t total, double col_inverse) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = quotient(i, m.cols, col_inverse);
    const int c = (int)(i - r * m.cols);
    const double xv = (double)load_one(x + i);
    double o;
    if constexpr (OP == MODULATE_CHUNKS) {
      const float* row = v + r * m.chunks * (int64_t)m.cols + c;
      o = xv * (1.0 + (double)row[(int64_t)m.second * m.cols]) + (double)row[(int64_t)m.first * m.cols];
    } else {
      float g;
      if constexpr (OP == GATED_ADD)
        g = v[quotient(r, m.per, m.per_inverse) * m.cols + c];
      else if constexpr (OP == ROW_GATED_ADD)
        g = v[r];
      else
        g = v[r * m.chunks * (int64_t)m.cols + (int64_t)m.first * m.cols + c];
      o = xv + (double)g * (double)load_one(y + i);
    }
    store_one(out + i, (float)o);
  }
}

template <typename T, int OP>
int row_map(const char* entry, const T* x, const T* y, const float* v, T* out, RowMap m, void* stream) {
  if (m.rows == 0) return 0;
  if (!x || !v || !out || (OP != MODULATE_CHUNKS && !y)) return refuse("%s: null operand", entry);
  const hipStream_t s = (hipStream_t)stream;
  constexpr int N = Chunk<T>::N;
  const int64_t values = m.rows * m.cols;
  if (values >= ((int64_t)1 << 50)) return refuse("%s: %lld values", entry, (long long)values);
  m.per_inverse = 1.0 / (double)m.per;
  // chunks of a row stay in the row, and the F32 factors load as float4s
  const bool chunked = m.cols % N == 0 && aligned16(x) && aligned16(out) && (!y || aligned16(y)) &&
                       (OP == ROW_GATED_ADD || aligned16(v));
  if (chunked) {
    m.row_chunks = m.cols / N;
    m.row_inverse = 1.0 / (double)m.row_chunks;
    const int64_t total = values / N;
    // one-wave blocks where they stream faster (gatedAdd 192 -> 183 us,
    // rowGatedAdd 185 -> 182 us at [65520, 3072] bf16); the ops reading two
    // or one F32 table rows a value take 512-thread blocks (modulateChunks
    // 393 us against 406 in 256-thread blocks, 414 in one-wave blocks;
    // gatedAddChunk 307 against 315)
    constexpr int kBlock = OP == MODULATE_CHUNKS || OP == GATED_ADD_CHUNK ? 512 : 64;
    // gatedAdd takes its row and sample from the grid where they fit it
    // ([65520, 3072] bf16: 185.0-185.3 -> 179.9-182.3 us); the other ops
    // measured even (gatedAddChunk) or slower (modulateChunks, 422 against
    // 406 us) that way, and rowGatedAdd's rows do not fit
    const int64_t samples = m.rows / m.per;
    if (OP == GATED_ADD && m.row_chunks % 64 == 0 && m.row_chunks / 64 <= INT32_MAX && m.per <= 65535 &&
        samples <= 65535 && samples * m.per == m.rows) {
      hipLaunchKernelGGL((row_map_by_row<T, OP>), dim3((unsigned)(m.row_chunks / 64), (unsigned)m.per,
                         (unsigned)samples), dim3(64), 0, s, x, y, v, out, m);
      return launched(entry);
    }
    hipLaunchKernelGGL((row_map_chunks<T, OP>), dim3(grid_for(total, kBlock, kOneShotBlocks)), dim3(kBlock), 0, s, x,
                       y, v, out, m, total);
  } else {
    hipLaunchKernelGGL((row_map_values<T, OP>), dim3(grid_for(values, 256, 8192)), dim3(256), 0, s, x, y, v, out, m,
                       values, 1.0 / (double)m.cols);
  }
  return launched(entry);
}

int check_shape(const char* entry, int64_t rows, int cols) {
  if (rows < 0) return refuse("%s: %lld rows", entry, (long long)rows);
  if (cols <= 0) return refuse("%s: rows of %d values", entry, cols);
  return 0;
}

template <typename T>
int gated_add(const char* entry, T* x, const T* y, const float* gate, int64_t rows, int32_t cols,
              int64_t rows_per_sample, void* stream) {
  clear_error();
  if (const int bad = check_shape(entry, rows, cols)) return bad;
  if (rows_per_sample <= 0) return refuse("%s: %lld rows per sample", entry, (long long)rows_per_sample);
  RowMap m{rows, cols, rows_per_sample, 1, 0, 0, 0, 0.0, 0.0};
  return row_map<T, GATED_ADD>(entry, x, y, gate, x, m, stream);
}

int check_chunks(const char* entry, int32_t chunks, std::initializer_list<int32_t> indices) {
  if (chunks <= 0) return refuse("%s: %d chunks per row", entry, chunks);
  for (int32_t index : indices)
    if (index < 0 || index >= chunks) return refuse("%s: chunk %d of %d", entry, index, chunks);
  return 0;
}

template <typename T>
int modulate_chunks(const char* entry, const T* x, const float* table, T* out, int64_t rows, int32_t channels,
                    int32_t chunks, int32_t shift, int32_t scale, void* stream) {
  clear_error();
  if (const int bad = check_shape(entry, rows, channels)) return bad;
  if (const int bad = check_chunks(entry, chunks, {shift, scale})) return bad;
  RowMap m{rows, channels, 1, chunks, shift, scale, 0, 0.0, 0.0};
  return row_map<T, MODULATE_CHUNKS>(entry, x, nullptr, table, out, m, stream);
}

template <typename T>
int gated_add_chunk(const char* entry, T* x, const T* y, const float* table, int64_t rows, int32_t channels,
                    int32_t chunks, int32_t gate, void* stream) {
  clear_error();
  if (const int bad = check_shape(entry, rows, channels)) return bad;
  if (const int bad = check_chunks(entry, chunks, {gate})) return bad;
  RowMap m{rows, channels, 1, chunks, gate, 0, 0, 0.0, 0.0};
  return row_map<T, GATED_ADD_CHUNK>(entry, x, y, table, x, m, stream);
}

template <typename T>
int row_gated_add(const char* entry, T* x, const T* y, const float* gate, int64_t rows, int32_t cols, void* stream) {
  clear_error();
  if (const int bad = check_shape(entry, rows, cols)) return bad;
  RowMap m{rows, cols, 1, 1, 0, 0, 0, 0.0, 0.0};
  return row_map<T, ROW_GATED_ADD>(entry, x, y, gate, x, m, stream);
}

}  // namespace
}  // namespace drift

using namespace drift;

extern "C" int drift_gated_add_f32(float* x, const float* y, const float* gate, int64_t rows, int32_t cols,
                                   int64_t rows_per_sample, void* stream) {
  return gated_add<float>("drift_gated_add_f32", x, y, gate, rows, cols, rows_per_sample, stream);
}

extern "C" int drift_gated_add_bf16(uint16_t* x, const uint16_t* y, const float* gate, int64_t rows, int32_t cols,
                                    int64_t rows_per_sample, void* stream) {
  return gated_add<uint16_t>("drift_gated_add_bf16", x, y, gate, rows, cols, rows_per_sample, stream);
}

extern "C" int drift_modulate_chunks_f32(const float* x, const float* table, float* out, int64_t rows,
                                         int32_t channels, int32_t chunks, int32_t shift, int32_t scale,
                                         void* stream) {
  return modulate_chunks<float>("drift_modulate_chunks_f32", x, table, out, rows, channels, chunks, shift, scale,
                                stream);
}

extern "C" int drift_modulate_chunks_bf16(const uint16_t* x, const float* table, uint16_t* out, int64_t rows,
                                          int32_t channels, int32_t chunks, int32_t shift, int32_t scale,
                                          void* stream) {
  return modulate_chunks<uint16_t>("drift_modulate_chunks_bf16", x, table, out, rows, channels, chunks, shift, scale,
                                   stream);
}

extern "C" int drift_gated_add_chunk_f32(float* x, const float* y, const float* table, int64_t rows,
                                         int32_t channels, int32_t chunks, int32_t gate, void* stream) {
  return gated_add_chunk<float>("drift_gated_add_chunk_f32", x, y, table, rows, channels, chunks, gate, stream);
}

extern "C" int drift_gated_add_chunk_bf16(uint16_t* x, const uint16_t* y, const float* table, int64_t rows,
                                          int32_t channels, int32_t chunks, int32_t gate, void* stream) {
  return gated_add_chunk<uint16_t>("drift_gated_add_chunk_bf16", x, y, table, rows, channels, chunks, gate, stream);
}

extern "C" int drift_row_gated_add_f32(float* x, const float* y, const float* gate, int64_t rows, int32_t cols,
                                       void* stream) {
  return row_gated_add<float>("drift_row_gated_add_f32", x, y, gate, rows, cols, stream);
}

extern "C" int drift_row_gated_add_bf16(uint16_t* x, const uint16_t* y, const float* gate, int64_t rows,
                                        int32_t cols, void* stream) {
  return row_gated_add<uint16_t>("drift_row_gated_add_bf16", x, y, gate, rows, cols, stream);
}
