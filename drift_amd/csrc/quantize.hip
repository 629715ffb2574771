// quantize_x for gfx950: F32 or BF16 values quantized per block of 32 into
// int8 codes, scales and code sums, the form the runner's int8 products read
// (kernels/quantize.h:6-25, kernels/matvec.hip:392-397). The norms and the
// gated product write the same side output as they write their results
// (quantize_chunk); this kernel is the separate launch they must equal.
//
// A lane takes one 16-byte chunk (4 F32 or 8 BF16 values), so 8 or 4
// consecutive lanes hold a block; unaligned inputs or codes take one value
// per lane, 32 lanes to a block.
#include "common.hpp"

namespace drift {
namespace {

template <typename T, int N>
__global__ void __launch_bounds__(256) quantize_chunks(const T* x, Quantized q, int64_t chunks) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < chunks; i += stride) {
    float v[N];
    if constexpr (N == 1)
      v[0] = load_one(x + i);
    else
      Chunk<T>::load(x + i * N, v);
    quantize_chunk<N>(v, i * N / 32, q);
  }
}

template <typename T>
int launch(const T* x, Quantized q, int64_t blocks, hipStream_t s) {
  constexpr int N = Chunk<T>::N;
  // chunks are whole lane groups, and a grid stride of whole waves keeps each
  // group's lanes on one block
  if (aligned16(x) && codes_storable(q.xq, N)) {
    const int64_t chunks = blocks * 32 / N;
    hipLaunchKernelGGL((quantize_chunks<T, N>), dim3(grid_for(chunks, 256, 8192)), dim3(256), 0, s, x, q, chunks);
  } else {
    const int64_t values = blocks * 32;
    hipLaunchKernelGGL((quantize_chunks<T, 1>), dim3(grid_for(values, 256, 8192)), dim3(256), 0, s, x, q, values);
  }
  return 0;
}

template <typename T>
int quantize_x(const char* entry, const T* x, int8_t* xq, float* xd, float* xs, int64_t blocks, void* stream) {
  clear_error();
  if (blocks < 0) return refuse("%s: %lld blocks", entry, (long long)blocks);
  if (blocks == 0) return 0;
  if (!x) return refuse("%s: null x", entry);
  const Quantized q{xq, xd, xs};
  if (!xq) return refuse("%s: null xq", entry);
  if (const int bad = check_quantized(entry, q, blocks * 32)) return bad;
  launch(x, q, blocks, (hipStream_t)stream);
  return launched(entry);
}

}  // namespace

int launch_quantize(const float* x, Quantized q, int64_t blocks, hipStream_t stream) {
  return launch(x, q, blocks, stream);
}

int launch_quantize(const uint16_t* x, Quantized q, int64_t blocks, hipStream_t stream) {
  return launch(x, q, blocks, stream);
}

int check_quantized(const char* entry, Quantized q, int64_t values) {
  if (!q.xq) return 0;
  if (!q.xd || !q.xs) return refuse("%s: xq without xd or xs", entry);
  if (values % 32 != 0) return refuse("%s: %lld values are not whole blocks of 32 to quantize", entry,
                                      (long long)values);
  if ((reinterpret_cast<uintptr_t>(q.xd) | reinterpret_cast<uintptr_t>(q.xs)) & 3u)
    return refuse("%s: xd or xs is not 4-byte aligned", entry);
  return 0;
}

}  // namespace drift

using namespace drift;

extern "C" int drift_quantize_x_f32(const float* x, int8_t* xq, float* xd, float* xs, int64_t blocks, void* stream) {
  return quantize_x<float>("drift_quantize_x_f32", x, xq, xd, xs, blocks, stream);
}

extern "C" int drift_quantize_x_bf16(const uint16_t* x, int8_t* xq, float* xd, float* xs, int64_t blocks,
                                     void* stream) {
  return quantize_x<uint16_t>("drift_quantize_x_bf16", x, xq, xd, xs, blocks, stream);
}
