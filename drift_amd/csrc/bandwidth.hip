// Streaming probes for gfx950: how fast this GPU moves bytes through HBM for
// a given mix of reads and writes, the ceiling each fused kernel is measured
// against.
//
// read_sum_f32x4 is the reference's probe (runner/kernels/bandwidth.hip:5-20,
// driven by runner/gpuTest/src/drift/runner/MemoryBandwidth.scala:17-88): a
// pure streaming read that leaves one partial sum per block. Here each lane
// keeps four 16-byte loads in flight per pass, the wave's loads covering
// 1 KiB runs, and the block's sum is taken by a DPP butterfly and LDS.
//
// stream_mix moves the byte mix of a fused kernel with nothing else in the
// way: read_chunks 16-byte chunks read and write_chunks written, by blocks
// that each only read or only write 256 x per_thread chunks (1, 2 or 4 a
// lane, each instruction of a wave covering 1 KiB of consecutive memory). The
// read blocks and write blocks are interleaved evenly in dispatch order, so
// the mix holds over the whole launch. A read block folds what it read into
// one value that is stored only if it equals a sentinel (never, for data
// other than all ones), so no read can be dropped. Loads and stores are
// non-temporal, as the fused kernels' are.
//
// row_probe moves a gather's bytes in a gather's pattern: a block per id reads
// the whole table row the id names (row_chunks 16-byte chunks, one or two a
// lane, all in flight together) and writes out_chunks chunks of output, each
// lane's stores carrying the XOR of what it read. Rows drawn at random from a
// table larger than the cache are read from scattered DRAM pages, which a
// contiguous stream does not measure.
#include "common.hpp"

namespace drift {
namespace {

constexpr int kSumPerLane = 4;

__global__ void __launch_bounds__(256) read_sum_kernel(const float* x, int64_t n4, float* partials) {
  __shared__ double wave_sums[4];
  const int64_t stride = (int64_t)gridDim.x * 256 * kSumPerLane;
  double sum = 0.0;
  for (int64_t base = (int64_t)blockIdx.x * 256 * kSumPerLane + threadIdx.x; base < n4; base += stride) {
    uint4 v[kSumPerLane];
#pragma unroll
    for (int k = 0; k < kSumPerLane; ++k) {
      const int64_t i = min(base + (int64_t)k * 256, n4 - 1);  // clamped, not branched: the loads issue together
      v[k] = stream_load(x + 4 * i);
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kSumPerLane; ++k)
      if (base + (int64_t)k * 256 < n4)
        s += (__uint_as_float(v[k].x) + __uint_as_float(v[k].y)) + (__uint_as_float(v[k].z) + __uint_as_float(v[k].w));
    sum += (double)s;
  }
  sum = group_sum<64>(sum);
  if ((threadIdx.x & 63) == 0) wave_sums[threadIdx.x >> 6] = sum;
  __syncthreads();
  if (threadIdx.x == 0) partials[blockIdx.x] = (float)((wave_sums[0] + wave_sums[1]) + (wave_sums[2] + wave_sums[3]));
}

template <int P>
__global__ void __launch_bounds__(256) stream_mix_kernel(const uint4* src, int64_t read_chunks, uint4* dst,
                                                         int64_t write_chunks, int64_t read_blocks,
                                                         int64_t write_blocks) {
  // block b reads when the evenly spread read count steps at b
  const int64_t b = blockIdx.x, all = read_blocks + write_blocks;
  const int64_t reads_before = b * read_blocks / all, reads_through = (b + 1) * read_blocks / all;
  if (reads_through > reads_before) {
    const int64_t base = reads_before * 256 * P + threadIdx.x;
    uint4 v[P];
#pragma unroll
    for (int k = 0; k < P; ++k) v[k] = stream_load(src + min(base + (int64_t)k * 256, read_chunks - 1));
    uint4 acc = v[0];
#pragma unroll
    for (int k = 1; k < P; ++k) acc = make_uint4(acc.x ^ v[k].x, acc.y ^ v[k].y, acc.z ^ v[k].z, acc.w ^ v[k].w);
    if ((acc.x & acc.y & acc.z & acc.w) == 0xffffffffu) dst[0] = acc;
  } else {
    const int64_t base = (b - reads_through) * 256 * P + threadIdx.x;
#pragma unroll
    for (int k = 0; k < P; ++k) {
      const int64_t i = base + (int64_t)k * 256;
      if (i < write_chunks) {
        const u32x4 q = {(uint32_t)i, (uint32_t)(i >> 32), (uint32_t)k, 0x5eedu};
        __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(dst + i));
      }
    }
  }
}

template <int L>
__global__ void __launch_bounds__(256) row_probe_kernel(const uint4* table, int64_t rows, int row_chunks,
                                                        const int32_t* ids, uint4* out, int out_chunks) {
  const int64_t t = blockIdx.x;
  const int64_t id = min(max((int64_t)ids[t], (int64_t)0), rows - 1);
  const uint4* row = table + id * row_chunks;
  uint4 v[L];
#pragma unroll
  for (int k = 0; k < L; ++k) v[k] = stream_load(row + min((int)threadIdx.x + k * 256, row_chunks - 1));
  uint4 acc = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int k = 0; k < L; ++k)
    if ((int)threadIdx.x + k * 256 < row_chunks)
      acc = make_uint4(acc.x ^ v[k].x, acc.y ^ v[k].y, acc.z ^ v[k].z, acc.w ^ v[k].w);
  uint4* target = out + t * out_chunks;
  for (int j = threadIdx.x; j < out_chunks; j += 256) {
    const u32x4 q = {acc.x ^ (uint32_t)j, acc.y, acc.z, acc.w};
    __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(target + j));
  }
}

}  // namespace
}  // namespace drift

using namespace drift;

extern "C" int drift_read_sum_f32x4(const float* x, int64_t n4, float* partials, int32_t blocks, void* stream) {
  const char* entry = "drift_read_sum_f32x4";
  clear_error();
  if (n4 < 0 || blocks <= 0 || blocks > (1 << 20))
    return refuse("%s: %lld float4 values over %d blocks", entry, (long long)n4, blocks);
  if (!x || !partials) return refuse("%s: null x or partials", entry);
  if (!aligned16(x)) return refuse("%s: x is not 16-byte aligned", entry);
  hipLaunchKernelGGL(read_sum_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, x, n4, partials);
  return launched(entry);
}

extern "C" int drift_stream_mix(const void* src, int64_t read_chunks, void* dst, int64_t write_chunks,
                                int32_t per_thread, void* stream) {
  const char* entry = "drift_stream_mix";
  clear_error();
  if (read_chunks < 0 || write_chunks < 1 || (per_thread != 1 && per_thread != 2 && per_thread != 4))
    return refuse("%s: %lld chunks read, %lld written, %d a lane (at least one written; 1, 2 or 4 a lane)", entry,
                  (long long)read_chunks, (long long)write_chunks, per_thread);
  if ((read_chunks > 0 && !src) || !dst) return refuse("%s: null src or dst", entry);
  if ((read_chunks > 0 && !aligned16(src)) || !aligned16(dst)) return refuse("%s: src or dst is not 16-byte aligned", entry);
  const int64_t read_blocks = ceil_div(read_chunks, 256 * per_thread);
  const int64_t write_blocks = ceil_div(write_chunks, 256 * per_thread);
  if (read_blocks + write_blocks > kOneShotBlocks)
    return refuse("%s: %lld chunks", entry, (long long)(read_chunks + write_chunks));
  const dim3 grid((unsigned)(read_blocks + write_blocks));
  const hipStream_t s = (hipStream_t)stream;
  const uint4* in = static_cast<const uint4*>(src);
  uint4* out = static_cast<uint4*>(dst);
  if (per_thread == 1)
    hipLaunchKernelGGL(stream_mix_kernel<1>, grid, dim3(256), 0, s, in, read_chunks, out, write_chunks, read_blocks,
                       write_blocks);
  else if (per_thread == 2)
    hipLaunchKernelGGL(stream_mix_kernel<2>, grid, dim3(256), 0, s, in, read_chunks, out, write_chunks, read_blocks,
                       write_blocks);
  else
    hipLaunchKernelGGL(stream_mix_kernel<4>, grid, dim3(256), 0, s, in, read_chunks, out, write_chunks, read_blocks,
                       write_blocks);
  return launched(entry);
}

extern "C" int drift_row_probe(const void* table, int64_t rows, int32_t row_chunks, const int32_t* ids, int64_t count,
                               void* out, int32_t out_chunks, void* stream) {
  const char* entry = "drift_row_probe";
  clear_error();
  if (rows < 1 || row_chunks < 1 || row_chunks > 512 || count < 0 || out_chunks < 1)
    return refuse("%s: %lld ids into %lld rows of %d chunks (1 to 512), %d chunks out each", entry, (long long)count,
                  (long long)rows, row_chunks, out_chunks);
  if (count == 0) return 0;
  if (!table || !ids || !out) return refuse("%s: null table, ids or out", entry);
  if (!aligned16(table) || !aligned16(out)) return refuse("%s: table or out is not 16-byte aligned", entry);
  if (count > kOneShotBlocks) return refuse("%s: %lld ids", entry, (long long)count);
  const dim3 grid((unsigned)count);
  const hipStream_t s = (hipStream_t)stream;
  const uint4* in = static_cast<const uint4*>(table);
  uint4* o = static_cast<uint4*>(out);
  if (row_chunks <= 256)
    hipLaunchKernelGGL(row_probe_kernel<1>, grid, dim3(256), 0, s, in, rows, row_chunks, ids, o, out_chunks);
  else
    hipLaunchKernelGGL(row_probe_kernel<2>, grid, dim3(256), 0, s, in, rows, row_chunks, ids, o, out_chunks);
  return launched(entry);
}
