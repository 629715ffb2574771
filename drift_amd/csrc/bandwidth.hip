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
//
// wave_copy and wave_row_probe are the same two patterns in the shape the
// fused kernels take: one-wave blocks, each wave reading its share of the
// input and then writing its share of the output, every store carrying the
// fold of what its lane read (so, as in a kernel, a wave's stores wait for
// its loads). wave_copy spreads the reads and the writes evenly over the
// waves; wave_row_probe gives each id `slices` waves, wave s of an id reading
// slice s of the row and writing slice s of the output row. At the sizes of
// the prefill shapes one-wave blocks stream faster than 256-thread blocks, so
// these are the tighter ceilings there.
#include "common.hpp"

#include <algorithm>
#include <climits>
#include <type_traits>

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

// One wave's part of a one-wave-block probe: lane l reads chunks r0 + l +
// 64 k (k < R) below r1, all in flight together, then writes chunks w0 + l +
// 64 k (k < W) below w1, each holding the XOR of what the lane read with its
// first word XORed with the chunk's index in [w0, w1).
template <int R, int W>
__device__ __forceinline__ void wave_part(const uint4* src, int64_t r0, int64_t r1, uint4* dst, int64_t w0,
                                          int64_t w1) {
  const int lane = threadIdx.x % kWave;
  uint4 v[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int64_t i = r0 + lane + (int64_t)k * kWave;
    v[k] = i < r1 ? stream_load(src + i) : make_uint4(0, 0, 0, 0);
  }
  uint4 acc = v[0];
#pragma unroll
  for (int k = 1; k < R; ++k) acc = make_uint4(acc.x ^ v[k].x, acc.y ^ v[k].y, acc.z ^ v[k].z, acc.w ^ v[k].w);
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const int64_t j = w0 + lane + (int64_t)k * kWave;
    if (j < w1) {
      const u32x4 q = {acc.x ^ (uint32_t)(j - w0), acc.y, acc.z, acc.w};
      __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(dst + j));
    }
  }
}

// wave b reads chunks [b rpw, (b + 1) rpw) and writes [b wpw, (b + 1) wpw),
// each cut at the end of its tensor
template <int R, int W>
__global__ void __launch_bounds__(kWave) wave_copy_kernel(const uint4* src, int64_t read_chunks, uint4* dst,
                                                          int64_t write_chunks, int rpw, int wpw) {
  const int64_t b = blockIdx.x;
  wave_part<R, W>(src, b * rpw, min(b * rpw + rpw, read_chunks), dst, b * wpw, min(b * wpw + wpw, write_chunks));
}

// the same in blocks of several waves: wave w of block k is wave b = k
// waves_per_block + w (a wave past the last finds both its ranges empty)
template <int R, int W>
__global__ void __launch_bounds__(1024) block_copy_kernel(const uint4* src, int64_t read_chunks, uint4* dst,
                                                          int64_t write_chunks, int rpw, int wpw) {
  const int64_t b = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  wave_part<R, W>(src, min(b * rpw, read_chunks), min(b * rpw + rpw, read_chunks), dst, min(b * wpw, write_chunks),
                  min(b * wpw + wpw, write_chunks));
}

// wave b takes slice s = b % slices of id t = b / slices (clamped into the
// table): row chunks [s rs, (s + 1) rs) and output chunks [s os, (s + 1) os)
template <int R, int W>
__global__ void __launch_bounds__(kWave) wave_row_kernel(const uint4* table, int64_t rows, int row_chunks,
                                                         const int32_t* ids, uint4* out, int out_chunks, uint32_t slices,
                                                         int rs, int os) {
  const uint32_t t = blockIdx.x / slices, s = blockIdx.x - t * slices;
  const int64_t id = min(max((int64_t)ids[t], (int64_t)0), rows - 1);
  const uint4* row = table + id * row_chunks;
  uint4* target = out + (int64_t)t * out_chunks;
  wave_part<R, W>(row, (int64_t)s * rs, min((int64_t)(s + 1) * rs, (int64_t)row_chunks), target, (int64_t)s * os,
                  min((int64_t)(s + 1) * os, (int64_t)out_chunks));
}

// the smallest of 1, 2, 4, 8 chunks a lane that covers `chunks` in a wave
// (0 if none does)
inline int lanes_cover(int64_t chunks) {
  for (int per = 1; per <= 8; per *= 2)
    if (chunks <= (int64_t)per * kWave) return per;
  return 0;
}

template <template <int, int> class Launch, typename... Args>
void launch_rw(int r, int w, Args... args) {
  auto by_w = [&](auto rc) {
    constexpr int R = decltype(rc)::value;
    switch (w) {
      case 1: Launch<R, 1>::go(args...); break;
      case 2: Launch<R, 2>::go(args...); break;
      case 4: Launch<R, 4>::go(args...); break;
      default: Launch<R, 8>::go(args...); break;
    }
  };
  switch (r) {
    case 1: by_w(std::integral_constant<int, 1>{}); break;
    case 2: by_w(std::integral_constant<int, 2>{}); break;
    case 4: by_w(std::integral_constant<int, 4>{}); break;
    default: by_w(std::integral_constant<int, 8>{}); break;
  }
}

template <int R, int W>
struct WaveCopyLaunch {
  static void go(int64_t waves, hipStream_t s, const uint4* in, int64_t reads, uint4* out, int64_t writes, int rpw,
                 int wpw) {
    hipLaunchKernelGGL((wave_copy_kernel<R, W>), dim3((unsigned)waves), dim3(kWave), 0, s, in, reads, out, writes,
                       rpw, wpw);
  }
};

template <int R, int W>
struct BlockCopyLaunch {
  static void go(int64_t blocks, int waves_per_block, hipStream_t s, const uint4* in, int64_t reads, uint4* out,
                 int64_t writes, int rpw, int wpw) {
    hipLaunchKernelGGL((block_copy_kernel<R, W>), dim3((unsigned)blocks), dim3(kWave * waves_per_block), 0, s, in,
                       reads, out, writes, rpw, wpw);
  }
};

template <int R, int W>
struct WaveRowLaunch {
  static void go(int64_t waves, hipStream_t s, const uint4* table, int64_t rows, int row_chunks, const int32_t* ids,
                 uint4* out, int out_chunks, int slices, int rs, int os) {
    hipLaunchKernelGGL((wave_row_kernel<R, W>), dim3((unsigned)waves), dim3(kWave), 0, s, table, rows, row_chunks,
                       ids, out, out_chunks, (uint32_t)slices, rs, os);
  }
};

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

namespace drift {
namespace {

// drift_wave_copy in blocks of waves_per_block waves (1: one-wave blocks)
int copy_probe(const char* entry, const void* src, int64_t read_chunks, void* dst, int64_t write_chunks,
               int32_t per_lane, int32_t waves_per_block, void* stream) {
  clear_error();
  if (read_chunks < 0 || write_chunks < 1 || lanes_cover((int64_t)per_lane * kWave) != per_lane)
    return refuse("%s: %lld chunks read, %lld written, %d a lane (at least one written; 1, 2, 4 or 8 a lane)", entry,
                  (long long)read_chunks, (long long)write_chunks, per_lane);
  if (waves_per_block < 1 || waves_per_block > 16 || (waves_per_block & (waves_per_block - 1)) != 0)
    return refuse("%s: %d waves a block (1, 2, 4, 8 or 16)", entry, waves_per_block);
  if ((read_chunks > 0 && !src) || !dst) return refuse("%s: null src or dst", entry);
  if ((read_chunks > 0 && !aligned16(src)) || !aligned16(dst)) return refuse("%s: src or dst is not 16-byte aligned", entry);
  const int64_t waves = std::max(ceil_div(read_chunks, (int64_t)per_lane * kWave),
                                 ceil_div(write_chunks, (int64_t)per_lane * kWave));
  if (waves > INT32_MAX) return refuse("%s: %lld chunks", entry, (long long)std::max(read_chunks, write_chunks));
  // a wave's share, ceil(chunks / waves), is at most per_lane * 64
  const int64_t rpw = ceil_div(read_chunks, waves), wpw = ceil_div(write_chunks, waves);
  const int r = std::max(lanes_cover(rpw), 1), w = lanes_cover(wpw);
  if (waves_per_block == 1)
    launch_rw<WaveCopyLaunch>(r, w, waves, (hipStream_t)stream, static_cast<const uint4*>(src), read_chunks,
                              static_cast<uint4*>(dst), write_chunks, (int)rpw, (int)wpw);
  else
    launch_rw<BlockCopyLaunch>(r, w, ceil_div(waves, (int64_t)waves_per_block), (int)waves_per_block,
                               (hipStream_t)stream, static_cast<const uint4*>(src), read_chunks,
                               static_cast<uint4*>(dst), write_chunks, (int)rpw, (int)wpw);
  return launched(entry);
}

}  // namespace
}  // namespace drift

extern "C" int drift_wave_copy(const void* src, int64_t read_chunks, void* dst, int64_t write_chunks,
                               int32_t per_lane, void* stream) {
  return copy_probe("drift_wave_copy", src, read_chunks, dst, write_chunks, per_lane, 1, stream);
}

extern "C" int drift_block_copy(const void* src, int64_t read_chunks, void* dst, int64_t write_chunks,
                                int32_t per_lane, int32_t waves_per_block, void* stream) {
  return copy_probe("drift_block_copy", src, read_chunks, dst, write_chunks, per_lane, waves_per_block, stream);
}

extern "C" int drift_wave_row_probe(const void* table, int64_t rows, int32_t row_chunks, const int32_t* ids,
                                    int64_t count, void* out, int32_t out_chunks, int32_t slices, void* stream) {
  const char* entry = "drift_wave_row_probe";
  clear_error();
  if (rows < 1 || row_chunks < 1 || count < 0 || out_chunks < 1 || slices < 1 ||
      ceil_div(row_chunks, slices) > 8 * kWave || ceil_div(out_chunks, slices) > 8 * kWave)
    return refuse("%s: %lld ids into %lld rows of %d chunks, %d chunks out each, %d waves a row (at most 512 chunks "
                  "a wave each way)", entry, (long long)count, (long long)rows, row_chunks, out_chunks, slices);
  if (count == 0) return 0;
  if (!table || !ids || !out) return refuse("%s: null table, ids or out", entry);
  if (!aligned16(table) || !aligned16(out)) return refuse("%s: table or out is not 16-byte aligned", entry);
  if (count > INT32_MAX / slices) return refuse("%s: %lld ids of %d waves", entry, (long long)count, slices);
  const int rs = (int)ceil_div(row_chunks, slices), os = (int)ceil_div(out_chunks, slices);
  launch_rw<WaveRowLaunch>(lanes_cover(rs), lanes_cover(os), count * slices, (hipStream_t)stream,
                           static_cast<const uint4*>(table), rows, (int)row_chunks, ids, static_cast<uint4*>(out),
                           (int)out_chunks, (int)slices, rs, os);
  return launched(entry);
}
