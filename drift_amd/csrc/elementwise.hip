// Elementwise kernels for gfx950: activations, gated activations (SwiGLU and
// kin) and float-type conversions. A thread takes one 16-byte chunk (8 bf16
// or 4 F32 values) and the grid covers the tensor in one pass (a grid-stride
// loop only past 2^30 blocks).
//
// The runner's CPU reference computes activations in double
// (ops/CpuNormalisation.scala:11-24). Here they run in float through forms
// that keep relative accuracy everywhere (no 1 + tanh or 1 + erf
// cancellation):
//   silu(v)      = v s(v),   s(v) = 1/(1 + e^-v) from e = e^-|v|
//   gelu_tanh(v) = v/2 (1 + tanh u) with 1 + tanh u = 2/(1 + e^-2u) or
//                  2e^2u/(1 + e^2u)
//   gelu_erf(v)  = v/2 erfc(-v/sqrt2)
// Where the reference's own double result is quantized (1 + tanh u and
// 1 + erf x below 2^-29 hold a whole number of 2^-53 steps, the spacing of
// doubles just above -1, so far enough into the tail one step is more than
// 1e-5 of the value), F32 outputs take the reference's steps in double
// instead: 1 + tanh u as the C library's tanh makes it (fdlibm's s_tanh.c,
// 1 - 2/(expm1(2|u|) + 2) for 1 <= |u| < 22, -1 beyond; equal to glibc's
// 1 + tanh(u) on every one of 2e7 sampled u in [-22.5, -1]), and 1 + erf x as
// CpuOps.erf makes it (ops/CpuOps.scala:26-50: 1 - (1 - E), E from the
// 60-level continued fraction). BF16 outputs round the float sum to the same
// step instead, well within their ulp. F32 outputs use the accurate library
// exp and IEEE division. BF16 outputs use the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32: about 1e-6 relative, far below a bf16 ulp, and BF16
// output is all the precision they feed), with GELU-tanh's sigmoid form
// folded to one exp2 argument:
//   gelu_tanh(v) = v h,  h = 1/(1 + 2^(v (c0 + c1 v^2))),
//   c0 = -2 log2(e) sqrt(2/pi), c1 = c0 * 0.044715.
#include "common.hpp"

namespace drift {
namespace {

template <bool ACCURATE>
__device__ __forceinline__ float divide(float a, float b) {
  if constexpr (ACCURATE)
    return a / b;
  else
    return a * __builtin_amdgcn_rcpf(b);
}

template <bool ACCURATE>
__device__ __forceinline__ float sigmoid_of(float v) {
  if constexpr (ACCURATE) {
    const float e = expf(-fabsf(v));
    const float r = 1.0f / (1.0f + e);
    return v >= 0.0f ? r : e * r;
  } else {
    const float e = __builtin_amdgcn_exp2f(-1.44269504088896341f * fabsf(v));
    const float r = __builtin_amdgcn_rcpf(1.0f + e);
    return v >= 0.0f ? r : e * r;
  }
}

// GELU-tanh of M values for BF16 outputs, in place (see the file comment).
// The tail quantization runs only when some lane has a value that needs it.
template <int M>
__device__ __forceinline__ void gelu_tanh_fast(float (&v)[M]) {
  constexpr float c0 = -2.30220819814432500f;  // -2 log2(e) sqrt(2/pi)
  constexpr float c1 = -0.10294323958002350f;  // c0 * 0.044715
  float h[M];
  bool tail = false;
#pragma unroll
  for (int j = 0; j < M; ++j) {
    const float a = v[j] * fmaf(c1, v[j] * v[j], c0);
    h[j] = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(a));  // (1 + tanh u) / 2
    tail |= h[j] < 0x1p-30f;
  }
  if (__builtin_expect(__any(tail), 0)) {
#pragma unroll
    for (int j = 0; j < M; ++j) h[j] = h[j] < 0x1p-30f ? rintf(h[j] * 0x1p54f) * 0x1p-54f : h[j];
  }
#pragma unroll
  for (int j = 0; j < M; ++j) v[j] *= h[j];
}

// The reference's double constants: sqrt(2 / pi), sqrt(pi) and sqrt(2) as
// math.sqrt rounds them.
constexpr double kSqrt2OverPi = 0x1.9884533d43651p-1;
constexpr double kSqrtPi = 0x1.c5bf891b4ef6ap+0;
constexpr double kSqrt2 = 0x1.6a09e667f3bcdp+0;

// GELU-tanh of an F32 value whose 1 + tanh u lies in the quantized tail, the
// reference's double arithmetic step by step (ops/CpuNormalisation.scala:14):
// u = sqrt(2/pi) (v + 0.044715 v^3); 1 + tanh u for u <= -1 from the C
// library's formula; 0.5 v (1 + tanh u).
__device__ __attribute__((noinline)) float gelu_tanh_tail(float value) {
  const double v = value;
  const double u = kSqrt2OverPi * (v + 0.044715 * v * v * v);
  const double a = -2.0 * u;  // 2|u|: the tail has u < -10
  const double t = a >= 44.0 ? 0.0 : 1.0 - (1.0 - 2.0 / (expm1(a) + 2.0));
  return (float)(0.5 * v * t);
}

// GELU-erf of an F32 value whose 1 + erf x lies in the quantized tail (x =
// v / sqrt 2 at or below -2.5): CpuOps.erf's continued fraction for -x, then
// 1 + erf x = 1 - (1 - E) as the reference's double sums make it.
__device__ __attribute__((noinline)) float gelu_erf_tail(float value) {
  const double v = value;
  const double x = -(v / kSqrt2);
  double fraction = 0.0;
  for (int n = 60; n >= 1; --n) fraction = (n / 2.0) / (x + fraction);
  const double e = exp(-x * x) / kSqrtPi / (x + fraction);
  return (float)(0.5 * v * (1.0 - (1.0 - e)));
}

template <bool ACCURATE>
__device__ __forceinline__ float activate(int kind, float v) {
  switch (kind) {
    case DRIFT_SILU:
      return v * sigmoid_of<ACCURATE>(v);
    case DRIFT_GELU_TANH: {
      if constexpr (!ACCURATE) {
        float one[1] = {v};
        gelu_tanh_fast(one);
        return one[0];
      }
      const float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
      const float e = expf(-2.0f * fabsf(u));
      const float t = (u >= 0.0f ? 2.0f : 2.0f * e) / (1.0f + e);  // 1 + tanh(u)
      return t < 0x1p-29f ? gelu_tanh_tail(v) : 0.5f * v * t;
    }
    case DRIFT_GELU_ERF: {
      const float t = erfcf(-v * 0.70710678118654752f);  // 1 + erf(v / sqrt 2)
      return t < 0x1p-29f ? gelu_erf_tail(v) : 0.5f * v * t;
    }
    case DRIFT_SIGMOID:
      return sigmoid_of<ACCURATE>(v);
    default:  // DRIFT_SITU: 4 tanh(v / 4) s(v)
      return 4.0f * tanhf(0.25f * v) * sigmoid_of<ACCURATE>(v);
  }
}

template <bool ACCURATE>
__device__ __forceinline__ float gated_up(int kind, float u) {
  return kind == DRIFT_SITU ? 25.0f * tanhf(divide<ACCURATE>(u, 25.0f)) : u;
}

// ------------------------------------------------------------------ kernels

template <typename T>
constexpr bool kAccurate = sizeof(T) == 4;

template <typename T, int KIND>
__global__ void __launch_bounds__(256) activation_kernel(const T* x, T* out, int64_t n, int kind, float scale) {
  constexpr int N = Chunk<T>::N;
  constexpr bool A = kAccurate<T>;
  const int k = KIND >= 0 ? KIND : kind;
  const int64_t chunks = n / N;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = tid; i < chunks; i += stride) {
    float a[N];
    Chunk<T>::load(x + i * N, a);
    if constexpr (KIND == DRIFT_GELU_TANH && !A) {
#pragma unroll
      for (int j = 0; j < N; ++j) a[j] *= scale;
      gelu_tanh_fast(a);
    } else {
#pragma unroll
      for (int j = 0; j < N; ++j) a[j] = activate<A>(k, scale * a[j]);
    }
    Chunk<T>::store(out + i * N, a);
  }
  const int64_t tail = chunks * N + tid;
  if (tail < n) store_one(out + tail, activate<A>(k, scale * load_one(x + tail)));
}

template <typename T>
__global__ void __launch_bounds__(256) activation_scalar(const T* x, T* out, int64_t n, int kind, float scale) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    store_one(out + i, activate<kAccurate<T>>(kind, scale * load_one(x + i)));
}

// With q.xq, out is quantized too as it is written (quantize_chunk; n a
// multiple of 32, so there is no tail and a wave's chunks are whole blocks).
template <typename T, int KIND>
__global__ void __launch_bounds__(256) gated_kernel(const T* gate, const T* up, T* out, int64_t n, int kind,
                                                    Quantized q) {
  constexpr int N = Chunk<T>::N;
  constexpr bool A = kAccurate<T>;
  const int k = KIND >= 0 ? KIND : kind;
  const int64_t chunks = n / N;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = tid; i < chunks; i += stride) {
    float g[N], u[N];
    Chunk<T>::load(gate + i * N, g);
    Chunk<T>::load(up + i * N, u);
#pragma unroll
    for (int j = 0; j < N; ++j) g[j] = activate<A>(k, g[j]) * gated_up<A>(k, u[j]);
    Chunk<T>::store(out + i * N, g);
    if (q.xq) {
      as_written<T>(g);
      quantize_chunk<N>(g, i * N / 32, q);
    }
  }
  const int64_t tail = chunks * N + tid;
  if (tail < n) store_one(out + tail, activate<A>(k, load_one(gate + tail)) * gated_up<A>(k, load_one(up + tail)));
}

template <typename T>
__global__ void __launch_bounds__(256) gated_scalar(const T* gate, const T* up, T* out, int64_t n, int kind) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    store_one(out + i, activate<kAccurate<T>>(kind, load_one(gate + i)) * gated_up<kAccurate<T>>(kind, load_one(up + i)));
}

// Conversions. F16 through the hardware converts: round to nearest even,
// subnormals kept.
__global__ void __launch_bounds__(256) convert_kernel(const void* x, void* out, int64_t n, int kind) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    switch (kind) {
      case DRIFT_F32_TO_BF16:
        static_cast<uint16_t*>(out)[i] = (uint16_t)bf16_bits(static_cast<const float*>(x)[i]);
        break;
      case DRIFT_BF16_TO_F32:
        static_cast<float*>(out)[i] = __uint_as_float((uint32_t) static_cast<const uint16_t*>(x)[i] << 16);
        break;
      case DRIFT_F32_TO_F16:
        static_cast<_Float16*>(out)[i] = (_Float16) static_cast<const float*>(x)[i];
        break;
      case DRIFT_F8E4M3_TO_F32: {
        // fp8 E4M3 "fn" (tensor/DType.scala:105-115): bias 7, no infinities,
        // NaN at S.1111.111
        const uint32_t code = static_cast<const uint8_t*>(x)[i];
        const int exponent = (int)((code >> 3) & 0xfu), mantissa = (int)(code & 7u);
        float magnitude;
        if (exponent == 0xf && mantissa == 7)
          magnitude = __builtin_nanf("");
        else if (exponent == 0)
          magnitude = ldexpf((float)mantissa, -9);
        else
          magnitude = ldexpf((float)(8 + mantissa), exponent - 10);
        static_cast<float*>(out)[i] = (code & 0x80u) ? -magnitude : magnitude;
        break;
      }
      default:
        static_cast<float*>(out)[i] = (float)static_cast<const _Float16*>(x)[i];
        break;
    }
  }
}

// 8 values per thread for the F32 <-> BF16 pairs.
__global__ void __launch_bounds__(256) convert_bf16_chunks(const void* x, void* out, int64_t chunks, int kind) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < chunks; i += stride) {
    float v[8];
    if (kind == DRIFT_F32_TO_BF16) {
      Chunk<float>::load(static_cast<const float*>(x) + i * 8, *reinterpret_cast<float(*)[4]>(v));
      Chunk<float>::load(static_cast<const float*>(x) + i * 8 + 4, *reinterpret_cast<float(*)[4]>(v + 4));
      Chunk<uint16_t>::store(static_cast<uint16_t*>(out) + i * 8, v);
    } else {
      Chunk<uint16_t>::load(static_cast<const uint16_t*>(x) + i * 8, v);
      Chunk<float>::store(static_cast<float*>(out) + i * 8, *reinterpret_cast<float(*)[4]>(v));
      Chunk<float>::store(static_cast<float*>(out) + i * 8 + 4, *reinterpret_cast<float(*)[4]>(v + 4));
    }
  }
}

template <typename T>
int activation(const char* entry, const T* x, T* out, int64_t n, int32_t kind, float scale, void* stream) {
  clear_error();
  if (n < 0) return refuse("%s: %lld values", entry, (long long)n);
  if (kind < DRIFT_SILU || kind > DRIFT_SITU) return refuse("%s: no activation %d", entry, kind);
  if (n == 0) return 0;
  if (!x || !out) return refuse("%s: null x or out", entry);
  const hipStream_t s = (hipStream_t)stream;
  constexpr int N = Chunk<T>::N;
  if (aligned16(x) && aligned16(out)) {
    // one-wave blocks: GELU-tanh over [65520, 3072] bf16 in place 123.5 us
    // in 256-thread blocks against 120.2
    const unsigned grid = grid_for(ceil_div(n, N), kWave, kOneShotBlocks);
    switch (kind) {
      case DRIFT_SILU:
        hipLaunchKernelGGL((activation_kernel<T, DRIFT_SILU>), dim3(grid), dim3(kWave), 0, s, x, out, n, kind, scale);
        break;
      case DRIFT_GELU_TANH:
        hipLaunchKernelGGL((activation_kernel<T, DRIFT_GELU_TANH>), dim3(grid), dim3(kWave), 0, s, x, out, n, kind,
                           scale);
        break;
      default:
        hipLaunchKernelGGL((activation_kernel<T, -1>), dim3(grid), dim3(kWave), 0, s, x, out, n, kind, scale);
        break;
    }
  } else {
    hipLaunchKernelGGL(activation_scalar<T>, dim3(grid_for(n, 256, 8192)), dim3(256), 0, s, x, out, n, kind, scale);
  }
  return launched(entry);
}

template <typename T>
int gated(const char* entry, const T* gate, const T* up, T* out, int64_t n, int32_t kind, Quantized q,
          void* stream) {
  clear_error();
  if (n < 0) return refuse("%s: %lld values", entry, (long long)n);
  if (kind < DRIFT_SILU || kind > DRIFT_SITU) return refuse("%s: no activation %d", entry, kind);
  if (const int bad = check_quantized(entry, q, n)) return bad;
  if (n == 0) return 0;
  if (!gate || !up || !out) return refuse("%s: null gate, up or out", entry);
  const hipStream_t s = (hipStream_t)stream;
  constexpr int N = Chunk<T>::N;
  const bool chunked = aligned16(gate) && aligned16(up) && aligned16(out);
  // the side output is written by the product when its chunks can store the
  // codes, else by a quantize_x launch over out right after
  const bool fused = q.xq && chunked && codes_storable(q.xq, N);
  const Quantized in_kernel = fused ? q : Quantized{nullptr, nullptr, nullptr};
  if (chunked) {
    const unsigned grid = grid_for(ceil_div(n, N), 256, kOneShotBlocks);
    if (kind == DRIFT_SILU)
      hipLaunchKernelGGL((gated_kernel<T, DRIFT_SILU>), dim3(grid), dim3(256), 0, s, gate, up, out, n, kind,
                         in_kernel);
    else
      hipLaunchKernelGGL((gated_kernel<T, -1>), dim3(grid), dim3(256), 0, s, gate, up, out, n, kind, in_kernel);
  } else {
    hipLaunchKernelGGL(gated_scalar<T>, dim3(grid_for(n, 256, 8192)), dim3(256), 0, s, gate, up, out, n, kind);
  }
  if (q.xq && !fused) {
    if (const int status = launched(entry)) return status;
    launch_quantize(out, q, n / 32, s);
  }
  return launched(entry);
}

}  // namespace
}  // namespace drift

using namespace drift;

extern "C" int drift_activation_f32(const float* x, float* out, int64_t n, int32_t kind, float scale,
                                    void* stream) {
  return activation<float>("drift_activation_f32", x, out, n, kind, scale, stream);
}

extern "C" int drift_activation_bf16(const uint16_t* x, uint16_t* out, int64_t n, int32_t kind, float scale,
                                     void* stream) {
  return activation<uint16_t>("drift_activation_bf16", x, out, n, kind, scale, stream);
}

extern "C" int drift_gated_f32(const float* gate, const float* up, float* out, int64_t n, int32_t kind,
                               int8_t* xq, float* xd, float* xs, void* stream) {
  return gated<float>("drift_gated_f32", gate, up, out, n, kind, Quantized{xq, xd, xs}, stream);
}

extern "C" int drift_gated_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n, int32_t kind,
                                int8_t* xq, float* xd, float* xs, void* stream) {
  return gated<uint16_t>("drift_gated_bf16", gate, up, out, n, kind, Quantized{xq, xd, xs}, stream);
}

extern "C" int drift_convert(const void* x, void* out, int64_t n, int32_t kind, void* stream) {
  const char* entry = "drift_convert";
  clear_error();
  if (n < 0) return refuse("%s: %lld values", entry, (long long)n);
  if (kind < DRIFT_F32_TO_F16 || kind > DRIFT_F8E4M3_TO_F32) return refuse("%s: no conversion %d", entry, kind);
  if (n == 0) return 0;
  if (!x || !out) return refuse("%s: null x or out", entry);
  if (x == out) return refuse("%s: x and out are the same buffer of different types", entry);
  const hipStream_t s = (hipStream_t)stream;
  const bool bf16 = kind == DRIFT_F32_TO_BF16 || kind == DRIFT_BF16_TO_F32;
  if (bf16 && n % 8 == 0 && aligned16(x) && aligned16(out))
    hipLaunchKernelGGL(convert_bf16_chunks, dim3(grid_for(n / 8, 256, 8192)), dim3(256), 0, s, x, out, n / 8, kind);
  else
    hipLaunchKernelGGL(convert_kernel, dim3(grid_for(n, 256, 8192)), dim3(256), 0, s, x, out, n, kind);
  return launched(entry);
}
