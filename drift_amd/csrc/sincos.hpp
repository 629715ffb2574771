// Double-precision sin and cos of a float angle, for the rope kernels'
// per-token angles (the CPU reference takes java.lang.Math.cos/sin of the
// float angle widened to double, ops/CpuAttention.scala:124-140).
//
// Method: Cody-Waite reduction x = k pi/2 + r with pi/2 split in three
// doubles and applied by fma (for |x| < 2^20, k < 2^20 and the split's
// parts are exact enough that r keeps full double accuracy), then the
// polynomial kernels of fdlibm's __kernel_sin and __kernel_cos (Sun
// Microsystems' freely distributable libm, k_sin.c and k_cos.c) on
// |r| <= pi/4, and the quadrant's swap and signs. Within 2 ulp of the C
// library's sin and cos over every angle the rope tables produce (a CPU test
// compiles this header and compares). Returns false outside |x| < 2^20, where
// the caller takes the library's sincos.
//
// Plain C++ with no HIP dependency beyond the __host__ __device__ markers, so
// the host test can build it with g++.
#pragma once

#include <cmath>

#ifndef __HIPCC__
#ifndef __host__
#define __host__
#endif
#ifndef __device__
#define __device__
#endif
#endif

namespace drift {

__host__ __device__ inline bool sincos_reduced(float angle, double* s, double* c) {
  const double x = (double)angle;
  if (!(fabs(x) < 1048576.0)) return false;
  const double kPio2Hi = 1.5707963267948966;      // 0x3FF921FB54442D18
  const double kPio2Mid = 6.123233995736766e-17;   // pi/2 - kPio2Hi, rounded
  const double kPio2Lo = -1.4973849048591698e-33;  // the rest
  const double k = rint(x * 0.6366197723675814);
  double r = fma(-k, kPio2Hi, x);
  r = fma(-k, kPio2Mid, r);
  r = fma(-k, kPio2Lo, r);
  const double z = r * r;
  // Horner steps as fma: one rounding a step instead of two, and half the
  // double-precision instructions (the kernels build with contraction off)
  // __kernel_sin(r, 0, 0): r + r z (S1 + z (S2 + z (S3 + z (S4 + z (S5 + z S6)))))
  const double S1 = -1.66666666666666324348e-01, S2 = 8.33333333332248946124e-03,
               S3 = -1.98412698298579493134e-04, S4 = 2.75573137070700676789e-06,
               S5 = -2.50507602534068634195e-08, S6 = 1.58969099521155010221e-10;
  const double ps = fma(z, fma(z, fma(z, fma(z, S6, S5), S4), S3), S2);
  const double sn = fma(r * z, fma(z, ps, S1), r);
  // __kernel_cos(r, 0): w + (((1 - w) - z/2) + z^2 (C1 + ...)), w = 1 - z/2
  const double C1 = 4.16666666666666019037e-02, C2 = -1.38888888888741095749e-03,
               C3 = 2.48015872894767294178e-05, C4 = -2.75573143513906633035e-07,
               C5 = 2.08757232129817482790e-09, C6 = -1.13596475577881948265e-11;
  const double pc = fma(z, fma(z, fma(z, fma(z, fma(z, C6, C5), C4), C3), C2), C1);
  const double hz = 0.5 * z, w = 1.0 - hz;
  const double cs = w + fma(z * z, pc, (1.0 - w) - hz);
  // quadrant k mod 4: sin, cos of k pi/2 + r (|k| < 2^20: an int holds it,
  // and its two's complement low bits are k mod 4 for negative k too)
  const int q = (int)k & 3;
  const double s0 = (q & 1) ? cs : sn, c0 = (q & 1) ? sn : cs;
  *s = (q & 2) ? -s0 : s0;
  *c = ((q + 1) & 2) ? -c0 : c0;
  return true;
}

}  // namespace drift
