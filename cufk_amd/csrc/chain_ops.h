// Device primitives for the NeRF chain scan on CDNA4 (gfx950, wave64).
//
// A chain step k maps internal coordinates (l, theta, phi) = (L[k+2], A[k+1], D[k]) to the
// rigid transform M = Rx(phi) * Rz(pi - theta) with translation l * M[:,0]
// (reference: src/cufk/csrc/affine.cuh:24-51).  The running product of these transforms
// is a rotation R (row-major R[r][c]) plus a translation; the reference composes general
// 3x4 affines (affine.cuh:53-58), here a new step is folded into a running rotation with
// two column rotations (24 FMA) and its translation is l times the new first column (3 FMA).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <limits>

namespace cufk_amd {

// ------------------------------------------------------------------ scalar types

// Storage types: float, double, _Float16 (torch.float16), __bf16 (torch.bfloat16).
// Compute type: double for double, float otherwise.  Half types are widened on load and
// rounded once on store (the reference instead rounds every payload operation to the
// storage type, scalar.cuh:8-92, which adds one storage-precision rounding per step).
template <typename T> struct compute_type { using type = float; };
template <> struct compute_type<double> { using type = double; };
template <typename T> using compute_t = typename compute_type<T>::type;

template <typename T> __device__ __forceinline__ compute_t<T> widen(T x) {
  return static_cast<compute_t<T>>(x);
}
template <typename T> __device__ __forceinline__ T narrow(compute_t<T> x) {
  return static_cast<T>(x);
}

// a * b + c for a constant c kept in a scalar register pair: one VOP3 v_fma_f64 (VOP3 reads
// one scalar operand).  A plain fma with a 64-bit literal addend is emitted as the
// two-address v_fmac with the literal first copied into two VGPRs, three VALU issues.
__device__ __forceinline__ double fma_sk(double a, double b, double c) {
  double d;
  asm("v_fma_f64 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "s"(c));
  return d;
}
// a * k - 0.5 for a constant k kept in a scalar register pair (-0.5 is an inline constant,
// which does not count against VOP3's one scalar operand): one v_fma_f64.
__device__ __forceinline__ double fma_sk_minus_half(double a, double k) {
  double d;
  asm("v_fma_f64 %0, %1, %2, -0.5" : "=v"(d) : "v"(a), "s"(k));
  return d;
}
// c0 * u + c1 for constants c0, c1: v_mul_f64 and v_add_f64, each with a scalar operand.
__device__ __forceinline__ double lin_sk(double u, double c0, double c1) {
  double t, d;
  asm("v_mul_f64 %0, %1, %2" : "=v"(t) : "v"(u), "s"(c0));
  asm("v_add_f64 %0, %1, %2" : "=v"(d) : "v"(t), "s"(c1));
  return d;
}

// Largest |x| the reduction in sin_cos_wide handles; beyond it (and for infinities) the
// library routine takes over.
constexpr float kWideReduceMax = 65536.0f;

// sin and cos of a float argument evaluated in double: Cody-Waite reduction by pi/2 (two-part
// constant), then near-minimax polynomials on |r| <= pi/4 (Chebyshev fits of
// (sin r / r - 1) / r^2 and (cos r - 1) / r^2, degree 4 in r^2 each): |error| < 1.4e-14 for sin
// and < 2.3e-13 for cos.  Rounded to float the results agree with correct rounding except in
// a few inputs per million, so s^2 + c^2 - 1 has no systematic bias.  (The library sincosf
// carries a bias of about -1.5e-8 in s^2 + c^2 that compounds into a scale drift along a
// 2000-step chain.)  FP64 FMA issues at the non-packed FP32 rate on CDNA3/4.
// With Checked, |x| > kWideReduceMax takes the library path; kernels that have verified the
// range of a whole chain beforehand call the unchecked form, which keeps the library code out
// of their unrolled loops.  NaN gives NaN on either path.
template <bool Checked = true>
__device__ __forceinline__ void sin_cos_wide(float xf, double& s, double& c) {
  const double x = xf;
  const double k = __builtin_rint(x * 0.63661977236758134308);
  double r = fma(-k, 1.5707963267948966, x);
  r = fma(-k, 6.123233995736766e-17, r);
  const double u = r * r;
  double ps = lin_sk(u, -2.4805636241834762e-08, 2.755599092956532e-06);
  ps = fma_sk(ps, u, -0.00019841266916985966);
  ps = fma_sk(ps, u, 0.008333333331079223);
  ps = fma_sk(ps, u, -0.16666666666663885);
  const double sn = fma(r * u, ps, r);
  double pc = lin_sk(u, -2.7237140418016e-07, 2.4799862190148396e-05);
  pc = fma_sk(pc, u, -0.00138888850913992);
  pc = fma_sk(pc, u, 0.04166666663739607);
  pc = fma_sk(pc, u, -0.4999999999996389);
  const double cs = fma_sk(u, pc, 1.0);
  const int q = static_cast<int>(k) & 3;
  const double so = (q & 1) ? cs : sn;
  const double co = (q & 1) ? sn : cs;
  s = (q & 2) ? -so : so;
  c = ((q + 1) & 2) ? -co : co;
  if constexpr (Checked) {
    if (fabsf(xf) > kWideReduceMax) sincos(x, &s, &c);
  }
}
// sin and cos of a float argument from a 128-entry table and degree-1 polynomials, for the hot
// loops of the forward kernels:
//   t = x * 64/pi + 1.5 * 2^52 rounds k = rint(64 x / pi) into the low mantissa bits of t,
//   r = x - k pi/64 (one-part reduction: |r| <= pi/128, absolute error <= |k| 2^-58, i.e.
//       4.4e-16 for |x| <= 2 pi and 4.7e-12 at kWideReduceMax),
//   sin r = r + s1 r u,  cos r = 1 + w,  w = u (c2 u - 1/2),  u = r^2
//   (s1 the minimax cubic term on |r| <= pi/128, solved for equal-ripple absolute error:
//   |error| < 9.8e-12; c2 a near-minimax fit with the u term held at -1/2, an inline
//   constant: |error| < 3.3e-14),
//   sin x = T_s[k] + T_s[k] w + T_c[k] sin r,  cos x = T_c[k] + T_c[k] w - T_s[k] sin r
// with (T_s, T_c)[j] = (sin, cos)(j pi/64) held in LDS (sin_cos_table_init) and indexed by the
// low 7 bits of t.  No quadrant selects or conversions to integer: 15 VALU issues.  The
// cubic sine keeps sin^2 + cos^2 within 1e-12 of 1 (what would bias a long float chain) and
// each angle within 1e-11; float outputs resolve 6e-8.  Same Checked convention as
// sin_cos_wide.
struct __align__(16) SinCosEntry {
  double s, c;
};
constexpr int kSinCosTable = 128;
__device__ __forceinline__ void sin_cos_table_init(SinCosEntry* table, int tid, int threads) {
  constexpr double kTable[kSinCosTable][2] = {
  {0.0, 1.0},
  {0.049067674327418015, 0.9987954562051724},
  {0.0980171403295606, 0.9951847266721969},
  {0.14673047445536175, 0.989176509964781},
  {0.19509032201612828, 0.9807852804032304},
  {0.2429801799032639, 0.970031253194544},
  {0.2902846772544624, 0.9569403357322088},
  {0.33688985339222005, 0.9415440651830208},
  {0.3826834323650898, 0.9238795325112867},
  {0.4275550934302821, 0.9039892931234433},
  {0.47139673682599764, 0.881921264348355},
  {0.5141027441932218, 0.8577286100002721},
  {0.5555702330196022, 0.8314696123025452},
  {0.5956993044924334, 0.8032075314806449},
  {0.6343932841636455, 0.773010453362737},
  {0.6715589548470184, 0.7409511253549591},
  {0.7071067811865476, 0.7071067811865476},
  {0.7409511253549591, 0.6715589548470184},
  {0.773010453362737, 0.6343932841636455},
  {0.8032075314806449, 0.5956993044924334},
  {0.8314696123025452, 0.5555702330196022},
  {0.8577286100002721, 0.5141027441932218},
  {0.881921264348355, 0.47139673682599764},
  {0.9039892931234433, 0.4275550934302821},
  {0.9238795325112867, 0.3826834323650898},
  {0.9415440651830208, 0.33688985339222005},
  {0.9569403357322088, 0.2902846772544624},
  {0.970031253194544, 0.2429801799032639},
  {0.9807852804032304, 0.19509032201612828},
  {0.989176509964781, 0.14673047445536175},
  {0.9951847266721969, 0.0980171403295606},
  {0.9987954562051724, 0.049067674327418015},
  {1.0, 0.0},
  {0.9987954562051724, -0.049067674327418015},
  {0.9951847266721969, -0.0980171403295606},
  {0.989176509964781, -0.14673047445536175},
  {0.9807852804032304, -0.19509032201612828},
  {0.970031253194544, -0.2429801799032639},
  {0.9569403357322088, -0.2902846772544624},
  {0.9415440651830208, -0.33688985339222005},
  {0.9238795325112867, -0.3826834323650898},
  {0.9039892931234433, -0.4275550934302821},
  {0.881921264348355, -0.47139673682599764},
  {0.8577286100002721, -0.5141027441932218},
  {0.8314696123025452, -0.5555702330196022},
  {0.8032075314806449, -0.5956993044924334},
  {0.773010453362737, -0.6343932841636455},
  {0.7409511253549591, -0.6715589548470184},
  {0.7071067811865476, -0.7071067811865476},
  {0.6715589548470184, -0.7409511253549591},
  {0.6343932841636455, -0.773010453362737},
  {0.5956993044924334, -0.8032075314806449},
  {0.5555702330196022, -0.8314696123025452},
  {0.5141027441932218, -0.8577286100002721},
  {0.47139673682599764, -0.881921264348355},
  {0.4275550934302821, -0.9039892931234433},
  {0.3826834323650898, -0.9238795325112867},
  {0.33688985339222005, -0.9415440651830208},
  {0.2902846772544624, -0.9569403357322088},
  {0.2429801799032639, -0.970031253194544},
  {0.19509032201612828, -0.9807852804032304},
  {0.14673047445536175, -0.989176509964781},
  {0.0980171403295606, -0.9951847266721969},
  {0.049067674327418015, -0.9987954562051724},
  {0.0, -1.0},
  {-0.049067674327418015, -0.9987954562051724},
  {-0.0980171403295606, -0.9951847266721969},
  {-0.14673047445536175, -0.989176509964781},
  {-0.19509032201612828, -0.9807852804032304},
  {-0.2429801799032639, -0.970031253194544},
  {-0.2902846772544624, -0.9569403357322088},
  {-0.33688985339222005, -0.9415440651830208},
  {-0.3826834323650898, -0.9238795325112867},
  {-0.4275550934302821, -0.9039892931234433},
  {-0.47139673682599764, -0.881921264348355},
  {-0.5141027441932218, -0.8577286100002721},
  {-0.5555702330196022, -0.8314696123025452},
  {-0.5956993044924334, -0.8032075314806449},
  {-0.6343932841636455, -0.773010453362737},
  {-0.6715589548470184, -0.7409511253549591},
  {-0.7071067811865476, -0.7071067811865476},
  {-0.7409511253549591, -0.6715589548470184},
  {-0.773010453362737, -0.6343932841636455},
  {-0.8032075314806449, -0.5956993044924334},
  {-0.8314696123025452, -0.5555702330196022},
  {-0.8577286100002721, -0.5141027441932218},
  {-0.881921264348355, -0.47139673682599764},
  {-0.9039892931234433, -0.4275550934302821},
  {-0.9238795325112867, -0.3826834323650898},
  {-0.9415440651830208, -0.33688985339222005},
  {-0.9569403357322088, -0.2902846772544624},
  {-0.970031253194544, -0.2429801799032639},
  {-0.9807852804032304, -0.19509032201612828},
  {-0.989176509964781, -0.14673047445536175},
  {-0.9951847266721969, -0.0980171403295606},
  {-0.9987954562051724, -0.049067674327418015},
  {-1.0, 0.0},
  {-0.9987954562051724, 0.049067674327418015},
  {-0.9951847266721969, 0.0980171403295606},
  {-0.989176509964781, 0.14673047445536175},
  {-0.9807852804032304, 0.19509032201612828},
  {-0.970031253194544, 0.2429801799032639},
  {-0.9569403357322088, 0.2902846772544624},
  {-0.9415440651830208, 0.33688985339222005},
  {-0.9238795325112867, 0.3826834323650898},
  {-0.9039892931234433, 0.4275550934302821},
  {-0.881921264348355, 0.47139673682599764},
  {-0.8577286100002721, 0.5141027441932218},
  {-0.8314696123025452, 0.5555702330196022},
  {-0.8032075314806449, 0.5956993044924334},
  {-0.773010453362737, 0.6343932841636455},
  {-0.7409511253549591, 0.6715589548470184},
  {-0.7071067811865476, 0.7071067811865476},
  {-0.6715589548470184, 0.7409511253549591},
  {-0.6343932841636455, 0.773010453362737},
  {-0.5956993044924334, 0.8032075314806449},
  {-0.5555702330196022, 0.8314696123025452},
  {-0.5141027441932218, 0.8577286100002721},
  {-0.47139673682599764, 0.881921264348355},
  {-0.4275550934302821, 0.9039892931234433},
  {-0.3826834323650898, 0.9238795325112867},
  {-0.33688985339222005, 0.9415440651830208},
  {-0.2902846772544624, 0.9569403357322088},
  {-0.2429801799032639, 0.970031253194544},
  {-0.19509032201612828, 0.9807852804032304},
  {-0.14673047445536175, 0.989176509964781},
  {-0.0980171403295606, 0.9951847266721969},
  {-0.049067674327418015, 0.9987954562051724}};
  for (int j = tid; j < kSinCosTable; j += threads) table[j] = SinCosEntry{kTable[j][0], kTable[j][1]};
}
template <bool Checked = true>
__device__ __forceinline__ void sin_cos_tab(float xf, const SinCosEntry* table, double& s, double& c) {
  constexpr double kRound = 6755399441055744.0;  // 1.5 * 2^52: ulp 1 over [2^52, 2^53)
  const double x = xf;
  const double t = fma(x, 20.371832715762604, kRound);
  const double k = t - kRound;
  const double r = fma(-k, 0.04908738521234052, x);
  const double u = r * r;
  const double sr = fma(r * u, -0.16666230391787032, r);
  const double pc = fma_sk_minus_half(u, 0.04166591860459361);
  const double w = u * pc;
  const SinCosEntry e = table[static_cast<uint32_t>(__builtin_bit_cast(uint64_t, t)) & (kSinCosTable - 1)];
  s = fma(e.s, w, fma(e.c, sr, e.s));
  c = fma(e.c, w, fma(-e.s, sr, e.c));
  if constexpr (Checked) {
    if (fabsf(xf) > kWideReduceMax) sincos(x, &s, &c);
  }
}

template <bool Checked = true>
__device__ __forceinline__ void sin_cos_wide(double x, double& s, double& c) { sincos(x, &s, &c); }

// True when sin_cos_wide<true> would leave its polynomial path for x.
__device__ __forceinline__ bool beyond_wide_reduce(float x) { return fabsf(x) > kWideReduceMax; }
__device__ __forceinline__ bool beyond_wide_reduce(double) { return false; }

// Unit (sin, cos) from a raw pair in double (torsion.cu:119-141 clamps rs^2 + rc^2 at 1e-16).
// For float pairs 1/sqrt comes from the float reciprocal square root refined by one Newton
// step in double (relative error ~1e-14, against a 20-odd instruction double sqrt and
// divide); beyond the float range of rs^2 + rc^2 and for double pairs it is 1/sqrt in double.
template <typename R> __device__ __forceinline__ void pair_unit(R rs, R rc, double& S, double& C) {
  const double a = rs, b = rc;
  const double n2 = a * a + b * b;
  const double eps2 = static_cast<double>(1.0e-8f * 1.0e-8f);
  const double m = n2 < eps2 ? eps2 : n2;
  double rinv;
  if constexpr (sizeof(R) == 4) {
    if (m < 1.0e38) {
      const double r0 = __builtin_amdgcn_rsqf(static_cast<float>(m));
      rinv = r0 * fma(-0.5 * m, r0 * r0, 1.5);
    } else {
      rinv = 1.0 / sqrt(m);
    }
  } else {
    rinv = 1.0 / sqrt(m);
  }
  S = a * rinv;
  C = b * rinv;
}

// Minimum of two bond lengths for the regularity test.  Positive floats order as their bit
// patterns do as integers (one v_min_i32 instead of a canonicalising fmin); a chain with a
// non-positive or NaN length fails that test whatever this returns.
__device__ __forceinline__ float min_positive(float a, float b) {
  return __builtin_bit_cast(float, min(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b)));
}
__device__ __forceinline__ double min_positive(double a, double b) { return fmin(a, b); }

__device__ __forceinline__ float rsqrt_r(float x) { return rsqrtf(x); }
__device__ __forceinline__ double rsqrt_r(double x) { return rsqrt(x); }
// 1/sqrt(x) for the position-based adjoint, whose regularity test keeps x normal: the bare
// v_rsq_f32 (rsqrtf adds a rescaling for denormal x; for normal x the two agree).
__device__ __forceinline__ float rsqrt_bond(float x) { return __builtin_amdgcn_rsqf(x); }
__device__ __forceinline__ double rsqrt_bond(double x) { return rsqrt(x); }

// ------------------------------------------------------------------ small vectors

template <typename R> struct V3 {
  R x, y, z;
};

template <typename R> __device__ __forceinline__ V3<R> operator+(V3<R> a, V3<R> b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
template <typename R> __device__ __forceinline__ V3<R> operator-(V3<R> a, V3<R> b) { return {a.x - b.x, a.y - b.y, a.z - b.z}; }
template <typename R> __device__ __forceinline__ V3<R> operator*(R s, V3<R> a) { return {s * a.x, s * a.y, s * a.z}; }
template <typename R> __device__ __forceinline__ R dot(V3<R> a, V3<R> b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
template <typename R> __device__ __forceinline__ V3<R> cross(V3<R> a, V3<R> b) {
  return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}

// frame_utils.cuh:17-21: v / sqrt(max(v.v, eps)) with eps = 1e-12f.
// v / max(|v|, 1e-6), the norm clamped as the reference clamps |v|^2 at 1e-12
// (frame_utils.cuh:17-31), as v times one reciprocal square root instead of a square root and
// three divisions (within 2 ulp of the quotients).
template <typename R> __device__ __forceinline__ V3<R> normalized(V3<R> v) {
  const R n2 = dot(v, v);
  const R eps = static_cast<R>(1.0e-12f);
  return rsqrt_r(n2 > eps ? n2 : eps) * v;
}

// ------------------------------------------------------------------ rigid transforms

// Rotation (row-major) plus translation.  12 scalars.
template <typename R> struct Rigid {
  R m[9];
  R v[3];
};

template <typename R> __device__ __forceinline__ Rigid<R> rigid_identity() {
  Rigid<R> a;
#pragma unroll
  for (int i = 0; i < 9; ++i) a.m[i] = (i % 4 == 0) ? R(1) : R(0);
  a.v[0] = a.v[1] = a.v[2] = R(0);
  return a;
}

// (a o b): rotation a.m b.m, translation a.v + a.m b.v; a is the earlier transform
// (reference affine.cuh:53-58, scan.cuh:48).
template <typename R> __device__ __forceinline__ Rigid<R> compose(const Rigid<R>& a, const Rigid<R>& b) {
  Rigid<R> o;
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c)
      o.m[3 * r + c] = a.m[3 * r] * b.m[c] + a.m[3 * r + 1] * b.m[3 + c] + a.m[3 * r + 2] * b.m[6 + c];
    o.v[r] = a.v[r] + a.m[3 * r] * b.v[0] + a.m[3 * r + 1] * b.v[1] + a.m[3 * r + 2] * b.v[2];
  }
  return o;
}

template <typename R, typename S> __device__ __forceinline__ Rigid<R> narrow_rigid(const Rigid<S>& a) {
  Rigid<R> o;
#pragma unroll
  for (int i = 0; i < 9; ++i) o.m[i] = static_cast<R>(a.m[i]);
#pragma unroll
  for (int i = 0; i < 3; ++i) o.v[i] = static_cast<R>(a.v[i]);
  return o;
}

template <typename R> __device__ __forceinline__ V3<R> rot_apply(const R (&m)[9], V3<R> x) {
  return {m[0] * x.x + m[1] * x.y + m[2] * x.z, m[3] * x.x + m[4] * x.y + m[5] * x.z, m[6] * x.x + m[7] * x.y + m[8] * x.z};
}

// R <- R * Rx(phi) * Rz(pi - theta), translation += l * (new R)[:,0].
// Equals composing with the reference local transform (affine.cuh:36-45).
template <typename R>
__device__ __forceinline__ void step_forward(R (&m)[9], R (&v)[3], R l, R s, R c, R S, R C) {
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    // Explicit fmas: the compiler has no contraction to choose, so every kernel that runs a
    // step (guarded or not, after step_first or not) rounds it identically.
    const R q0 = m[3 * r], q1 = m[3 * r + 1], q2 = m[3 * r + 2];
    const R a1 = fma(C, q1, S * q2);
    const R a2 = fma(C, q2, -(S * q1));
    const R n0 = fma(s, a1, -(c * q0));
    const R n1 = fma(-s, q0, -(c * a1));
    m[3 * r] = n0;
    m[3 * r + 1] = n1;
    m[3 * r + 2] = a2;
    v[r] = fma(l, n0, v[r]);
  }
}

// step_forward from the identity: R = Rx(phi) * Rz(pi - theta), translation l * R[:,0]
// (the reference local transform, affine.cuh:36-45), without composing onto an identity the
// compiler cannot fold away.  Every value rounds as step_forward's would from the identity, and
// the next step consumes them through explicit fmas only, so kernels that run the loop guarded
// (one basic block per step) or unguarded produce the same bits.
template <typename R>
__device__ __forceinline__ void step_first(R (&m)[9], R (&v)[3], R l, R s, R c, R S, R C) {
  m[0] = -c;
  m[1] = -s;
  m[2] = R(0);
  m[3] = s * C;
  m[4] = -(c * C);
  m[5] = -S;
  m[6] = s * S;
  m[7] = -(c * S);
  m[8] = C;
  v[0] = l * m[0];
  v[1] = l * m[3];
  v[2] = l * m[6];
}

// Inverse of the rotation part of step_forward: R <- R * Rz(pi - theta)^T * Rx(phi)^T.
template <typename R>
__device__ __forceinline__ void step_backward(R (&m)[9], R s, R c, R S, R C) {
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const R n0 = m[3 * r], n1 = m[3 * r + 1], a2 = m[3 * r + 2];
    const R q0 = -(c * n0) - s * n1;
    const R a1 = s * n0 - c * n1;
    m[3 * r] = q0;
    m[3 * r + 1] = C * a1 - S * a2;
    m[3 * r + 2] = S * a1 + C * a2;
  }
}

// ------------------------------------------------------------------ first frame

// block.cu:113-148 compute_first_frame (A.2): p1, p2, d0, t0, d1, frame = [d1 | n x d1 | n].
template <typename R> struct FirstFrame {
  V3<R> p0, p1, p2, d0, t0, d1;
  R frame[9];  // row-major
  R L0, L1, sinA0;
};

template <typename T>
__device__ __forceinline__ FirstFrame<compute_t<T>> first_frame(compute_t<T> L0, compute_t<T> L1, compute_t<T> A0,
                                                                const T* __restrict__ p0, const T* __restrict__ fd,
                                                                const T* __restrict__ n0) {
  using R = compute_t<T>;
  FirstFrame<R> f;
  f.p0 = {widen(p0[0]), widen(p0[1]), widen(p0[2])};
  f.d0 = normalized(V3<R>{widen(fd[0]), widen(fd[1]), widen(fd[2])});
  f.p1 = f.p0 + L0 * f.d0;
  V3<R> nn = {widen(n0[0]), widen(n0[1]), widen(n0[2])};
  nn = nn - dot(nn, f.d0) * f.d0;
  if (dot(nn, nn) < static_cast<R>(1.0e-12f)) {  // block.cu:41,126; frame_utils.cuh:23-31
    const bool use_y = fabs(f.d0.x) >= R(0.9);
    const V3<R> helper = {use_y ? R(0) : R(1), use_y ? R(1) : R(0), R(0)};
    nn = normalized(cross(f.d0, helper));
  } else {
    nn = normalized(nn);
  }
  f.t0 = normalized(cross(nn, f.d0));
  double sd, cd;
  sin_cos_wide(A0, sd, cd);
  const R s = static_cast<R>(sd), c = static_cast<R>(cd);
  f.L0 = L0;
  f.L1 = L1;
  f.sinA0 = s;
  f.d1 = (-c) * f.d0 + s * f.t0;
  f.p2 = f.p1 + L1 * f.d1;
  const V3<R> n = normalized(cross(f.d0, f.d1));
  const V3<R> side = cross(n, f.d1);
  f.frame[0] = f.d1.x; f.frame[1] = side.x; f.frame[2] = n.x;
  f.frame[3] = f.d1.y; f.frame[4] = side.y; f.frame[5] = n.y;
  f.frame[6] = f.d1.z; f.frame[7] = side.z; f.frame[8] = n.z;
  return f;
}

// ------------------------------------------------------------------ wave64 scans

// DPP controls (GFX9 encoding, valid on gfx950).
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;

// Lane value moved by DPP; lanes whose source is outside the pattern (or whose row is
// masked off) receive `old`.
template <int Ctrl, int RowMask>
__device__ __forceinline__ float dpp_move(float old, float src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, src),
                                                               Ctrl, RowMask, 0xf, false));
}
template <int Ctrl, int RowMask> __device__ __forceinline__ int dpp_move(int old, int src) {
  return __builtin_amdgcn_update_dpp(old, src, Ctrl, RowMask, 0xf, false);
}
template <int Ctrl, int RowMask>
__device__ __forceinline__ double dpp_move(double old, double src) {
  const uint64_t o = __builtin_bit_cast(uint64_t, old), x = __builtin_bit_cast(uint64_t, src);
  const int lo = __builtin_amdgcn_update_dpp(static_cast<int>(o), static_cast<int>(x), Ctrl, RowMask, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(static_cast<int>(o >> 32), static_cast<int>(x >> 32), Ctrl, RowMask, 0xf, false);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo));
}

// x of lane ^ D (D < 32) through ds_swizzle's bit mode (and-mask 0x1f, xor-mask D): no
// address register, unlike __shfl_xor's ds_bpermute.
template <int D> __device__ __forceinline__ int lane_xor(int x) {
  static_assert(D > 0 && D < 32, "swizzle masks reach within 32 lanes");
  return __builtin_amdgcn_ds_swizzle(x, 0x1f | (D << 10));
}
template <int D> __device__ __forceinline__ float lane_xor(float x) {
  return __builtin_bit_cast(float, lane_xor<D>(__builtin_bit_cast(int, x)));
}
template <int D> __device__ __forceinline__ double lane_xor(double x) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const int lo = lane_xor<D>(static_cast<int>(u)), hi = lane_xor<D>(static_cast<int>(u >> 32));
  return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo));
}

template <int Ctrl, int RowMask, typename R>
__device__ __forceinline__ Rigid<R> dpp_rigid(const Rigid<R>& x) {
  Rigid<R> y;
#pragma unroll
  for (int i = 0; i < 9; ++i) y.m[i] = dpp_move<Ctrl, RowMask>((i % 4 == 0) ? R(1) : R(0), x.m[i]);
#pragma unroll
  for (int i = 0; i < 3; ++i) y.v[i] = dpp_move<Ctrl, RowMask>(R(0), x.v[i]);
  return y;
}

// Inclusive left-to-right scan of rigid transforms over the 64 lanes of a wave:
// four row_shr rounds inside each 16-lane row, then row_bcast:15 and row_bcast:31.
template <typename R> __device__ __forceinline__ Rigid<R> wave_prefix(Rigid<R> x) {
  x = compose(dpp_rigid<kRowShr1, 0xf>(x), x);
  x = compose(dpp_rigid<kRowShr2, 0xf>(x), x);
  x = compose(dpp_rigid<kRowShr4, 0xf>(x), x);
  x = compose(dpp_rigid<kRowShr8, 0xf>(x), x);
  x = compose(dpp_rigid<kRowBcast15, 0xa>(x), x);
  x = compose(dpp_rigid<kRowBcast31, 0xc>(x), x);
  return x;
}

// One level of wave_prefix for float rigids, as one block of DPP-fused VALU operations: every
// output starts as the lane's own entry, and v_mul/v_fmac with a DPP source (the earlier lane's
// row) overwrite it on lanes whose source is in range (CTRL's row_shr / row_bcast pattern and
// row mask); lanes without a source keep their own transform, the identity composition.  51
// VALU issues against about 62 for compose() over dpp_rigid(), which first copies the 12
// entries with identity defaults.  The s_nop at each end supplies the wait states a DPP read
// needs after a VALU write of its source: the compiler does not count them across inline asm.
#define CUFK_RIGID_DPP_LEVEL(CTRL, x, o) \
  asm("s_nop 1\n" \
      "v_mov_b32 %[o0], %[x0]\n" \
      "v_mul_f32_dpp %[o0], %[x0], %[x0] " CTRL "\n" \
      "v_fmac_f32_dpp %[o0], %[x1], %[x3] " CTRL "\n" \
      "v_fmac_f32_dpp %[o0], %[x2], %[x6] " CTRL "\n" \
      "v_mov_b32 %[o1], %[x1]\n" \
      "v_mul_f32_dpp %[o1], %[x0], %[x1] " CTRL "\n" \
      "v_fmac_f32_dpp %[o1], %[x1], %[x4] " CTRL "\n" \
      "v_fmac_f32_dpp %[o1], %[x2], %[x7] " CTRL "\n" \
      "v_mov_b32 %[o2], %[x2]\n" \
      "v_mul_f32_dpp %[o2], %[x0], %[x2] " CTRL "\n" \
      "v_fmac_f32_dpp %[o2], %[x1], %[x5] " CTRL "\n" \
      "v_fmac_f32_dpp %[o2], %[x2], %[x8] " CTRL "\n" \
      "v_mov_b32 %[o3], %[x3]\n" \
      "v_mul_f32_dpp %[o3], %[x3], %[x0] " CTRL "\n" \
      "v_fmac_f32_dpp %[o3], %[x4], %[x3] " CTRL "\n" \
      "v_fmac_f32_dpp %[o3], %[x5], %[x6] " CTRL "\n" \
      "v_mov_b32 %[o4], %[x4]\n" \
      "v_mul_f32_dpp %[o4], %[x3], %[x1] " CTRL "\n" \
      "v_fmac_f32_dpp %[o4], %[x4], %[x4] " CTRL "\n" \
      "v_fmac_f32_dpp %[o4], %[x5], %[x7] " CTRL "\n" \
      "v_mov_b32 %[o5], %[x5]\n" \
      "v_mul_f32_dpp %[o5], %[x3], %[x2] " CTRL "\n" \
      "v_fmac_f32_dpp %[o5], %[x4], %[x5] " CTRL "\n" \
      "v_fmac_f32_dpp %[o5], %[x5], %[x8] " CTRL "\n" \
      "v_mov_b32 %[o6], %[x6]\n" \
      "v_mul_f32_dpp %[o6], %[x6], %[x0] " CTRL "\n" \
      "v_fmac_f32_dpp %[o6], %[x7], %[x3] " CTRL "\n" \
      "v_fmac_f32_dpp %[o6], %[x8], %[x6] " CTRL "\n" \
      "v_mov_b32 %[o7], %[x7]\n" \
      "v_mul_f32_dpp %[o7], %[x6], %[x1] " CTRL "\n" \
      "v_fmac_f32_dpp %[o7], %[x7], %[x4] " CTRL "\n" \
      "v_fmac_f32_dpp %[o7], %[x8], %[x7] " CTRL "\n" \
      "v_mov_b32 %[o8], %[x8]\n" \
      "v_mul_f32_dpp %[o8], %[x6], %[x2] " CTRL "\n" \
      "v_fmac_f32_dpp %[o8], %[x7], %[x5] " CTRL "\n" \
      "v_fmac_f32_dpp %[o8], %[x8], %[x8] " CTRL "\n" \
      "v_mov_b32 %[o9], %[x9]\n" \
      "v_mov_b32_dpp %[o9], %[x9] " CTRL "\n" \
      "v_fmac_f32_dpp %[o9], %[x0], %[x9] " CTRL "\n" \
      "v_fmac_f32_dpp %[o9], %[x1], %[x10] " CTRL "\n" \
      "v_fmac_f32_dpp %[o9], %[x2], %[x11] " CTRL "\n" \
      "v_mov_b32 %[o10], %[x10]\n" \
      "v_mov_b32_dpp %[o10], %[x10] " CTRL "\n" \
      "v_fmac_f32_dpp %[o10], %[x3], %[x9] " CTRL "\n" \
      "v_fmac_f32_dpp %[o10], %[x4], %[x10] " CTRL "\n" \
      "v_fmac_f32_dpp %[o10], %[x5], %[x11] " CTRL "\n" \
      "v_mov_b32 %[o11], %[x11]\n" \
      "v_mov_b32_dpp %[o11], %[x11] " CTRL "\n" \
      "v_fmac_f32_dpp %[o11], %[x6], %[x9] " CTRL "\n" \
      "v_fmac_f32_dpp %[o11], %[x7], %[x10] " CTRL "\n" \
      "v_fmac_f32_dpp %[o11], %[x8], %[x11] " CTRL "\n" \
      "s_nop 1" \
      : [o0] "=&v"(o.m[0]), [o1] "=&v"(o.m[1]), [o2] "=&v"(o.m[2]), [o3] "=&v"(o.m[3]), [o4] "=&v"(o.m[4]), [o5] "=&v"(o.m[5]), [o6] "=&v"(o.m[6]), [o7] "=&v"(o.m[7]), [o8] "=&v"(o.m[8]), [o9] "=&v"(o.v[0]), [o10] "=&v"(o.v[1]), [o11] "=&v"(o.v[2]) \
      : [x0] "v"(x.m[0]), [x1] "v"(x.m[1]), [x2] "v"(x.m[2]), [x3] "v"(x.m[3]), [x4] "v"(x.m[4]), [x5] "v"(x.m[5]), [x6] "v"(x.m[6]), [x7] "v"(x.m[7]), [x8] "v"(x.m[8]), [x9] "v"(x.v[0]), [x10] "v"(x.v[1]), [x11] "v"(x.v[2]))

// wave_prefix for float rigids (the cross-lane scan of every float and half-type chain).
__device__ __forceinline__ Rigid<float> wave_prefix(Rigid<float> x) {
  Rigid<float> o;
  CUFK_RIGID_DPP_LEVEL("row_shr:1 row_mask:0xf bank_mask:0xf", x, o);
  CUFK_RIGID_DPP_LEVEL("row_shr:2 row_mask:0xf bank_mask:0xf", o, x);
  CUFK_RIGID_DPP_LEVEL("row_shr:4 row_mask:0xf bank_mask:0xf", x, o);
  CUFK_RIGID_DPP_LEVEL("row_shr:8 row_mask:0xf bank_mask:0xf", o, x);
  CUFK_RIGID_DPP_LEVEL("row_bcast:15 row_mask:0xa bank_mask:0xf", x, o);
  CUFK_RIGID_DPP_LEVEL("row_bcast:31 row_mask:0xc bank_mask:0xf", o, x);
  return x;
}
// Inclusive ordered product over each aligned group of G lanes (G a power of two <= 16, so a
// group lies inside one 16-lane DPP row; t = lane % G): wave_prefix's row_shr levels below G.
// A level's DPP source must stay active in EXEC (a disabled source lane reads as out of
// range), so lanes whose source lies in the previous group (t < D) are restored to their own
// transform afterwards, one select per entry; at D = 4 in groups of 8 those lanes are banks 0
// and 2 of each row, which bank_mask leaves unwritten instead.  With G = 16 the row bound
// already excludes them.
template <int G> __device__ __forceinline__ Rigid<float> group_prefix(Rigid<float> x, int t) {
  static_assert(G >= 1 && G <= 16 && (G & (G - 1)) == 0, "groups are powers of two inside one DPP row");
  Rigid<float> o;
  auto keep_own = [&](bool own) {
#pragma unroll
    for (int i = 0; i < 9; ++i) o.m[i] = own ? x.m[i] : o.m[i];
#pragma unroll
    for (int i = 0; i < 3; ++i) o.v[i] = own ? x.v[i] : o.v[i];
  };
  if constexpr (G >= 2) {
    CUFK_RIGID_DPP_LEVEL("row_shr:1 row_mask:0xf bank_mask:0xf", x, o);
    if constexpr (G < 16) keep_own(t < 1);
    x = o;
  }
  if constexpr (G >= 4) {
    CUFK_RIGID_DPP_LEVEL("row_shr:2 row_mask:0xf bank_mask:0xf", x, o);
    if constexpr (G < 16) keep_own(t < 2);
    x = o;
  }
  if constexpr (G == 8) {
    CUFK_RIGID_DPP_LEVEL("row_shr:4 row_mask:0xf bank_mask:0xa", x, o);
    x = o;
  } else if constexpr (G == 16) {
    CUFK_RIGID_DPP_LEVEL("row_shr:4 row_mask:0xf bank_mask:0xf", x, o);
    x = o;
    CUFK_RIGID_DPP_LEVEL("row_shr:8 row_mask:0xf bank_mask:0xf", x, o);
    x = o;
  }
  return x;
}

#undef CUFK_RIGID_DPP_LEVEL

// OR of a predicate over the workgroup: one vote per wave into flags[], then a barrier.
// Uses W words of LDS (the compiler's __syncthreads_or reserves more).
template <int W> __device__ __forceinline__ bool block_any(bool v, int (&flags)[W], int lane, int wave) {
  const bool w = __any(v);
  if (lane == 0) flags[wave] = w ? 1 : 0;
  __syncthreads();
  bool any = false;
#pragma unroll
  for (int i = 0; i < W; ++i) any = any || flags[i] != 0;
  return any;
}

// ------------------------------------------------------------------ lane exchanges
// Every exchange across lanes is a DPP move or a v_readlane (the packed kernels' group
// reductions use ds_swizzle): __shfl_* compiles to ds_bpermute plus VALU instructions for the
// lane address, and waits on an LDS round trip.

constexpr int kRowShl1 = 0x101, kRowShl2 = 0x102, kRowShl4 = 0x104, kRowShl8 = 0x108;
constexpr int kWaveShl1 = 0x130, kWaveShr1 = 0x138;

// v of lane l, in every lane.
__device__ __forceinline__ int lane_value(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float lane_value(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ double lane_value(double v, int l) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_readlane(static_cast<int>(u), l);
  const int hi = __builtin_amdgcn_readlane(static_cast<int>(u >> 32), l);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo));
}

// Value of lane-1 (identity in lane 0), by the wave_shr:1 DPP move.
template <typename R> __device__ __forceinline__ Rigid<R> wave_shift_up(const Rigid<R>& x, int) {
  Rigid<R> y;
#pragma unroll
  for (int i = 0; i < 9; ++i) y.m[i] = dpp_move<kWaveShr1, 0xf>((i % 4 == 0) ? R(1) : R(0), x.m[i]);
#pragma unroll
  for (int i = 0; i < 3; ++i) y.v[i] = dpp_move<kWaveShr1, 0xf>(R(0), x.v[i]);
  return y;
}
// Value of lane-1, and `first` in lane 0 (the same two moves per entry as wave_shift_up).
template <typename R> __device__ __forceinline__ Rigid<R> wave_shift_up_from(const Rigid<R>& x, const Rigid<R>& first) {
  Rigid<R> y;
#pragma unroll
  for (int i = 0; i < 9; ++i) y.m[i] = dpp_move<kWaveShr1, 0xf>(first.m[i], x.m[i]);
#pragma unroll
  for (int i = 0; i < 3; ++i) y.v[i] = dpp_move<kWaveShr1, 0xf>(first.v[i], x.v[i]);
  return y;
}

// Additive force/moment pair (torsion.cu:184-211).
template <typename R> struct ForceMoment {
  V3<R> f, m;
};

// Inclusive right-to-left (suffix) sum over the lanes of a wave: row_shl adds within each row
// of 16 lanes, after which each row's first lane holds the row's total; the totals of the
// later rows are read back and added.
template <typename R> __device__ __forceinline__ R wave_suffix_sum(R x, int lane) {
  x += dpp_move<kRowShl1, 0xf>(R(0), x);  // lane + 1 in the same row, else 0
  x += dpp_move<kRowShl2, 0xf>(R(0), x);
  x += dpp_move<kRowShl4, 0xf>(R(0), x);
  x += dpp_move<kRowShl8, 0xf>(R(0), x);
  const R r3 = lane_value(x, 48);
  const R r2 = lane_value(x, 32) + r3;
  const R r1 = lane_value(x, 16) + r2;
  const int row = lane >> 4;
  return x + (row == 0 ? r1 : row == 1 ? r2 : row == 2 ? r3 : R(0));
}
template <typename R> __device__ __forceinline__ ForceMoment<R> wave_suffix(ForceMoment<R> a, int lane) {
  a.f = {wave_suffix_sum(a.f.x, lane), wave_suffix_sum(a.f.y, lane), wave_suffix_sum(a.f.z, lane)};
  a.m = {wave_suffix_sum(a.m.x, lane), wave_suffix_sum(a.m.y, lane), wave_suffix_sum(a.m.z, lane)};
  return a;
}

// Value of lane+1 (zero in lane 63), by the wave_shl:1 DPP move.
template <typename R> __device__ __forceinline__ ForceMoment<R> wave_shift_down(const ForceMoment<R>& a, int) {
  ForceMoment<R> b;
  b.f = {dpp_move<kWaveShl1, 0xf>(R(0), a.f.x), dpp_move<kWaveShl1, 0xf>(R(0), a.f.y),
         dpp_move<kWaveShl1, 0xf>(R(0), a.f.z)};
  b.m = {dpp_move<kWaveShl1, 0xf>(R(0), a.m.x), dpp_move<kWaveShl1, 0xf>(R(0), a.m.y),
         dpp_move<kWaveShl1, 0xf>(R(0), a.m.z)};
  return b;
}

// Wave-wide reduction along the scan's DPP pattern (row shifts, then the two row
// broadcasts; lane 63 ends with the whole wave), read back to every lane.  Lanes with no DPP
// source receive `none`: the identity of op.
template <typename V, typename Op> __device__ __forceinline__ V wave_reduce(V x, V none, Op op) {
  x = op(x, dpp_move<kRowShr1, 0xf>(none, x));
  x = op(x, dpp_move<kRowShr2, 0xf>(none, x));
  x = op(x, dpp_move<kRowShr4, 0xf>(none, x));
  x = op(x, dpp_move<kRowShr8, 0xf>(none, x));
  x = op(x, dpp_move<kRowBcast15, 0xa>(none, x));
  x = op(x, dpp_move<kRowBcast31, 0xc>(none, x));
  return lane_value(x, 63);
}
template <typename R> __device__ __forceinline__ R wave_sum(R x) {
  return wave_reduce(x, R(0), [](R a, R b) { return a + b; });
}

// Wave-wide minimum of positive values and maximum of non-negative values for the regularity
// test.  Floats reduce as integer min/max of their bit patterns (positive floats order as
// their patterns do; no canonicalising of NaNs as fmin/fmax need).  Other inputs give some
// input's pattern: a chain with a non-positive or NaN length fails the test on its own, and an
// infinite coordinate still compares as the largest.
__device__ __forceinline__ float wave_min_positive(float x) {
  const int r = wave_reduce(__builtin_bit_cast(int, x), 0x7fffffff, [](int a, int b) { return min(a, b); });
  return __builtin_bit_cast(float, r);
}
__device__ __forceinline__ float wave_max_nonneg(float x) {
  const int r = wave_reduce(__builtin_bit_cast(int, x), static_cast<int>(0x80000000u), [](int a, int b) { return max(a, b); });
  return __builtin_bit_cast(float, r);
}
__device__ __forceinline__ double wave_min_positive(double x) {
  return wave_reduce(x, std::numeric_limits<double>::infinity(), [](double a, double b) { return fmin(a, b); });
}
__device__ __forceinline__ double wave_max_nonneg(double x) {
  return wave_reduce(x, 0.0, [](double a, double b) { return fmax(a, b); });
}

template <typename R> __device__ __forceinline__ V3<R> load3(const R* p) { return {p[0], p[1], p[2]}; }

// ------------------------------------------------------------------ workgroup scans

template <typename R, int W>
__device__ __forceinline__ void store_rigid(R (&dst)[W][12], int w, const Rigid<R>& a) {
#pragma unroll
  for (int i = 0; i < 9; ++i) dst[w][i] = a.m[i];
#pragma unroll
  for (int i = 0; i < 3; ++i) dst[w][9 + i] = a.v[i];
}

template <typename R, int W>
__device__ __forceinline__ Rigid<R> load_rigid(const R (&src)[W][12], int w) {
  Rigid<R> a;
#pragma unroll
  for (int i = 0; i < 9; ++i) a.m[i] = src[w][i];
#pragma unroll
  for (int i = 0; i < 3; ++i) a.v[i] = src[w][9 + i];
  return a;
}

// Exclusive prefix of the chain's rigid transforms before this lane's first step:
// wave-level scan, then the totals of earlier waves (scan.cuh:63-101 restated for wave64).
// Lane 0 of each wave starts from `first` (the identity unless the caller prepends a transform
// to the chain: then wave 0 passes it and its lane 0 has already composed it into its total).
// Contains one __syncthreads(); must be called by every thread of the workgroup.
template <typename R, int W>
__device__ __forceinline__ Rigid<R> lane_carry(const Rigid<R>& lane_total, R (&wave_total)[W][12], int lane, int wave,
                                               const Rigid<R>& first = rigid_identity<R>()) {
  const Rigid<R> incl = wave_prefix(lane_total);
  if (lane == 63) store_rigid(wave_total, wave, incl);
  Rigid<R> excl = wave_shift_up_from(incl, first);
  __syncthreads();
  if constexpr (W > 1) {
    if (wave > 0) {
      Rigid<R> carry = load_rigid(wave_total, 0);
#pragma unroll
      for (int w = 1; w < W - 1; ++w)
        if (w < wave) carry = compose(carry, load_rigid(wave_total, w));
      excl = compose(carry, excl);
    }
  }
  return excl;
}

// Exclusive suffix of per-lane force/moment sums (all later lanes of the chain).
// Contains one __syncthreads().
template <typename R, int W>
__device__ __forceinline__ ForceMoment<R> lane_suffix(const ForceMoment<R>& lane_sum, R (&wave_sum)[W][6], int lane,
                                                      int wave) {
  const ForceMoment<R> incl = wave_suffix(lane_sum, lane);
  if (lane == 0) {
    wave_sum[wave][0] = incl.f.x; wave_sum[wave][1] = incl.f.y; wave_sum[wave][2] = incl.f.z;
    wave_sum[wave][3] = incl.m.x; wave_sum[wave][4] = incl.m.y; wave_sum[wave][5] = incl.m.z;
  }
  ForceMoment<R> excl = wave_shift_down(incl, lane);
  __syncthreads();
  if constexpr (W > 1) {
#pragma unroll
    for (int w = 1; w < W; ++w) {
      if (w > wave) {
        excl.f = excl.f + V3<R>{wave_sum[w][0], wave_sum[w][1], wave_sum[w][2]};
        excl.m = excl.m + V3<R>{wave_sum[w][3], wave_sum[w][4], wave_sum[w][5]};
      }
    }
  }
  return excl;
}

}  // namespace cufk_amd
