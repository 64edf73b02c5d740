// Pieces of the fused losses shared by the reconstruct and torsion kernels.
//
// No reference counterpart: the reference returns coordinates and leaves the loss to PyTorch.
// A fused loss reduces a per-chain loss from the positions in registers in the forward, and
// forms grad_xyz from the saved positions and the target inside the backward, so neither the
// loss terms nor grad_xyz ever exist in HBM.
//   kLossSquared     sum_i |x_i - t_i|^2
//   kLossSuperposed  mean squared deviation after optimal superposition (superpose.h), or its
//                    square root (the RMSD)
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

#include "chain_ops.h"
#include "superpose.h"

namespace cufk_amd {

constexpr int kLossNone = 0;
constexpr int kLossSquared = 1;
constexpr int kLossSuperposed = 2;

// Gradient of a fused loss with respect to one point x (target t), formed inside the backward.
struct NoResidual {};
// sum_i |x_i - t_i|^2, times the upstream weight: w2 = 2 w.
template <typename R> struct SquaredResidual {
  R w2;
  __device__ __forceinline__ V3<R> operator()(V3<R> x, V3<R> t) const { return w2 * (x - t); }
};
// The superposed losses: c (x - M t - a) with M = R^T and a = xbar - R^T tbar of the chain's
// optimal superposition, c = (2/N) w for the mean squared deviation (times 1 / (2 rmsd) for
// the RMSD).  Formed in double and rounded once: x, M t and a are each about the chain's
// distance from the origin while the residual is a fraction of a nanometre, and M rounded to
// float would rotate every residual by the same 1e-7 error, which the adjoint's moment sums
// add up along the chain (measured: 9e-5 relative gradient error at N = 2049 against 1e-5
// with the residual in double).
template <typename R> struct SuperposedResidual {
  double c;
  double m[9];
  double a[3];
  __device__ __forceinline__ V3<R> operator()(V3<R> x, V3<R> t) const {
    const double tx = t.x, ty = t.y, tz = t.z;
    const double gx = c * ((static_cast<double>(x.x) - a[0]) - (m[0] * tx + m[1] * ty + m[2] * tz));
    const double gy = c * ((static_cast<double>(x.y) - a[1]) - (m[3] * tx + m[4] * ty + m[5] * tz));
    const double gz = c * ((static_cast<double>(x.z) - a[2]) - (m[6] * tx + m[7] * ty + m[8] * tz));
    return {static_cast<R>(gx), static_cast<R>(gy), static_cast<R>(gz)};
  }
};

// The residual of chain `row` for the loss backward: upstream weight w (grad_loss, or 1).
template <int LossKind, typename R>
__device__ __forceinline__ auto make_residual(R w, const double* __restrict__ record, int points, int squared) {
  if constexpr (LossKind == kLossSuperposed) {
    SuperposedResidual<R> res;
    const double msd = record[12];
    double c = 2.0 * static_cast<double>(w) / points;
    if (!squared) c = msd > 0.0 ? c / (2.0 * sqrt(msd)) : 0.0;
    res.c = c;
#pragma unroll
    for (int k = 0; k < 9; ++k) res.m[k] = record[k];
#pragma unroll
    for (int k = 0; k < 3; ++k) res.a[k] = record[9 + k];
    return res;
  } else {
    return SquaredResidual<R>{R(2) * w};
  }
}

// Per-thread accumulation of a chain's loss from its stored positions xs (rounded to the
// storage type, in the compute type R) and the target t.
//
// The superposed sums are the chain's moments about the shift points cx (its stored x2) and ct
// (the target's point 2), which the solve centres (S = sum x' t'^T - N xbar tbar^T) and cancels
// (msd = (sum |x'|^2 + sum |t'|^2 - 2 lambda) / N, about 250x at N = 2049 with 0.3 nm of noise),
// so their rounding is amplified: summed in float about cx and ct, the products' 1e-7 relative
// rounding at the chain's extent turned the solved rotation by a few 1e-7, which leaves the
// residual with a net torque that the adjoint's moment sums add up along the chain (measured at
// the C2 shape: 1e-4 relative gradient error on 98 of 4096 chains, the RMSD 9e-6 relative off).
// So each thread sums about its own first point and that point's target (xl, tl), which its at
// most 15 points stay within a few nanometres of: the nine products and two squares in R (their
// rounding is now that of a few nm^2), the six first moments in double (they are later
// multiplied by the thread's distance from the chain's centroid).  finish() moves the sums to
// cx and ct in double (superpose_move; e = xl - cx and f = tl - ct are exact there) before the
// cross-thread reduction.  Against all 17 sums in double per point this takes 12 double
// operations per point instead of 33 and no more VGPRs than float sums (measured at the C2
// shape: the RMSD step 2-3 % slower than with float sums, against 9 % all in double).
//
// The float products leave an absolute floor on the MSD: measured at N = 2049 with 1e-3 nm of
// noise (MSD 3e-6 nm^2), 2e-9 nm^2, 7e-4 relative; the RMSD and the scale of its gradient,
// 1 / (2 rmsd), carry half that relative error (2.5e-4 measured).  Chains fitted more closely
// than that have a relatively coarser loss.
template <int LossKind, typename R> struct LossAccumulator {
  static constexpr bool kSuperposed = LossKind == kLossSuperposed;
  double acc = 0.0;
  double s1[kSuperposed ? 6 : 1] = {};   // sum a, sum b (about xl, tl)
  R s2[kSuperposed ? 11 : 1] = {};       // sum a b^T (row-major), sum |a|^2, sum |b|^2
  int m = 0;                             // points summed by this thread
  V3<R> cx = {R(0), R(0), R(0)}, ct = {R(0), R(0), R(0)};  // the chain's shift points
  V3<R> xl = {R(0), R(0), R(0)}, tl = {R(0), R(0), R(0)};  // this thread's

  // Superposed: the chain's shift points, which are also the thread's until local_shift()
  // gives it its own (its first point and that point's target).
  __device__ __forceinline__ void chain_shift(V3<R> x, V3<R> t) {
    cx = xl = x;
    ct = tl = t;
  }
  __device__ __forceinline__ void local_shift(V3<R> x, V3<R> t) {
    xl = x;
    tl = t;
  }

  __device__ __forceinline__ void add(V3<R> xs, V3<R> t) {
    if constexpr (kSuperposed) {
      const V3<R> av = xs - xl, bv = t - tl;
      const R a[3] = {av.x, av.y, av.z}, b[3] = {bv.x, bv.y, bv.z};
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        s1[i] += static_cast<double>(a[i]);
        s1[3 + i] += static_cast<double>(b[i]);
#pragma unroll
        for (int j = 0; j < 3; ++j) s2[3 * i + j] = fma(a[i], b[j], s2[3 * i + j]);
      }
      s2[9] = fma(a[2], a[2], fma(a[1], a[1], fma(a[0], a[0], s2[9])));
      s2[10] = fma(b[2], b[2], fma(b[1], b[1], fma(b[0], b[0], s2[10])));
      ++m;
    } else {
      const V3<R> d = xs - t;
      acc += static_cast<double>(dot(d, d));
    }
  }

  // Workgroup reduction (W waves; contains one __syncthreads), written by thread 0: the sum of
  // squares as the chain's loss, or the superposed sums and shift points into the chain's
  // record, which superpose_records_kernel then solves (it also writes the loss).
  template <typename T, int W>
  __device__ __forceinline__ void finish(T* __restrict__ loss, double* __restrict__ record, int lane, int wave,
                                         int tid) {
    if constexpr (LossKind == kLossSuperposed) {
      // This thread's sums moved to the chain's shift points, in double.
      const double e[3] = {static_cast<double>(xl.x) - static_cast<double>(cx.x),
                           static_cast<double>(xl.y) - static_cast<double>(cx.y),
                           static_cast<double>(xl.z) - static_cast<double>(cx.z)};
      const double f[3] = {static_cast<double>(tl.x) - static_cast<double>(ct.x),
                           static_cast<double>(tl.y) - static_cast<double>(ct.y),
                           static_cast<double>(tl.z) - static_cast<double>(ct.z)};
      double s2d[11];
#pragma unroll
      for (int k = 0; k < 11; ++k) s2d[k] = static_cast<double>(s2[k]);
      double sp[kSuperposeSums];
      superpose_move(s1, s2d, static_cast<double>(m), e, f, sp);
      __shared__ double part[W][kSuperposeSums];
#pragma unroll
      for (int k = 0; k < kSuperposeSums; ++k) {
        const double v = wave_sum(sp[k]);
        if (lane == 0) part[wave][k] = v;
      }
      __syncthreads();
      if (tid < kSuperposeSums) {
        double sum = 0.0;
#pragma unroll
        for (int w = 0; w < W; ++w) sum += part[w][tid];
        record[tid] = sum;
      } else if (tid < kSuperposeSums + 6) {
        const int k = tid - kSuperposeSums;
        const V3<R> c = k < 3 ? cx : ct;
        record[tid] = static_cast<double>(k % 3 == 0 ? c.x : (k % 3 == 1 ? c.y : c.z));
      }
    } else {
      __shared__ double part[W];
      const double v = wave_sum(acc);
      if (lane == 0) part[wave] = v;
      __syncthreads();
      if (tid == 0) {
        double sum = 0.0;
#pragma unroll
        for (int w = 0; w < W; ++w) sum += part[w];
        *loss = narrow<T>(static_cast<R>(sum));
      }
    }
  }
};

}  // namespace cufk_amd

namespace cufk_amd {

// One thread per chain: solve the superposition from the sums the fused forward stored in the
// chain's record (superpose.h), replace them with the record the backward reads, and write the
// loss: the mean squared deviation, or its square root unless `squared`.  A separate launch keeps
// the 4x4 eigenproblem, a serial chain of double operations, out of the forward's workgroups.
constexpr int kSolveThreads = 256;
template <typename T>
__global__ __launch_bounds__(kSolveThreads) void superpose_records_kernel(double* __restrict__ record,
                                                                          T* __restrict__ loss, int64_t batch,
                                                                          int points, int squared) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * kSolveThreads + threadIdx.x;
  if (b >= batch) return;
  double rec[kSuperposeRecord];
  double* const r = record + b * kSuperposeRecord;
#pragma unroll
  for (int k = 0; k < kSuperposeRecord; ++k) rec[k] = r[k];
  superpose_solve_record(rec, points);
#pragma unroll
  for (int k = 0; k < kSuperposeRecord; ++k) r[k] = rec[k];
  using R = compute_t<T>;
  loss[b] = narrow<T>(static_cast<R>(squared ? rec[12] : sqrt(rec[12])));
}

}  // namespace cufk_amd
