// Reconstruction kernels (reference: src/cufk/csrc/block.cu).
//
// One workgroup of W wave64s per chain; lane t owns steps [tK, tK+K) (point s+3 for step s).
//   reconstruct_forward_kernel     block_forward_kernel (block.cu:157-204)
//   reconstruct_backward_saved     block_backward_kernel (block.cu:230-313) given the forward's
//                                  output: the world-frame force/moment adjoint over the saved
//                                  positions (the form torsion.cu:204-217 uses) for chains the
//                                  forward marked regular, the exact recompute for the others
//   reconstruct_backward_recompute block_backward_kernel without a saved output: the forward
//                                  scan rerun in registers, then the same adjoint over those
//                                  positions (exact recompute for irregular chains)
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <limits>
#include <type_traits>

#include "chain_ops.h"
#include "fused_loss.h"
#include "staging.h"

namespace cufk_amd {

// When the position-based adjoint is accurate: every bond length positive, every bond angle
// with sin >= kSinMin, and every coordinate within kScale shortest bonds of the origin (the
// stored positions then resolve bond directions to about kScale ulp / bond).  The shortest
// bond is also at least kMinLength, which keeps every squared bond length and squared bond
// normal that the adjoint normalises far from the denormal range (rsqrt_bond), and every
// coordinate at most kMaxExtent, which keeps them below the largest finite value (bonds are
// then at most 2 sqrt(3) kMaxExtent long).  float16/bfloat16 outputs are too coarse for it;
// their float copy (reconstruct_forward_shadow_kernel) takes the float test.
template <typename T> struct FastPath {
  static constexpr bool kEnabled = false;
  static constexpr double kSinMin = 2.0;
  static constexpr double kScale = 0.0;
  static constexpr double kMinLength = 0.0;
  static constexpr double kMaxExtent = 0.0;
};
template <> struct FastPath<float> {
  static constexpr bool kEnabled = true;
  static constexpr double kSinMin = 0.5;
  static constexpr double kScale = 256.0;
  static constexpr double kMinLength = 0x1p-20;  // |b|^2 >= 2^-40, |b1 x b2|^2 >= 2^-82
  static constexpr double kMaxExtent = 0x1p29;   // |b|^2 <= 12 * 2^58, |b1 x b2|^2 <= 2^123.2 < FLT_MAX
};
template <> struct FastPath<double> {
  static constexpr bool kEnabled = true;
  static constexpr double kSinMin = 1.0e-2;
  static constexpr double kScale = 8192.0;
  static constexpr double kMinLength = 0.0;  // the double adjoint keeps the library rsqrt
  static constexpr double kMaxExtent = 0x1p250;
};

// The extent tests of the fast path for a chain with largest |coordinate| xmax and shortest
// bond lmin (the bond and angle tests are separate).
template <typename Fast, typename R> __device__ __forceinline__ bool fast_extent_ok(R xmax, R lmin) {
  return xmax <= static_cast<R>(Fast::kScale) * lmin && lmin >= static_cast<R>(Fast::kMinLength) &&
         xmax <= static_cast<R>(Fast::kMaxExtent);
}

template <typename R> __device__ __forceinline__ R abs_max3(R m, V3<R> x) {
  m = fmax(m, fabs(x.x));
  m = fmax(m, fabs(x.y));
  return fmax(m, fabs(x.z));
}

// total = excl o q in double (row-major rotation, then translation).
template <typename R>
__device__ __forceinline__ void store_total(double* __restrict__ total, const Rigid<R>& excl, const Rigid<double>& q) {
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c)
      total[3 * r + c] = static_cast<double>(excl.m[3 * r]) * q.m[c] + static_cast<double>(excl.m[3 * r + 1]) * q.m[3 + c] +
                         static_cast<double>(excl.m[3 * r + 2]) * q.m[6 + c];
    total[9 + r] = static_cast<double>(excl.v[r]) + static_cast<double>(excl.m[3 * r]) * q.v[0] +
                   static_cast<double>(excl.m[3 * r + 1]) * q.v[1] + static_cast<double>(excl.m[3 * r + 2]) * q.v[2];
  }
}

// Per-chain sums for the anchor gradients, written by the thread that computes the
// first-frame terms: F = sum_i g_i over all points and tau = sum_i (x_i - p0) x g_i, from the
// sums over points >= 3 the adjoint ends with (F3, and M3 about x2) and points 0..2 relative to
// x2 (P0 = p0 - x2, P1 = x1 - x2, x2 itself at the origin).
template <typename R>
__device__ __forceinline__ void store_anchor_sums(double* __restrict__ out, V3<R> F3, V3<R> M3, V3<R> P0, V3<R> P1,
                                                  V3<R> g0, V3<R> g1, V3<R> g2) {
  const V3<R> f = F3 + g0 + g1 + g2;
  const V3<R> tau = M3 - cross(P0, F3) + cross(P1 - P0, g1) - cross(P0, g2);
  out[0] = f.x;
  out[1] = f.y;
  out[2] = f.z;
  out[3] = tau.x;
  out[4] = tau.y;
  out[5] = tau.z;
}

// ============================================================================ lane scan

// Lane-serial scan of one lane's K items in double: q is the lane-local prefix transform and
// y[i] its translation after item i, rounded to R.  Item i reads its (length, angle,
// dihedral) from Ls[i], As[i], Ds[i] (the lane's run of three step-layout LDS rows).  With
// Guard only items < count run; without it every item runs, and the caller has padded the
// lane's tail (pad_lane_tail) or ignores the lane.  ok and lmin accumulate the regularity
// tests (Fast::kSinMin).  With Table, float angles take sin/cos from the LDS table.  Checked
// selects the sin/cos form that handles angles beyond kWideReduceMax.  Every item is a
// scheduling region of its own, which keeps the independent sin/cos of later items from being
// hoisted (and held in registers) where the compiler would otherwise do so.
template <typename T, int K, bool Checked, bool Guard, bool Table, typename Fast = FastPath<T>>
__device__ __forceinline__ void lane_scan(const compute_t<T>* Ls, const compute_t<T>* As, const compute_t<T>* Ds,
                                          int count, const SinCosEntry* table, Rigid<double>& q,
                                          compute_t<T> (&y)[K][3], bool& ok, compute_t<T>& lmin) {
  using R = compute_t<T>;
  // Each item's parameters are read from LDS one item ahead, so that their latency overlaps
  // the previous item's arithmetic (C2 forward 48.2 -> 47.5 us, same outputs).
  R ln = Ls[0], an = As[0], dn = Ds[0];
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (!Guard || i < count) {
      const R l = ln, a = an, d = dn;
      if (i + 1 < K) {
        ln = Ls[i + 1];
        an = As[i + 1];
        dn = Ds[i + 1];
      }
      double s, c, S, C;
      if constexpr (Table && sizeof(R) == 4) {
        sin_cos_tab<Checked>(a, table, s, c);
        sin_cos_tab<Checked>(d, table, S, C);
      } else {
        sin_cos_wide<Checked>(a, s, c);
        sin_cos_wide<Checked>(d, S, C);
      }
      if (i == 0)
        step_first(q.m, q.v, static_cast<double>(l), s, c, S, C);
      else
        step_forward(q.m, q.v, static_cast<double>(l), s, c, S, C);
      ok = ok && l > R(0) && s >= Fast::kSinMin;
      lmin = min_positive(lmin, l);
    }
    y[i][0] = static_cast<R>(q.v[0]);
    y[i][1] = static_cast<R>(q.v[1]);
    y[i][2] = static_cast<R>(q.v[2]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The lane holding the chain's last step pads the rest of its items in the three step rows
// with steps that pass the regularity tests (longest bond, right angle, no twist), so that
// lane_scan can run every item unguarded; they follow the chain's last point and feed
// nothing that is stored.  Call before the barrier that publishes the rows.
template <int K, typename R>
__device__ __forceinline__ void pad_lane_tail(R* Ls, R* As, R* Ds, int count) {
  if (count > 0 && count < K) {
    for (int i = count; i < K; ++i) {
      Ls[i] = std::numeric_limits<R>::max();
      As[i] = R(1.5707963267948966);
      Ds[i] = R(0);
    }
  }
}

// lane_scan over a whole chain: the hot instance unguarded (lanes past the chain scan garbage
// that reaches no stored point and reset their flags), the library-sin/cos instance guarded and
// one region per item (unguarded or unscheduled it needs more registers than the hot one).  No
// wave skips the scan: every plan (with_scan_plan) gives each of its waves some of the chain's
// steps, and a skip would cost every wave the registers' defaults for the waves that take it
// (36 VALU per wave at C2).  q needs no starting value: each lane's first item sets it
// (step_first), and lanes past the chain feed only later lanes, which store nothing either.
template <typename T, int K, bool Table, typename Fast = FastPath<T>>
__device__ __forceinline__ void lane_scan_chain(const compute_t<T>* Ls, const compute_t<T>* As,
                                                const compute_t<T>* Ds, int count, bool wide,
                                                const SinCosEntry* table, Rigid<double>& q, compute_t<T> (&y)[K][3],
                                                bool& ok, compute_t<T>& lmin) {
  if (wide)  // uniform per workgroup
    lane_scan<T, K, true, true, Table, Fast>(Ls, As, Ds, count, table, q, y, ok, lmin);
  else
    lane_scan<T, K, false, false, Table, Fast>(Ls, As, Ds, count, table, q, y, ok, lmin);
  if (count <= 0) {
    ok = true;
    lmin = compute_t<T>(1.0e30);
  }
}

// ============================================================================ forward

// x0 = p0, x1, x2 from the first frame (block.cu:113-155), x_{k+3} = p2 + F P_k.v, for one
// chain (Lr, Ar, Dr: its parameter rows, out: its (points, 3) row).  When `regular` is
// non-null, *regular receives the fast-path predicate for the chain.  Rows are staged through
// LDS (coalesced 16-byte streams in and out).
//
// Segmented: the rows are a segment of a longer chain, seen as a chain of its own whose
// points 0..2 are the three points before the segment.  The first segment (head) runs as a
// whole chain; the others start from the identity frame at the origin, so they write their
// points in the frame of the segment start (x2 of the view) and leave points 0..2 alone.
// Every segment writes its total transform (row-major rotation, then translation; double) to
// total[0..11].
//
// Loss (kLossSquared): *loss also receives sum_i |x_i - target_i|^2 over the chain's points
// (target: the chain's (points, 3) row), from the positions as stored (rounded to T),
// accumulated in double.  kLossSuperposed: record receives the sums and shift points of the
// optimal superposition of the stored positions onto the target, which
// superpose_records_kernel solves into the loss and the record the backward needs.
//
// Shadow (float16/bfloat16 whole chains): the positions are also stored unrounded, in float,
// to shadow (the chain's (points, 3) row), and *regular receives the float32 chains' test
// (FastPath<float>) on them, for the position-based backward over that copy.
template <typename T, typename Lay, bool Segmented, int LossKind = kLossNone, bool Shadow = false>
__device__ __forceinline__ void forward_chain(const T* __restrict__ Lr, const T* __restrict__ Ar,
                                              const T* __restrict__ Dr, const T* __restrict__ p0,
                                              const T* __restrict__ first_direction,
                                              const T* __restrict__ initial_normal, T* __restrict__ out,
                                              uint8_t* __restrict__ regular, int points, bool head,
                                              double* __restrict__ total, const T* __restrict__ target = nullptr,
                                              T* __restrict__ loss = nullptr, float* __restrict__ shadow = nullptr,
                                              double* __restrict__ record = nullptr) {
  using R = compute_t<T>;
  constexpr bool Loss = LossKind != kLossNone;
  constexpr bool Superposed = LossKind == kLossSuperposed;
  static_assert(!Loss || !Segmented, "the fused losses take whole chains");
  static_assert(!Shadow || (!Segmented && !Loss && std::is_same_v<R, float>), "shadow rows: whole half-type chains");
  using Fast = std::conditional_t<Shadow, FastPath<R>, FastPath<T>>;
  constexpr int W = Lay::kWaves;
  constexpr int K = Lay::kItems;
  constexpr int kStage = 3 * Lay::kStepRow > Lay::kPointRow ? 3 * Lay::kStepRow : Lay::kPointRow;
  __shared__ __align__(16) R stage[kStage];
  __shared__ R wave_total[W][12];
  __shared__ R base[12];  // first-frame rotation (row-major) and p2
  __shared__ R wave_stat[W][3];
  __shared__ int wide_vote[W];
  __shared__ SinCosEntry sc_table[kSinCosTable];

  const int steps = points - 3;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int s0 = tid * K;
  const int count = steps - s0 < K ? steps - s0 : K;  // items of this lane (may be <= 0)
  const int b0 = Lay::lane_step_base(tid);

  bool wide;  // some angle of the chain needs the library sin/cos
  {
    R* const dst[3] = {stage, stage + Lay::kStepRow, stage + 2 * Lay::kStepRow};
    const T* const src[3] = {Lr + 2, Ar + 1, Dr};
    wide = load_step_rows<Lay, 3, 0b110u>(dst, src, steps, tid);
  }
  if constexpr (sizeof(R) == 4) sin_cos_table_init(sc_table, tid, Lay::kLanes);
  if constexpr (!Segmented) pad_lane_tail<K>(stage + b0, stage + Lay::kStepRow + b0, stage + 2 * Lay::kStepRow + b0, count);
  // Loss: the target of the lane's own points, loaded now so that the scan hides the latency.
  R tr[Loss ? 3 * K : 1];
  if constexpr (Loss) load_run<3 * K>(target + 9 + 3 * s0, count > 0 ? 3 * count : 0, tr);
  wide = block_any<W>(wide, wide_vote, lane, wave);

  // Lane-local serial scan in double (rounding only at the lane boundary); y[i] is the
  // translation of the lane-local prefix after item i.  Items are read from LDS as the scan
  // reaches them, so only y stays in registers.  Segments run it guarded: their last lane's
  // total transform is stored.  Measured at C2 (5 waves per SIMD), the table beats
  // sin_cos_wide (56.5 against 58.2 us).
  Rigid<double> q;  // set by each lane's first step (step_first, lane_scan_chain)
  R y[K][3];
  bool ok = true;
  R lmin = R(1.0e30);
  {
    const R* const Ls = stage + b0;
    const R* const As = stage + Lay::kStepRow + b0;
    const R* const Ds = stage + 2 * Lay::kStepRow + b0;
    constexpr bool kTable = sizeof(R) == 4;
    if constexpr (Segmented) {
      if (wide)
        lane_scan<T, K, true, true, kTable>(Ls, As, Ds, count, sc_table, q, y, ok, lmin);
      else if ((wave + 1) * 64 * K <= steps)  // every lane of the wave has K steps: no guard
        lane_scan<T, K, false, false, kTable>(Ls, As, Ds, count, sc_table, q, y, ok, lmin);
      else
        lane_scan<T, K, false, true, kTable>(Ls, As, Ds, count, sc_table, q, y, ok, lmin);
    } else {
      lane_scan_chain<T, K, kTable, Fast>(Ls, As, Ds, count, wide, sc_table, q, y, ok, lmin);
    }
  }

  // The first frame (block.cu:113-148) after the lane scan: no other wave waits on it before
  // lane_carry's barrier, which publishes base[].
  FirstFrame<R> ff;
  if (wave == 0) {
    if (!Segmented || head) {
      ff = first_frame<T>(widen(Lr[0]), widen(Lr[1]), widen(Ar[0]), p0, first_direction, initial_normal);
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < 9; ++i) base[i] = ff.frame[i];
        base[9] = ff.p2.x;
        base[10] = ff.p2.y;
        base[11] = ff.p2.z;
      }
    } else if (lane == 0) {
#pragma unroll
      for (int i = 0; i < 12; ++i) base[i] = (i == 0 || i == 4 || i == 8) ? R(1) : R(0);
    }
  }

  // Segments: the lane with the last step parks its double transform in LDS for the segment's
  // total, so that no lane holds it in registers across the carry (107 -> 88 VGPRs).
  __shared__ double last_q[Segmented ? 12 : 1];
  const bool last_lane = count > 0 && count + s0 == steps;
  if constexpr (Segmented) {
    if (last_lane) {
#pragma unroll
      for (int i = 0; i < 9; ++i) last_q[i] = q.m[i];
#pragma unroll
      for (int i = 0; i < 3; ++i) last_q[9 + i] = q.v[i];
    }
  }
  // The first frame's rotation F enters the scan once, composed into the total of the chain's
  // first lane (and given to that lane as its exclusive prefix), so every lane's prefix comes
  // out as its world rotation and translation relative to x2, and no lane applies F afterwards
  // (36 VALU once per workgroup instead of once per wave).  Explicit fmas, so that every kernel
  // instance rounds the positions alike.  A segment after the head has F = identity; the head
  // segment's total then includes F, which long_forward_frames_kernel accounts for.
  Rigid<R> lane_total = narrow_rigid<R>(q);
  Rigid<R> first = rigid_identity<R>();
  if (wave == 0 && (!Segmented || head)) {
    const R* const Fr = ff.frame;
#pragma unroll
    for (int i = 0; i < 9; ++i) first.m[i] = Fr[i];
    if (lane == 0) {
      const Rigid<R> t = lane_total;
#pragma unroll
      for (int r = 0; r < 3; ++r) {
#pragma unroll
        for (int c = 0; c < 3; ++c)
          lane_total.m[3 * r + c] = fma(Fr[3 * r + 2], t.m[6 + c], fma(Fr[3 * r + 1], t.m[3 + c], Fr[3 * r] * t.m[c]));
        lane_total.v[r] = fma(Fr[3 * r + 2], t.v[2], fma(Fr[3 * r + 1], t.v[1], Fr[3 * r] * t.v[0]));
      }
    }
  }
  // lane_carry's barrier also publishes base[] and retires every read of the staged step
  // rows, which the point row below overwrites.
  const Rigid<R> excl = lane_carry<R, W>(lane_total, wave_total, lane, wave, first);
  if constexpr (Segmented) {
    if (last_lane) {
      Rigid<double> qt;
#pragma unroll
      for (int i = 0; i < 9; ++i) qt.m[i] = last_q[i];
#pragma unroll
      for (int i = 0; i < 3; ++i) qt.v[i] = last_q[9 + i];
      store_total(total, excl, qt);
    }
  }
  const V3<R> p2 = {base[9], base[10], base[11]};

  // World transform at the lane start: (F, p2) o excl, with F already inside excl.
  R gm[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) gm[i] = excl.m[i];
  const V3<R> gv = {p2.x + excl.v[0], p2.y + excl.v[1], p2.z + excl.v[2]};

  R xmax = R(0);
  // The fused loss's share of this thread; superposed sums about the stored x2 and the
  // target's point 2 for the chain, the thread's first point and its target for the thread.
  LossAccumulator<LossKind, R> lossacc;
  if constexpr (Superposed) {
    lossacc.chain_shift(V3<R>{widen(narrow<T>(p2.x)), widen(narrow<T>(p2.y)), widen(narrow<T>(p2.z))},
                        V3<R>{widen(target[6]), widen(target[7]), widen(target[8])});
  }
  {
    const int o0 = Lay::lane_point_base(tid);
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (i < count) {
        // gv as the addend of the first fma: three issues per coordinate, not four.
        const V3<R> x = {fma(gm[2], y[i][2], fma(gm[1], y[i][1], fma(gm[0], y[i][0], gv.x))),
                         fma(gm[5], y[i][2], fma(gm[4], y[i][1], fma(gm[3], y[i][0], gv.y))),
                         fma(gm[8], y[i][2], fma(gm[7], y[i][1], fma(gm[6], y[i][0], gv.z)))};
        if constexpr (Loss) {
          const V3<R> xs = {widen(narrow<T>(x.x)), widen(narrow<T>(x.y)), widen(narrow<T>(x.z))};
          if constexpr (Superposed) {
            if (i == 0) lossacc.local_shift(xs, V3<R>{tr[0], tr[1], tr[2]});
          }
          lossacc.add(xs, V3<R>{tr[3 * i], tr[3 * i + 1], tr[3 * i + 2]});
        }
        stage[o0 + 3 * i] = x.x;
        stage[o0 + 3 * i + 1] = x.y;
        stage[o0 + 3 * i + 2] = x.z;
        xmax = abs_max3(xmax, x);
      }
    }
    if (tid == 0 && (!Segmented || head)) {
      if constexpr (Loss) {
        const V3<R> h[3] = {ff.p0, ff.p1, ff.p2};
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const V3<R> xs = {widen(narrow<T>(h[j].x)), widen(narrow<T>(h[j].y)), widen(narrow<T>(h[j].z))};
          lossacc.add(xs, V3<R>{widen(target[3 * j]), widen(target[3 * j + 1]), widen(target[3 * j + 2])});
        }
      }
      stage[0] = ff.p0.x; stage[1] = ff.p0.y; stage[2] = ff.p0.z;
      stage[3] = ff.p1.x; stage[4] = ff.p1.y; stage[5] = ff.p1.z;
      stage[6] = ff.p2.x; stage[7] = ff.p2.y; stage[8] = ff.p2.z;
    }
  }
  if constexpr (Fast::kEnabled) {
    if (regular != nullptr) {
      const bool wave_ok = __all(ok);
      const R wmin = wave_min_positive(lmin);
      const R wmax = wave_max_nonneg(xmax);
      if (lane == 0) {
        wave_stat[wave][0] = wave_ok ? R(1) : R(0);
        wave_stat[wave][1] = wmin;
        wave_stat[wave][2] = wmax;
      }
    }
  }
  __syncthreads();
  if (regular != nullptr && tid == 0) {
    bool reg = false;
    if constexpr (Fast::kEnabled) {
      // A segment after the head has no first frame: its own steps and local positions only.
      R m = R(1.0e30), x = R(0);
      reg = true;
      if (!Segmented || head) {
        reg = ff.L0 > R(0) && ff.L1 > R(0) && ff.sinA0 >= Fast::kSinMin;
        m = fmin(ff.L0, ff.L1);
        x = abs_max3(abs_max3(abs_max3(R(0), ff.p0), ff.p1), ff.p2);
      }
#pragma unroll
      for (int w = 0; w < W; ++w) {
        reg = reg && wave_stat[w][0] != R(0);
        m = fmin(m, wave_stat[w][1]);
        x = fmax(x, wave_stat[w][2]);
      }
      reg = reg && fast_extent_ok<Fast>(x, m);
    }
    *regular = reg ? 1 : 0;
  }
  if constexpr (Loss) lossacc.template finish<T, W>(loss, record, lane, wave, tid);
  // A half-type chain's backward reads the float copy, not the rounded output.
  store_point_row<Lay, Shadow>(out, stage, points, tid, !Segmented || head);
  if constexpr (Shadow) store_point_row<Lay>(shadow, stage, points, tid);
}

template <typename T, int W, int K, int Pad = 4>
__global__ __launch_bounds__(64 * W) void reconstruct_forward_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    T* __restrict__ xyz, uint8_t* __restrict__ regular, int points) {
  const int64_t row = blockIdx.x;
  forward_chain<T, Layout<W, K, Pad>, false, kLossNone, false>(lengths + row * (points - 1), angles + row * (points - 2),
                                             dihedrals + row * (points - 3), p0, first_direction, initial_normal,
                                             xyz + row * points * 3, regular != nullptr ? regular + row : nullptr,
                                             points, true, nullptr);
}

// The forward of a float16/bfloat16 chain that also keeps its positions in float (shadow, a
// (B, N, 3) float array) and flags the chains whose backward may take the position-based
// adjoint over them.
template <typename T, int W, int K, int Pad>
__global__ __launch_bounds__(64 * W) void reconstruct_forward_shadow_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    T* __restrict__ xyz, float* __restrict__ shadow, uint8_t* __restrict__ regular, int points) {
  const int64_t row = blockIdx.x;
  forward_chain<T, Layout<W, K, Pad>, false, kLossNone, true>(
      lengths + row * (points - 1), angles + row * (points - 2), dihedrals + row * (points - 3), p0, first_direction,
      initial_normal, xyz + row * points * 3, regular + row, points, true, nullptr, nullptr, nullptr,
      shadow + row * points * 3);
}

// ============================================================================ exact backward

// World-frame adjoint with exact frame axes for one chain, recomputing the forward scan from
// the parameters (valid for every finite input):
//   F_i = sum_{j>=i} g_j,  M_i = sum_{j>=i} x_j x g_j,  tau = M_{k+3} - x_{k+2} x F_{k+3}
//   dL/dL[k+2] = R_k[:,0].F_{k+3},  dL/dA[k+1] = -R_k[:,2].tau,  dL/dD[k] = R_{k-1}[:,0].tau
// with R_k the world rotation after step k; first-frame terms restate block.cu:206-228.
// Positions are relative to x2 (the moments are translation invariant).  Every thread of
// the workgroup calls this; pstage holds 3 step rows, gstage one point row.  The reverse walk
// recomputes each step's sin/cos instead of keeping them in registers, so this path does not
// raise the register count of a kernel that also carries the position-based path.
//
// Segmented: the rows are a segment of a longer chain (as in forward_chain).  A segment other
// than the first (head) starts from the world rotation frame[0..8] (row-major) at its x2,
// and carry[0..5] holds F and M (about that x2) of every point after the segment; only the
// head writes the first-frame terms.
template <typename T, typename Lay, bool Segmented = false, bool StageGrad = true>
__device__ __forceinline__ void exact_chain(const T* __restrict__ Lr, const T* __restrict__ Ar,
                                            const T* __restrict__ Dr, const T* __restrict__ p0,
                                            const T* __restrict__ first_direction,
                                            const T* __restrict__ initial_normal, const T* __restrict__ Gr,
                                            T* __restrict__ gLr, T* __restrict__ gAr, T* __restrict__ gDr,
                                            compute_t<T>* pstage, compute_t<T>* gstage,
                                            compute_t<T> (&wave_total)[Lay::kWaves][12],
                                            compute_t<T> (&wave_sum)[Lay::kWaves][6], int (&wide_vote)[Lay::kWaves],
                                            int points, bool head = true, const double* __restrict__ frame = nullptr,
                                            const double* __restrict__ carry = nullptr,
                                            double* __restrict__ anchor = nullptr) {
  using R = compute_t<T>;
  constexpr int W = Lay::kWaves;
  constexpr int K = Lay::kItems;
  const int steps = points - 3;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int s0 = tid * K;
  const int b0 = Lay::lane_step_base(tid);
  const int o0 = Lay::lane_point_base(tid);
  bool wide;  // some angle of the chain needs the library sin/cos
  {
    R* const dst[3] = {pstage, pstage + Lay::kStepRow, pstage + 2 * Lay::kStepRow};
    const T* const src[3] = {Lr + 2, Ar + 1, Dr};
    wide = load_step_rows<Lay, 3, 0b110u>(dst, src, steps, tid);
    if constexpr (StageGrad) {  // otherwise the caller left the gradient row in gstage
      R* const gdst[1] = {gstage};
      const T* const gsrc[1] = {Gr};
      load_point_rows<Lay, 1>(gdst, gsrc, points, tid);
    }
  }
  FirstFrame<R> ff;
  R Fm[9];  // world rotation at x2
  if (!Segmented || head) {
    ff = first_frame<T>(widen(Lr[0]), widen(Lr[1]), widen(Ar[0]), p0, first_direction, initial_normal);
#pragma unroll
    for (int i = 0; i < 9; ++i) Fm[i] = ff.frame[i];
  } else {
#pragma unroll
    for (int i = 0; i < 9; ++i) Fm[i] = static_cast<R>(frame[i]);
  }
  wide = block_any<W>(wide, wide_vote, lane, wave);

  // Pass 1: lane-local scan (double); Y = sum_i y_i g_i^T and sum_i g_i.
  Rigid<double> qd = rigid_identity<double>();
  R Y[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) Y[i] = R(0);
  V3<R> gsum = {R(0), R(0), R(0)};
  auto pass1 = [&]<bool Checked>() {
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (s0 + i < steps) {
        const R l = pstage[b0 + i];
        double s, c, S, C;
        sin_cos_wide<Checked>(pstage[Lay::kStepRow + b0 + i], s, c);
        sin_cos_wide<Checked>(pstage[2 * Lay::kStepRow + b0 + i], S, C);
        step_forward(qd.m, qd.v, static_cast<double>(l), s, c, S, C);
        const V3<R> g = load3(&gstage[o0 + 3 * i]);
        const R yv[3] = {static_cast<R>(qd.v[0]), static_cast<R>(qd.v[1]), static_cast<R>(qd.v[2])};
#pragma unroll
        for (int a = 0; a < 3; ++a) {
          Y[3 * a + 0] += yv[a] * g.x;
          Y[3 * a + 1] += yv[a] * g.y;
          Y[3 * a + 2] += yv[a] * g.z;
        }
        gsum = gsum + g;
      }
    }
  };
  if (wide)
    pass1.template operator()<true>();
  else
    pass1.template operator()<false>();

  const Rigid<R> q = narrow_rigid<R>(qd);
  const Rigid<R> excl = lane_carry<R, W>(q, wave_total, lane, wave);

  // World frame at the lane start, origin at x2: R0 = F excl.m, X0 = F excl.v.
  R R0[9];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c)
      R0[3 * r + c] = Fm[3 * r] * excl.m[c] + Fm[3 * r + 1] * excl.m[3 + c] + Fm[3 * r + 2] * excl.m[6 + c];
  }
  const V3<R> X0 = rot_apply(Fm, V3<R>{excl.v[0], excl.v[1], excl.v[2]});

  // Lane moment sum_i (X0 + R0 y_i) x g_i = X0 x gsum + axial part of R0 Y.
  R Z[9];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c) Z[3 * r + c] = R0[3 * r] * Y[c] + R0[3 * r + 1] * Y[3 + c] + R0[3 * r + 2] * Y[6 + c];
  }
  ForceMoment<R> lane_sum;
  lane_sum.f = gsum;
  lane_sum.m = cross(X0, gsum) + V3<R>{Z[5] - Z[7], Z[6] - Z[2], Z[1] - Z[3]};

  // World state after the lane's last step.
  R Rm[9];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c) Rm[3 * r + c] = R0[3 * r] * q.m[c] + R0[3 * r + 1] * q.m[3 + c] + R0[3 * r + 2] * q.m[6 + c];
  }
  V3<R> x = X0 + rot_apply(R0, V3<R>{q.v[0], q.v[1], q.v[2]});

  const ForceMoment<R> tail = lane_suffix<R, W>(lane_sum, wave_sum, lane, wave);

  // Pass 2: walk the lane's steps backwards; the outputs of step s replace g_{s+3} in LDS.
  V3<R> Fs = tail.f, Ms = tail.m;
  if constexpr (Segmented) {
    Fs = Fs + V3<R>{static_cast<R>(carry[0]), static_cast<R>(carry[1]), static_cast<R>(carry[2])};
    Ms = Ms + V3<R>{static_cast<R>(carry[3]), static_cast<R>(carry[4]), static_cast<R>(carry[5])};
  }
  auto pass2 = [&]<bool Checked>() {
#pragma unroll
    for (int i = K - 1; i >= 0; --i) {
      if (s0 + i < steps) {
        const V3<R> g = load3(&gstage[o0 + 3 * i]);
        Fs = Fs + g;
        Ms = Ms + cross(x, g);
        const R l = pstage[b0 + i];
        const V3<R> col0 = {Rm[0], Rm[3], Rm[6]};
        const V3<R> col2 = {Rm[2], Rm[5], Rm[8]};
        const V3<R> xp = x - l * col0;
        const V3<R> tau = Ms - cross(xp, Fs);
        const R gl = dot(col0, Fs);
        const R ga = -dot(col2, tau);
        double s, c, S, C;
        sin_cos_wide<Checked>(pstage[Lay::kStepRow + b0 + i], s, c);
        sin_cos_wide<Checked>(pstage[2 * Lay::kStepRow + b0 + i], S, C);
        step_backward(Rm, static_cast<R>(s), static_cast<R>(c), static_cast<R>(S), static_cast<R>(C));
        const R gd = dot(V3<R>{Rm[0], Rm[3], Rm[6]}, tau);
        gstage[o0 + 3 * i] = gl;
        gstage[o0 + 3 * i + 1] = ga;
        gstage[o0 + 3 * i + 2] = gd;
        x = xp;
      }
    }
  };
  if (wide)
    pass2.template operator()<true>();
  else
    pass2.template operator()<false>();
  if (tid == 0 && (!Segmented || head)) {
    // First-frame parameters (block.cu:206-228); x2 is the origin, so M_2 = M_3.
    const V3<R> g1 = load3(&gstage[3]);
    const V3<R> g2 = load3(&gstage[6]);
    const V3<R> F2 = Fs + g2;
    const V3<R> x1 = ff.p1 - ff.p2;
    const V3<R> tau2 = Ms - cross(x1, F2);
    if (anchor != nullptr) store_anchor_sums(anchor, Fs, Ms, ff.p0 - ff.p2, x1, load3(&gstage[0]), g1, g2);
    gLr[0] = narrow<T>(dot(ff.d0, F2 + g1));
    gLr[1] = narrow<T>(dot(ff.d1, F2));
    gAr[0] = narrow<T>(-dot(cross(ff.d0, ff.t0), tau2));
  }
  __syncthreads();
  store_interleaved_rows<Lay>(gLr + 2, gAr + 1, gDr, gstage, steps, tid);
}

// ============================================================================ position-based backward

// Position-based adjoint for one chain the forward marked regular:
//   T_j = M_j - x_{j-1} x F_j,  dL/dL[j-1] = u(b_{j-1}).F_j,
//   dL/dA[j-2] = u(b_{j-1} x b_{j-2}).T_j,  dL/dD[j-3] = u(b_{j-2}).T_j,  b_i = x_{i+1} - x_i,
// where F_j, M_j are suffix sums of g and x x g and u(v) = v/|v|.  Positions are taken
// relative to x2.  Lane t owns points [3+tK, 3+tK+K) and writes the outputs of steps
// [tK, tK+K).  Rows are staged through LDS (xs, gs: one point row each); each lane copies its
// points [tK, tK+K+3) and gradients into registers, and its outputs replace its gradients in
// LDS for a coalesced store.
// The adjoint above once positions (xs) and gradients (gs) sit in LDS point rows, visible to
// the whole workgroup.
//
// Segmented: the rows are a segment of a longer chain (as in exact_chain).  carry[0..5] holds
// F and M (about the segment's x2, world axes) of every point after the segment.  The head
// segment holds world positions.  A later segment holds positions local to its x2, whose
// world rotation is frame[0..8] (row-major): there x2 is the origin, x1 = (-bond1, 0, 0) for
// the bond x1-x2 (the running frame's first axis is the bond into its origin), and the
// gradients and the carry are turned to the local axes; only the head writes the
// first-frame terms.
//
// Res (the fused losses' backward): gs holds a target row and the gradient of point x with
// target t is res(x, t) (SquaredResidual, SuperposedResidual), formed as the lane loads its
// points; NoResidual: gs holds the gradient row itself.
template <typename T, typename Lay, bool Segmented = false, typename Res = NoResidual>
__device__ __forceinline__ void position_adjoint(T* __restrict__ gLr, T* __restrict__ gAr, T* __restrict__ gDr,
                                                 compute_t<T>* xs, compute_t<T>* gs,
                                                 compute_t<T> (&wave_sum)[Lay::kWaves][6], int points,
                                                 double* __restrict__ anchor = nullptr, bool head = true,
                                                 const double* __restrict__ frame = nullptr,
                                                 const double* __restrict__ carry = nullptr,
                                                 compute_t<T> bond1 = 0, const Res& res = Res{}) {
  using R = compute_t<T>;
  constexpr bool Residual = !std::is_same_v<Res, NoResidual>;
  constexpr int W = Lay::kWaves;
  constexpr int K = Lay::kItems;
  const int steps = points - 3;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int s0 = tid * K;
  const int count = steps - s0 < K ? steps - s0 : K;  // points of this lane (may be <= 0)
  const int last = count - 1;

  // xr holds points s0 .. s0+K+2 (point s0+j at 3j), gr the gradients of points 3+s0 ...
  R xr[3 * K + 9], gr[3 * K];
  V3<R> c;
  {
    c = load3(&xs[6]);
    const int o0 = Lay::lane_point_base(tid);
#pragma unroll
    for (int i = 0; i < 3 * K; ++i) gr[i] = gs[o0 + i];
    // Points s0 .. s0+2 precede the lane's own run (they belong to the previous lane or are
    // points 0..2); points s0+3 .. sit in the lane's own slots.
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const V3<R> x = load3(&xs[Lay::point_slot(3 * (s0 + j))]);
      xr[3 * j] = x.x;
      xr[3 * j + 1] = x.y;
      xr[3 * j + 2] = x.z;
    }
#pragma unroll
    for (int i = 0; i < 3 * K; ++i) xr[9 + i] = xs[o0 + i];
    if constexpr (Residual) {
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const V3<R> g = res(V3<R>{xr[9 + 3 * i], xr[10 + 3 * i], xr[11 + 3 * i]},
                            V3<R>{gr[3 * i], gr[3 * i + 1], gr[3 * i + 2]});
        gr[3 * i] = g.x;
        gr[3 * i + 1] = g.y;
        gr[3 * i + 2] = g.z;
      }
    }
  }
  double q[9];  // Segmented, after the head: the world rotation at x2
  if constexpr (Segmented) {
    if (!head) {
#pragma unroll
      for (int i = 0; i < 9; ++i) q[i] = frame[i];
      c = {R(0), R(0), R(0)};
      if (tid == 0) {  // points 0..2 of the row belong to the previous segment
#pragma unroll
        for (int i = 0; i < 9; ++i) xr[i] = R(0);
        xr[3] = -bond1;
      }
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const R g0 = gr[3 * i], g1 = gr[3 * i + 1], g2 = gr[3 * i + 2];
#pragma unroll
        for (int k = 0; k < 3; ++k)
          gr[3 * i + k] = static_cast<R>(q[k]) * g0 + static_cast<R>(q[3 + k]) * g1 + static_cast<R>(q[6 + k]) * g2;
      }
    }
  }
  auto pos = [&](int j) { return V3<R>{xr[3 * j], xr[3 * j + 1], xr[3 * j + 2]} - c; };

  ForceMoment<R> lane_sum = {{R(0), R(0), R(0)}, {R(0), R(0), R(0)}};
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (i <= last) {
      const V3<R> g = {gr[3 * i], gr[3 * i + 1], gr[3 * i + 2]};
      lane_sum.f = lane_sum.f + g;
      lane_sum.m = lane_sum.m + cross(pos(i + 3), g);
    }
  }
  const ForceMoment<R> tail = lane_suffix<R, W>(lane_sum, wave_sum, lane, wave);

  // Reverse walk: item i is point p = 3+s0+i (xr index i+3) with neighbours i+2, i+1.
  V3<R> F = tail.f, M = tail.m;
  if constexpr (Segmented) {
    V3<double> cf = {carry[0], carry[1], carry[2]}, cm = {carry[3], carry[4], carry[5]};
    if (!head) {
      cf = {q[0] * cf.x + q[3] * cf.y + q[6] * cf.z, q[1] * cf.x + q[4] * cf.y + q[7] * cf.z,
            q[2] * cf.x + q[5] * cf.y + q[8] * cf.z};
      cm = {q[0] * cm.x + q[3] * cm.y + q[6] * cm.z, q[1] * cm.x + q[4] * cm.y + q[7] * cm.z,
            q[2] * cm.x + q[5] * cm.y + q[8] * cm.z};
    }
    F = F + V3<R>{static_cast<R>(cf.x), static_cast<R>(cf.y), static_cast<R>(cf.z)};
    M = M + V3<R>{static_cast<R>(cm.x), static_cast<R>(cm.y), static_cast<R>(cm.z)};
  }
  R oL[K], oA[K], oD[K];
#pragma unroll
  for (int i = K - 1; i >= 0; --i) {
    if (i <= last) {
      const V3<R> xa = pos(i + 3), xb = pos(i + 2), xc = pos(i + 1);
      const V3<R> g = {gr[3 * i], gr[3 * i + 1], gr[3 * i + 2]};
      F = F + g;
      M = M + cross(xa, g);
      const V3<R> Tq = M - cross(xb, F);
      const V3<R> b1 = xa - xb;
      const V3<R> b2 = xb - xc;
      const V3<R> n = cross(b1, b2);
      oL[i] = dot(b1, F) * rsqrt_bond(dot(b1, b1));
      oA[i] = dot(n, Tq) * rsqrt_bond(dot(n, n));
      oD[i] = dot(b2, Tq) * rsqrt_bond(dot(b2, b2));
    }
  }
  if (tid == 0 && (!Segmented || head)) {
    // Atoms 2 and 1: dL/dL[1], dL/dA[0] and dL/dL[0]; x2 is the origin, so M_2 = M_3.
    const V3<R> x0 = pos(0), x1 = pos(1), x2 = pos(2);
    auto grad = [&](int j) {
      const V3<R> g = load3(&gs[3 * j]);
      if constexpr (Residual) return res(load3(&xs[3 * j]), g);
      return g;
    };
    const V3<R> g1 = grad(1);
    const V3<R> g2 = grad(2);
    if (anchor != nullptr) store_anchor_sums(anchor, F, M, x0, x1, grad(0), g1, g2);
    F = F + g2;
    const V3<R> Tq = M - cross(x1, F);
    const V3<R> b1 = x2 - x1;
    const V3<R> b0 = x1 - x0;
    const V3<R> n = cross(b1, b0);
    gLr[1] = narrow<T>(dot(b1, F) * rsqrt_bond(dot(b1, b1)));
    gAr[0] = narrow<T>(dot(n, Tq) * rsqrt_bond(dot(n, n)));
    gLr[0] = narrow<T>(dot(b0, F + g1) * rsqrt_bond(dot(b0, b0)));
  }
  {
    const int o0 = Lay::lane_point_base(tid);
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (i <= last) {
        gs[o0 + 3 * i] = oL[i];
        gs[o0 + 3 * i + 1] = oA[i];
        gs[o0 + 3 * i + 2] = oD[i];
      }
    }
    __syncthreads();
    store_interleaved_rows<Lay>(gLr + 2, gAr + 1, gDr, gs, steps, tid);
  }
}

// Positions Xr of element type P: the chain's own output (P = T), or the float copy a
// float16/bfloat16 forward kept (P = float).
template <typename T, typename Lay, typename P = T>
__device__ __forceinline__ void position_chain(const P* __restrict__ Xr, const T* __restrict__ Gr,
                                               T* __restrict__ gLr, T* __restrict__ gAr, T* __restrict__ gDr,
                                               compute_t<T>* xs, compute_t<T>* gs,
                                               compute_t<T> (&wave_sum)[Lay::kWaves][6], int points,
                                               double* __restrict__ anchor = nullptr) {
  static_assert(std::is_same_v<compute_t<P>, compute_t<T>>, "positions in the compute type");
  if constexpr (std::is_same_v<P, T>) {
    compute_t<T>* const dst[2] = {xs, gs};
    const T* const src[2] = {Xr, Gr};
    load_point_rows<Lay, 2>(dst, src, points, threadIdx.x);
  } else {
    load_point_rows_pair<Lay>(xs, Xr, gs, Gr, points, threadIdx.x);
  }
  __syncthreads();
  position_adjoint<T, Lay>(gLr, gAr, gDr, xs, gs, wave_sum, points, anchor);
}

// ============================================================================ recompute backward

// Backward without a saved output: the forward scan is rerun in registers (double lane-serial,
// float cross-lane), giving every lane its points relative to x2 in the compute precision;
// chains that pass the regularity test on those positions (FastPath<compute type>) take the
// position-based adjoint over them, the others exact_chain.  For float16/bfloat16 chains this
// replaces the exact recompute, whose reverse walk costs about twice the forward, and it needs
// no float copy of the half-precision output.  pstage: 3 step rows (then the positions),
// gstage: the gradient row.
template <typename T, typename Lay>
__device__ __forceinline__ void recompute_chain(const T* __restrict__ Lr, const T* __restrict__ Ar,
                                                const T* __restrict__ Dr, const T* __restrict__ p0,
                                                const T* __restrict__ first_direction,
                                                const T* __restrict__ initial_normal, const T* __restrict__ Gr,
                                                T* __restrict__ gLr, T* __restrict__ gAr, T* __restrict__ gDr,
                                                compute_t<T>* pstage, compute_t<T>* gstage,
                                                compute_t<T> (&wave_total)[Lay::kWaves][12],
                                                compute_t<T> (&wave_sum)[Lay::kWaves][6],
                                                compute_t<T> (&wave_stat)[Lay::kWaves][3], int (&wide_vote)[Lay::kWaves],
                                                int points, double* __restrict__ anchor = nullptr) {
  using R = compute_t<T>;
  using Fast = FastPath<R>;
  constexpr int W = Lay::kWaves;
  constexpr int K = Lay::kItems;
  const int steps = points - 3;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int s0 = tid * K;
  const int count = steps - s0 < K ? steps - s0 : K;
  const int b0 = Lay::lane_step_base(tid);
  bool wide;
  {
    R* const dst[3] = {pstage, pstage + Lay::kStepRow, pstage + 2 * Lay::kStepRow};
    const T* const src[3] = {Lr + 2, Ar + 1, Dr};
    wide = load_step_rows<Lay, 3, 0b110u>(dst, src, steps, tid);
    R* const gdst[1] = {gstage};
    const T* const gsrc[1] = {Gr};
    load_point_rows<Lay, 1>(gdst, gsrc, points, tid);
  }
  // sin/cos without the LDS table: measured at C4 (bf16, 2 waves x 8 steps, 10 waves per CU)
  // the table's bank conflicts cost more than its arithmetic saves (237 against 210 us).
  pad_lane_tail<K>(pstage + b0, pstage + Lay::kStepRow + b0, pstage + 2 * Lay::kStepRow + b0, count);
  const FirstFrame<R> ff = first_frame<T>(widen(Lr[0]), widen(Lr[1]), widen(Ar[0]), p0, first_direction, initial_normal);
  wide = block_any<W>(wide, wide_vote, lane, wave);

  Rigid<double> q;  // set by each lane's first step (lane_scan_chain)
  R y[K][3];
  bool ok = true;
  R lmin = R(1.0e30);
  lane_scan_chain<T, K, false, Fast>(pstage + b0, pstage + Lay::kStepRow + b0, pstage + 2 * Lay::kStepRow + b0,
                                           count, wide, nullptr, q, y, ok, lmin);
  const Rigid<R> excl = lane_carry<R, W>(narrow_rigid<R>(q), wave_total, lane, wave);

  // World frame at the lane start, origin at x2.
  R R0[9];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c)
      R0[3 * r + c] = ff.frame[3 * r] * excl.m[c] + ff.frame[3 * r + 1] * excl.m[3 + c] + ff.frame[3 * r + 2] * excl.m[6 + c];
  }
  const V3<R> X0 = rot_apply(ff.frame, V3<R>{excl.v[0], excl.v[1], excl.v[2]});
  V3<R> x[K];
  R xmax = R(0);
#pragma unroll
  for (int i = 0; i < K; ++i) {
    x[i] = X0 + rot_apply(R0, V3<R>{y[i][0], y[i][1], y[i][2]});
    if (i < count) xmax = abs_max3(xmax, x[i]);
  }
  {
    const bool wave_ok = __all(ok);
    const R wmin = wave_min_positive(lmin);
    const R wmax = wave_max_nonneg(xmax);
    if (lane == 0) {
      wave_stat[wave][0] = wave_ok ? R(1) : R(0);
      wave_stat[wave][1] = wmin;
      wave_stat[wave][2] = wmax;
    }
  }
  __syncthreads();  // also retires every read of the step rows, which the positions replace
  bool regular = ff.L0 > R(0) && ff.L1 > R(0) && ff.sinA0 >= static_cast<R>(Fast::kSinMin);
  {
    R m = fmin(ff.L0, ff.L1);
    R xm = abs_max3(abs_max3(R(0), ff.p0 - ff.p2), ff.p1 - ff.p2);
#pragma unroll
    for (int w = 0; w < W; ++w) {
      regular = regular && wave_stat[w][0] != R(0);
      m = fmin(m, wave_stat[w][1]);
      xm = fmax(xm, wave_stat[w][2]);
    }
    regular = regular && fast_extent_ok<Fast>(xm, m);
  }
  if (regular) {
    const int o0 = Lay::lane_point_base(tid);
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (i < count) {
        pstage[o0 + 3 * i] = x[i].x;
        pstage[o0 + 3 * i + 1] = x[i].y;
        pstage[o0 + 3 * i + 2] = x[i].z;
      }
    }
    if (tid == 0) {
      const V3<R> a = ff.p0 - ff.p2, b = ff.p1 - ff.p2;
      pstage[0] = a.x; pstage[1] = a.y; pstage[2] = a.z;
      pstage[3] = b.x; pstage[4] = b.y; pstage[5] = b.z;
      pstage[6] = R(0); pstage[7] = R(0); pstage[8] = R(0);
    }
    __syncthreads();
    position_adjoint<T, Lay>(gLr, gAr, gDr, pstage, gstage, wave_sum, points, anchor);
  } else {
    exact_chain<T, Lay>(Lr, Ar, Dr, p0, first_direction, initial_normal, Gr, gLr, gAr, gDr, pstage, gstage, wave_total,
                        wave_sum, wide_vote, points, true, nullptr, nullptr, anchor);
  }
}

// ============================================================================ refused chains first

// A chain the position-based adjoint refuses (regular flag 0) runs the exact path, which takes
// about twice as long as a position-based chain.  Spread through the grid, the ones dispatched
// last would set the kernel's end (at C2's shape, one refused chain in 64 took the backward from
// 58 to 81 us, one in 16 to 97 us).  So the grids of the backwards that choose per chain start
// with kFrontRanks front workgroups per group of kFrontGroup consecutive chains: front workgroup
// r of a group takes the group's r-th refused chain, if any, and further on that chain's own
// workgroup does nothing.  Up to kFrontRanks refused chains in every kFrontGroup thus start at
// the head of the grid, and every chain is still processed by exactly one workgroup.
//
// Workgroups go to the eight XCDs round-robin by index, so two orders keep the exact work spread
// over them: the front region is rank-major (every group's rank-0 workgroup, then rank 1, ...),
// so the busy ones form a prefix whatever the number of refused chains per group; and group g
// counts its chains from position 4g mod 16 (cyclically), so the chains whose own workgroups
// skip do not always sit at the same positions, i.e. on the same XCDs.
//
// Measured at C2's shape (step, one box, interleaved): every chain regular 94.8-95.2 us for one,
// two or four ranks alike; one refused chain in 4: 138.5, 112.6, 114.9 us for 1, 2, 4 ranks
// (146 us before); one in 8: 106.6, 105.1, 106.2 us; every chain refused: 143.7, 148.1, 155.0 us
// (148 us before), the skipping workgroups briefly holding LDS that exact ones could use.
constexpr int kFrontGroup = 16;
constexpr int kFrontRanks = 2;

__host__ __device__ constexpr int64_t chain_groups(int64_t batch) { return (batch + kFrontGroup - 1) / kFrontGroup; }
__host__ __device__ constexpr int64_t front_groups(int64_t batch) { return chain_groups(batch) * kFrontRanks; }

// Group g's refused chains as a kFrontGroup-bit mask in its counting order: bit q for the chain
// at position (q + 4g) mod kFrontGroup (chains at or past batch never refused).  Each wave loads
// the group's flags itself, so the mask is uniform over the workgroup without LDS.
__device__ __forceinline__ unsigned refused_mask(const uint8_t* __restrict__ regular, int64_t g, int64_t batch) {
  const int lane = threadIdx.x & 63;
  const int64_t chain = g * kFrontGroup + ((lane + 4 * g) & (kFrontGroup - 1));
  return static_cast<unsigned>(__ballot(lane < kFrontGroup && chain < batch && regular[chain] == 0));
}

// The chain this backward workgroup takes (the grid is front_groups(batch) + batch
// workgroups), or -1 for none.
__device__ __forceinline__ int64_t backward_row(const uint8_t* __restrict__ regular, int64_t batch) {
  const int64_t groups = chain_groups(batch);
  const int64_t wg = blockIdx.x;
  if (wg < groups * kFrontRanks) {
    const int64_t g = wg % groups;
    unsigned mask = refused_mask(regular, g, batch);
    for (int r = static_cast<int>(wg / groups); r > 0 && mask != 0; --r) mask &= mask - 1;  // drop r lowest
    return mask == 0 ? -1 : g * kFrontGroup + ((__builtin_ctz(mask) + 4 * g) & (kFrontGroup - 1));
  }
  const int64_t row = wg - groups * kFrontRanks;
  if (regular[row] != 0) return row;
  const int64_t g = row / kFrontGroup;
  const int q = static_cast<int>((row - g * kFrontGroup - 4 * g) & (kFrontGroup - 1));  // counting position
  return __builtin_popcount(refused_mask(regular, g, batch) & ((1u << q) - 1)) < kFrontRanks ? -1 : row;
}


// Backward without a saved output, one workgroup per chain.
template <typename T, int W, int K, int Pad>
__global__ __launch_bounds__(64 * W) void reconstruct_backward_recompute_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    const T* __restrict__ grad_xyz, T* __restrict__ grad_lengths, T* __restrict__ grad_angles,
    T* __restrict__ grad_dihedrals, int points, double* __restrict__ anchor = nullptr) {
  using R = compute_t<T>;
  using Lay = Layout<W, K, Pad>;
  constexpr int kA = 3 * Lay::kStepRow > Lay::kPointRow ? 3 * Lay::kStepRow : Lay::kPointRow;
  __shared__ __align__(16) R region_a[kA];
  __shared__ __align__(16) R region_b[Lay::kPointRow];
  __shared__ R wave_total[W][12];
  __shared__ R wave_sum[W][6];
  __shared__ R wave_stat[W][3];
  __shared__ int wide_vote[W];
  const int64_t row = blockIdx.x;
  recompute_chain<T, Lay>(lengths + row * (points - 1), angles + row * (points - 2), dihedrals + row * (points - 3), p0,
                          first_direction, initial_normal, grad_xyz + row * points * 3, grad_lengths + row * (points - 1),
                          grad_angles + row * (points - 2), grad_dihedrals + row * (points - 3), region_a, region_b,
                          wave_total, wave_sum, wave_stat, wide_vote, points,
                          anchor != nullptr ? anchor + row * 6 : nullptr);
}

// Backward given the forward's own output: one workgroup per chain, the position-based
// adjoint for chains with regular[row] != 0 and the exact recompute for the others, in one
// launch.  The two paths share the LDS: region A holds xs or the parameter rows, region B
// the gradient row.  P = float reads the float positions a float16/bfloat16 forward kept
// (reconstruct_forward_shadow_kernel) in place of its output.
template <typename T, int W, int K, int Pad, typename P = T>
__global__ __launch_bounds__(64 * W) void reconstruct_backward_saved_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    const P* __restrict__ xyz, const uint8_t* __restrict__ regular, const T* __restrict__ grad_xyz,
    T* __restrict__ grad_lengths, T* __restrict__ grad_angles, T* __restrict__ grad_dihedrals, int points,
    int64_t batch, double* __restrict__ anchor = nullptr) {
  using R = compute_t<T>;
  using Lay = Layout<W, K, Pad>;
  constexpr int kA = 3 * Lay::kStepRow > Lay::kPointRow ? 3 * Lay::kStepRow : Lay::kPointRow;
  __shared__ __align__(16) R region_a[kA];
  __shared__ __align__(16) R region_b[Lay::kPointRow];
  __shared__ R wave_total[W][12];
  __shared__ R wave_sum[W][6];
  __shared__ int wide_vote[W];
  const int64_t row = backward_row(regular, batch);  // uniform over the workgroup
  if (row < 0) return;
  double* const an = anchor != nullptr ? anchor + row * 6 : nullptr;
  T* gLr = grad_lengths + row * (points - 1);
  T* gAr = grad_angles + row * (points - 2);
  T* gDr = grad_dihedrals + row * (points - 3);
  if (regular[row] != 0) {
    position_chain<T, Lay, P>(xyz + row * points * 3, grad_xyz + row * points * 3, gLr, gAr, gDr, region_a, region_b,
                              wave_sum, points, an);
  } else {
    exact_chain<T, Lay>(lengths + row * (points - 1), angles + row * (points - 2), dihedrals + row * (points - 3), p0,
                        first_direction, initial_normal, grad_xyz + row * points * 3, gLr, gAr, gDr, region_a,
                        region_b, wave_total, wave_sum, wide_vote, points, true, nullptr, nullptr, an);
  }
}

// ============================================================================ anchor gradients

// One workgroup: the per-chain sums (F, tau) of `part` reduced over the batch in double, then
// mapped to the anchors (no reference counterpart; the map follows from every point being
// p0 + Q c_i with Q = [d, t, n] the orthonormal first frame):
//   dL/dp0 = F;  dL = dd . (tau x d) - (tau . d)(dn . t) for a rotation moving d by dd and n by
//   dn, then the chain rule through the normalisation of first_direction and the Gram-Schmidt
//   step (or the fixed-helper normal stable_perpendicular(d) when that step degenerates).
constexpr int kAnchorThreads = 256;
template <typename T>
__global__ __launch_bounds__(kAnchorThreads) void anchor_gradients_kernel(
    const double* __restrict__ part, int64_t batch, const T* __restrict__ first_direction,
    const T* __restrict__ initial_normal, T* __restrict__ grad_p0, T* __restrict__ grad_first_direction,
    T* __restrict__ grad_initial_normal) {
  __shared__ double red[kAnchorThreads / 64][6];
  double acc[6] = {0, 0, 0, 0, 0, 0};
  for (int64_t b = threadIdx.x; b < batch; b += kAnchorThreads) {
#pragma unroll
    for (int k = 0; k < 6; ++k) acc[k] += part[b * 6 + k];
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const double v = wave_sum(acc[k]);
    if (lane == 0) red[wave][k] = v;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  double sum[6] = {0, 0, 0, 0, 0, 0};
  for (int w = 0; w < kAnchorThreads / 64; ++w)
    for (int k = 0; k < 6; ++k) sum[k] += red[w][k];
  const V3<double> F = {sum[0], sum[1], sum[2]};
  const V3<double> tau = {sum[3], sum[4], sum[5]};
  using R = compute_t<T>;
  // The branch is decided as first_frame decides it, in the compute precision.
  bool degenerate;
  {
    const V3<R> dr = normalized(V3<R>{widen(first_direction[0]), widen(first_direction[1]), widen(first_direction[2])});
    const V3<R> nr0 = {widen(initial_normal[0]), widen(initial_normal[1]), widen(initial_normal[2])};
    const V3<R> nn = nr0 - dot(nr0, dr) * dr;
    degenerate = dot(nn, nn) < static_cast<R>(1.0e-12f);
  }
  const V3<double> f0 = {widen(first_direction[0]), widen(first_direction[1]), widen(first_direction[2])};
  const V3<double> n0 = {widen(initial_normal[0]), widen(initial_normal[1]), widen(initial_normal[2])};
  const double dn = sqrt(fmax(dot(f0, f0), static_cast<double>(1.0e-12f)));
  const V3<double> d = {f0.x / dn, f0.y / dn, f0.z / dn};
  const V3<double> nr = n0 - dot(n0, d) * d;
  V3<double> gfd, gn0;
  if (degenerate) {  // n = stable_perpendicular(d)
    const V3<double> h = fabs(d.x) >= 0.9 ? V3<double>{0, 1, 0} : V3<double>{1, 0, 0};
    const V3<double> dh = cross(d, h);
    const double dhn = sqrt(dot(dh, dh));
    const V3<double> n = {dh.x / dhn, dh.y / dhn, dh.z / dhn};
    const V3<double> t = cross(n, d);
    const V3<double> v = cross(tau, d) - (dot(tau, d) / dhn) * cross(h, t);
    const V3<double> vp = v - dot(v, d) * d;
    gfd = {vp.x / dn, vp.y / dn, vp.z / dn};
    gn0 = {0, 0, 0};
  } else {
    const double nn = sqrt(dot(nr, nr));
    const V3<double> n = {nr.x / nn, nr.y / nn, nr.z / nn};
    const V3<double> t = cross(n, d);
    const V3<double> v = cross(tau, d) + (dot(tau, d) * dot(n0, d) / nn) * t;
    gfd = {v.x / dn, v.y / dn, v.z / dn};
    gn0 = (-dot(tau, d) / nn) * t;
  }
  const double out[9] = {F.x, F.y, F.z, gfd.x, gfd.y, gfd.z, gn0.x, gn0.y, gn0.z};
  T* const dst[3] = {grad_p0, grad_first_direction, grad_initial_normal};
  for (int k = 0; k < 9; ++k) dst[k / 3][k % 3] = narrow<T>(static_cast<R>(out[k]));
}

// ============================================================================ fused coordinate loss

// Forward of sum_i |x_i - target_i|^2 per chain: the flagged forward (positions and the
// regularity flag written as reconstruct_forward_kernel writes them) with the loss reduced in
// the workgroup from the positions in registers.
template <typename T, int W, int K, int Pad>
__global__ __launch_bounds__(64 * W) void reconstruct_loss_forward_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    const T* __restrict__ target, T* __restrict__ xyz, uint8_t* __restrict__ regular, T* __restrict__ loss,
    int points) {
  const int64_t row = blockIdx.x;
  forward_chain<T, Layout<W, K, Pad>, false, kLossSquared>(lengths + row * (points - 1), angles + row * (points - 2),
                                                   dihedrals + row * (points - 3), p0, first_direction, initial_normal,
                                                   xyz + row * points * 3, regular + row, points, true, nullptr,
                                                   target + row * points * 3, loss + row);
}

// Forward of the superposed losses: the flagged forward, plus the sums of the optimal
// superposition onto the target in each chain's record (superpose_records_kernel follows).
template <typename T, int W, int K, int Pad>
__global__ __launch_bounds__(64 * W) void reconstruct_superposed_forward_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    const T* __restrict__ target, T* __restrict__ xyz, uint8_t* __restrict__ regular, double* __restrict__ record,
    int points) {
  const int64_t row = blockIdx.x;
  forward_chain<T, Layout<W, K, Pad>, false, kLossSuperposed>(
      lengths + row * (points - 1), angles + row * (points - 2), dihedrals + row * (points - 3), p0, first_direction,
      initial_normal, xyz + row * points * 3, regular + row, points, true, nullptr, target + row * points * 3, nullptr,
      nullptr, record + row * kSuperposeRecord);
}

// The backward of the fused losses over the saved positions: the gradient row is formed from
// the staged positions and target (grad_xyz never exists in HBM), in registers as the
// position-based adjoint loads them for regular chains, in LDS before the exact adjoint for the
// others.  kLossSquared: 2 w_b (x - target).  kLossSuperposed: c (x - M t - a) from the
// chain's superposition record (superpose.h), c = (2/N) w_b, divided by 2 rmsd unless
// `squared` (0 where rmsd = 0).  With `anchor`, each chain also writes its six anchor sums
// (store_anchor_sums) for anchor_gradients_kernel.
template <typename T, int W, int K, int Pad, int LossKind = kLossSquared>
__global__ __launch_bounds__(64 * W) void reconstruct_loss_backward_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    const T* __restrict__ xyz, const uint8_t* __restrict__ regular, const T* __restrict__ target,
    const T* __restrict__ grad_loss, T* __restrict__ grad_lengths, T* __restrict__ grad_angles,
    T* __restrict__ grad_dihedrals, int points, int64_t batch, const double* __restrict__ record = nullptr,
    int squared = 0, double* __restrict__ anchor = nullptr) {
  using R = compute_t<T>;
  using Lay = Layout<W, K, Pad>;
  using Res = std::conditional_t<LossKind == kLossSuperposed, SuperposedResidual<R>, SquaredResidual<R>>;
  constexpr int kA = 3 * Lay::kStepRow > Lay::kPointRow ? 3 * Lay::kStepRow : Lay::kPointRow;
  __shared__ __align__(16) R region_a[kA];
  __shared__ __align__(16) R region_b[Lay::kPointRow];
  __shared__ R wave_total[W][12];
  __shared__ R wave_sum[W][6];
  __shared__ int wide_vote[W];
  // Refused chains first (backward_row) where the position path exists; every half-type chain
  // takes the exact path, in grid order.
  const int64_t row = FastPath<T>::kEnabled ? backward_row(regular, batch) : static_cast<int64_t>(blockIdx.x);
  if (row < 0) return;
  const int tid = threadIdx.x;
  {
    R* const dst[2] = {region_a, region_b};
    const T* const src[2] = {xyz + row * points * 3, target + row * points * 3};
    load_point_rows<Lay, 2>(dst, src, points, tid);
  }
  const R w = grad_loss != nullptr ? widen(grad_loss[row]) : R(1);
  const Res res = make_residual<LossKind>(w, record != nullptr ? record + row * kSuperposeRecord : nullptr, points,
                                          squared);
  __syncthreads();
  T* gLr = grad_lengths + row * (points - 1);
  T* gAr = grad_angles + row * (points - 2);
  T* gDr = grad_dihedrals + row * (points - 3);
  double* const an = anchor != nullptr ? anchor + row * 6 : nullptr;
  if (FastPath<T>::kEnabled && regular[row] != 0) {
    position_adjoint<T, Lay, false, Res>(gLr, gAr, gDr, region_a, region_b, wave_sum, points, an, true, nullptr, nullptr,
                                         R(0), res);
  } else {
    for (int p = tid; p < points; p += Lay::kLanes) {
      const int slot = Lay::point_slot(3 * p);  // a point's three coordinates share a lane segment
      const V3<R> g = res(load3(&region_a[slot]), load3(&region_b[slot]));
      region_b[slot] = g.x;
      region_b[slot + 1] = g.y;
      region_b[slot + 2] = g.z;
    }
    __syncthreads();
    exact_chain<T, Lay, false, false>(lengths + row * (points - 1), angles + row * (points - 2),
                                      dihedrals + row * (points - 3), p0, first_direction, initial_normal, nullptr, gLr,
                                      gAr, gDr, region_a, region_b, wave_total, wave_sum, wide_vote, points, true,
                                      nullptr, nullptr, an);
  }
}

}  // namespace cufk_amd
