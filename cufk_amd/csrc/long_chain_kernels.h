// Long chains: more local transforms than one workgroup scans (the reference stops at 2048,
// extension_utils.cuh:128-130; its README:58 leaves longer chains to a separate repository).
//
// The chain is cut into segments of S steps.  Each segment is scanned by one workgroup as a
// chain of its own (forward_chain / exact_chain in their segmented form) and the segments are
// joined by short per-chain passes in double.  No workgroup ever waits for another: every
// dependency between segments crosses a kernel boundary.
//
// Segment j of chain b covers steps [jS, jS + n_j), n_j = min(S, steps - jS), i.e. places
// points jS+3 .. jS+n_j+2; its "x2" is point jS+2, the last point before it.
//
// State, float64, per (chain, segment), written by the forward:
//   [0..11]  the segment's own total transform (row-major rotation, then translation)
//   [12..23] the world frame at the segment's x2: rotation (row-major), then x2 itself
// Work, float64, per (chain, segment), used by the backward:
//   [0..5]   F = sum g and M = sum (x - x2) x g over the segment's own points
//   [6..11]  the same sums over every point after the segment, about the segment's x2
//
// The state buffer then holds, after its records, one flag byte per (chain, segment) (the
// forward's regularity test on the segment's own positions) and the local positions of
// segments j >= 1 (a (points, 3) row of T per chain).
//
// Forward: segments (identity frame for j >= 1, local positions) -> frames -> place.
// Backward: sums (saved positions) -> carry -> segments (position-based adjoint over the local
// positions where the flags allow it, else the exact adjoint with frame and carry).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "chain_ops.h"
#include "launch.h"
#include "reconstruct_kernels.h"
#include "staging.h"

namespace cufk_amd {

constexpr int kLongThreads = 256;  // per-point and per-chain passes

struct SegmentOf {
  int64_t chain;
  int index;  // j
  int first;  // first step, jS
  int steps;  // n_j
};

// Workgroup g of a grid over (chain, segment j >= j0), chain-major.
__device__ __forceinline__ SegmentOf segment_of(int64_t g, int points, int seg_steps, int segments, int j0) {
  const int per = segments - j0;
  SegmentOf s;
  s.chain = g / per;
  s.index = j0 + static_cast<int>(g - s.chain * per);
  s.first = s.index * seg_steps;
  const int left = points - 3 - s.first;
  s.steps = left < seg_steps ? left : seg_steps;
  return s;
}

// ---------------------------------------------------------------------------- forward

template <typename T, int W, int K, int Pad>
__global__ __launch_bounds__(64 * W) void long_forward_segments_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    T* __restrict__ xyz, T* __restrict__ local, uint8_t* __restrict__ flags, double* __restrict__ state, int points,
    int seg_steps, int segments) {
  const SegmentOf s = segment_of(blockIdx.x, points, seg_steps, segments, 0);
  const int64_t b = s.chain;
  const int64_t at = b * segments + s.index;
  T* const out = (s.index == 0 ? xyz : local) + (b * points + s.first) * 3;
  forward_chain<T, Layout<W, K, Pad>, true>(
      lengths + b * (points - 1) + s.first, angles + b * (points - 2) + s.first, dihedrals + b * (points - 3) + s.first,
      p0, first_direction, initial_normal, out, flags + at, s.steps + 3, s.index == 0, state + at * kLongStateDoubles);
}

// One wave per chain: the world frame at every segment's x2, composed in double from x2 of
// the first frame (the one the head segment used) and the segment totals, the head's total
// already carrying the first frame's rotation (forward_chain composes it into the scan); the
// head's own frame is the first frame.  Lane l handles segment 64c + l of chunk c: an ordered
// wave scan of the totals, then the running frame of the earlier chunks in front.
template <typename T>
__global__ __launch_bounds__(kLongThreads) void long_forward_frames_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ p0,
    const T* __restrict__ first_direction, const T* __restrict__ initial_normal, double* __restrict__ state,
    int64_t batch, int points, int segments) {
  using R = compute_t<T>;
  const int lane = threadIdx.x & 63;
  const int64_t b = static_cast<int64_t>(blockIdx.x) * (kLongThreads / 64) + (threadIdx.x >> 6);
  if (b >= batch) return;  // uniform per wave
  const T* Lr = lengths + b * (points - 1);
  const T* Ar = angles + b * (points - 2);
  const FirstFrame<R> ff = first_frame<T>(widen(Lr[0]), widen(Lr[1]), widen(Ar[0]), p0, first_direction, initial_normal);
  Rigid<double> run = rigid_identity<double>();  // (I, x2) o the totals of earlier chunks
  run.v[0] = static_cast<double>(ff.p2.x);
  run.v[1] = static_cast<double>(ff.p2.y);
  run.v[2] = static_cast<double>(ff.p2.z);
  double* st = state + b * segments * kLongStateDoubles;
  for (int j0 = 0; j0 < segments; j0 += 64) {
    const int j = j0 + lane;
    Rigid<double> t = rigid_identity<double>();
    if (j < segments) {
      const double* tj = st + j * kLongStateDoubles;
#pragma unroll
      for (int i = 0; i < 9; ++i) t.m[i] = tj[i];
#pragma unroll
      for (int i = 0; i < 3; ++i) t.v[i] = tj[9 + i];
    }
    const Rigid<double> incl = wave_prefix(t);
    Rigid<double> f = compose(run, wave_shift_up(incl, lane));
    if (j == 0) {
#pragma unroll
      for (int i = 0; i < 9; ++i) f.m[i] = static_cast<double>(ff.frame[i]);
    }
    if (j < segments) {
      double* fj = st + j * kLongStateDoubles + 12;
#pragma unroll
      for (int i = 0; i < 9; ++i) fj[i] = f.m[i];
#pragma unroll
      for (int i = 0; i < 3; ++i) fj[9 + i] = f.v[i];
    }
    Rigid<double> chunk;
#pragma unroll
    for (int i = 0; i < 9; ++i) chunk.m[i] = lane_value(incl.m[i], 63);
#pragma unroll
    for (int i = 0; i < 3; ++i) chunk.v[i] = lane_value(incl.v[i], 63);
    run = compose(run, chunk);
  }
}

// Segments j >= 1: local positions y -> x2 + F y in world coordinates.
template <typename T>
__global__ __launch_bounds__(kLongThreads) void long_forward_place_kernel(T* __restrict__ xyz,
                                                                         const T* __restrict__ local,
                                                                         const double* __restrict__ state, int points,
                                                                         int seg_steps, int segments) {
  const SegmentOf s = segment_of(blockIdx.x, points, seg_steps, segments, 1);
  const double* f = state + (s.chain * segments + s.index) * kLongStateDoubles + 12;
  double m[9], o[3];
#pragma unroll
  for (int i = 0; i < 9; ++i) m[i] = f[i];
#pragma unroll
  for (int i = 0; i < 3; ++i) o[i] = f[9 + i];
  T* x = xyz + (s.chain * points + s.first + 3) * 3;
  const T* y = local + (s.chain * points + s.first + 3) * 3;
  for (int i = threadIdx.x; i < s.steps; i += kLongThreads) {
    const double y0 = static_cast<double>(widen(y[3 * i]));
    const double y1 = static_cast<double>(widen(y[3 * i + 1]));
    const double y2 = static_cast<double>(widen(y[3 * i + 2]));
#pragma unroll
    for (int r = 0; r < 3; ++r)
      x[3 * i + r] = narrow<T>(static_cast<compute_t<T>>(o[r] + m[3 * r] * y0 + m[3 * r + 1] * y1 + m[3 * r + 2] * y2));
  }
}

// ---------------------------------------------------------------------------- backward

// Segments j >= 1: F and M about the segment's x2 over its own points, from the saved
// positions, in double.
template <typename T>
__global__ __launch_bounds__(kLongThreads) void long_backward_sums_kernel(const T* __restrict__ xyz,
                                                                         const T* __restrict__ grad_xyz,
                                                                         const double* __restrict__ state,
                                                                         double* __restrict__ work, int points,
                                                                         int seg_steps, int segments) {
  __shared__ double part[kLongThreads / 64][6];
  const SegmentOf s = segment_of(blockIdx.x, points, seg_steps, segments, 1);
  const int64_t at = s.chain * segments + s.index;
  const double* o = state + at * kLongStateDoubles + 21;
  const double o0 = o[0], o1 = o[1], o2 = o[2];
  const int64_t base = (s.chain * points + s.first + 3) * 3;
  const T* x = xyz + base;
  const T* g = grad_xyz + base;
  double acc[6] = {0, 0, 0, 0, 0, 0};
  auto add = [&](double x0, double x1, double x2, double g0, double g1, double g2) {
    const double d0 = x0 - o0, d1 = x1 - o1, d2 = x2 - o2;
    acc[0] += g0;
    acc[1] += g1;
    acc[2] += g2;
    acc[3] += d1 * g2 - d2 * g1;
    acc[4] += d2 * g0 - d0 * g2;
    acc[5] += d0 * g1 - d1 * g0;
  };
  int first = 0;
  if constexpr (std::is_same_v<T, float>) {
    // Four points (12 floats, three dword-aligned 16-byte loads per row) per thread and pass.
    const int quads = s.steps >> 2;
    for (int q = threadIdx.x; q < quads; q += kLongThreads) {
      float xv[12], gv[12];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const f32x4 a = *reinterpret_cast<const f32x4u*>(x + 12 * q + 4 * k);
        const f32x4 b = *reinterpret_cast<const f32x4u*>(g + 12 * q + 4 * k);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xv[4 * k + e] = a[e];
          gv[4 * k + e] = b[e];
        }
      }
#pragma unroll
      for (int p = 0; p < 4; ++p)
        add(xv[3 * p], xv[3 * p + 1], xv[3 * p + 2], gv[3 * p], gv[3 * p + 1], gv[3 * p + 2]);
    }
    first = 4 * quads;
  }
  for (int i = first + static_cast<int>(threadIdx.x); i < s.steps; i += kLongThreads)
    add(static_cast<double>(widen(x[3 * i])), static_cast<double>(widen(x[3 * i + 1])),
        static_cast<double>(widen(x[3 * i + 2])), static_cast<double>(widen(g[3 * i])),
        static_cast<double>(widen(g[3 * i + 1])), static_cast<double>(widen(g[3 * i + 2])));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const double v = wave_sum(acc[k]);
    if (lane == 0) part[wave][k] = v;
  }
  __syncthreads();
  if (threadIdx.x < 6) {
    double v = 0;
#pragma unroll
    for (int w = 0; w < kLongThreads / 64; ++w) v += part[w][threadIdx.x];
    work[at * kLongWorkDoubles + threadIdx.x] = v;
  }
}

// One wave per chain: the suffix carry of every segment.  With moments taken about the
// world origin (W = M + x2 x F for a segment's own sums), the carry of segment j is
// F = sum_{l>j} F_l and M = sum_{l>j} W_l - x2_j x F: an exclusive suffix sum over segments,
// lane l holding segment 64c + l, chunks from the last.
static __global__ __launch_bounds__(kLongThreads) void long_backward_carry_kernel(const double* __restrict__ state,
                                                                                 double* __restrict__ work,
                                                                                 int64_t batch, int segments) {
  const int lane = threadIdx.x & 63;
  const int64_t b = static_cast<int64_t>(blockIdx.x) * (kLongThreads / 64) + (threadIdx.x >> 6);
  if (b >= batch) return;  // uniform per wave
  const double* st = state + b * segments * kLongStateDoubles;
  double* wk = work + b * segments * kLongWorkDoubles;
  ForceMoment<double> later = {{0, 0, 0}, {0, 0, 0}};  // every chunk after this one
  for (int c = (segments - 1) / 64; c >= 0; --c) {
    const int j = 64 * c + lane;
    ForceMoment<double> own = {{0, 0, 0}, {0, 0, 0}};
    V3<double> o = {0, 0, 0};
    if (j < segments) {
      const double* x2 = st + j * kLongStateDoubles + 21;
      o = {x2[0], x2[1], x2[2]};
      if (j >= 1) {  // the head's own sums are never needed
        const double* w = wk + j * kLongWorkDoubles;
        own.f = {w[0], w[1], w[2]};
        own.m = V3<double>{w[3], w[4], w[5]} + cross(o, own.f);
      }
    }
    const ForceMoment<double> incl = wave_suffix(own, lane);
    ForceMoment<double> after = wave_shift_down(incl, lane);  // lanes above this one
    after.f = after.f + later.f;                                  // then the later chunks
    after.m = after.m + later.m;
    if (j < segments) {
      double* w = wk + j * kLongWorkDoubles + 6;
      const V3<double> m = after.m - cross(o, after.f);
      w[0] = after.f.x; w[1] = after.f.y; w[2] = after.f.z;
      w[3] = m.x; w[4] = m.y; w[5] = m.z;
    }
    later.f = later.f + V3<double>{lane_value(incl.f.x, 0), lane_value(incl.f.y, 0), lane_value(incl.f.z, 0)};
    later.m = later.m + V3<double>{lane_value(incl.m.x, 0), lane_value(incl.m.y, 0), lane_value(incl.m.z, 0)};
  }
}

template <typename T, int W, int K, int Pad>
__global__ __launch_bounds__(64 * W) void long_backward_segments_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    const T* __restrict__ xyz, const T* __restrict__ local, const uint8_t* __restrict__ flags,
    const T* __restrict__ grad_xyz, T* __restrict__ grad_lengths, T* __restrict__ grad_angles,
    T* __restrict__ grad_dihedrals, const double* __restrict__ state, const double* __restrict__ work, int points,
    int seg_steps, int segments, double* __restrict__ anchor = nullptr) {
  using R = compute_t<T>;
  using Lay = Layout<W, K, Pad>;
  constexpr int kA = 3 * Lay::kStepRow > Lay::kPointRow ? 3 * Lay::kStepRow : Lay::kPointRow;
  __shared__ __align__(16) R pstage[kA];
  __shared__ __align__(16) R gstage[Lay::kPointRow];
  __shared__ R wave_total[W][12];
  __shared__ R wave_sum[W][6];
  __shared__ int wide_vote[W];
  const SegmentOf s = segment_of(blockIdx.x, points, seg_steps, segments, 0);
  const int64_t b = s.chain;
  const int64_t at = b * segments + s.index;
  const bool head = s.index == 0;
  // The head segment's adjoint holds the whole chain's force and moment sums (its carry holds
  // every later segment's): it writes the chain's anchor sums.
  double* const an = head && anchor != nullptr ? anchor + b * 6 : nullptr;
  // Position-based adjoint where this segment and the one before it (which holds the bond
  // x1-x2) passed the forward's tests on their own positions.
  if (FastPath<T>::kEnabled && flags[at] != 0 && (head || flags[at - 1] != 0)) {
    const int64_t row = (b * points + s.first) * 3;
    R* const dst[2] = {pstage, gstage};
    const T* const src[2] = {(head ? xyz : local) + row, grad_xyz + row};
    load_point_rows<Lay, 2>(dst, src, s.steps + 3, threadIdx.x);
    __syncthreads();
    position_adjoint<T, Lay, true>(grad_lengths + b * (points - 1) + s.first, grad_angles + b * (points - 2) + s.first,
                                   grad_dihedrals + b * (points - 3) + s.first, pstage, gstage, wave_sum, s.steps + 3,
                                   an, head, state + at * kLongStateDoubles + 12, work + at * kLongWorkDoubles + 6,
                                   head ? R(0) : widen(lengths[b * (points - 1) + s.first + 1]));
    return;
  }
  exact_chain<T, Lay, true>(lengths + b * (points - 1) + s.first, angles + b * (points - 2) + s.first,
                            dihedrals + b * (points - 3) + s.first, p0, first_direction, initial_normal,
                            grad_xyz + (b * points + s.first) * 3, grad_lengths + b * (points - 1) + s.first,
                            grad_angles + b * (points - 2) + s.first, grad_dihedrals + b * (points - 3) + s.first,
                            pstage, gstage, wave_total, wave_sum, wide_vote, s.steps + 3, s.index == 0,
                            state + at * kLongStateDoubles + 12, work + at * kLongWorkDoubles + 6, an);
}

}  // namespace cufk_amd
