// Torsion-only kernels (reference: src/cufk/csrc/torsion.cu).
//
// Step k uses bond length l[(k+2)%3], bond angle (k+1)%3 and the normalised raw pair k
// (torsion.cu:67-73, 119-141).  K is a multiple of 12: every lane's item i has phase i % 3.
// The forward stages its rows with one pad word per lane (Layout Pad = 1): against Pad = 4
// it needs 81 instead of 97 VGPRs and 9.6 instead of 10.3 KB of LDS at (1, 12), so 16
// workgroups share a CU instead of 15 (at C3, 8192 chains fill two rounds of 16 per CU
// exactly), and measured 29.9 against 33.9 us.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "chain_ops.h"
#include "fused_loss.h"
#include "staging.h"

namespace cufk_amd {

struct TorsionArgs {
  float length[3];
  double sin[3];
  double cos[3];
  float inv_length[3];  // 1.0f / length, formed in float (torsion.cu:216)
};

// Raw pairs (sin, cos interleaved, src[2s], src[2s+1]) into two step-layout rows, two-phase
// like stage_rows: all global loads of the thread are issued before the LDS writes.
template <typename Lay, typename T>
__device__ __forceinline__ void load_pair_rows(compute_t<T>* __restrict__ srow, compute_t<T>* __restrict__ crow,
                                               const T* __restrict__ src, int steps, int tid) {
  using R = compute_t<T>;
  if constexpr (std::is_same_v<T, float>) {
    constexpr int kPer = (Lay::kCap / 2 + Lay::kLanes - 1) / Lay::kLanes;
    const int groups = steps >> 1;  // two pairs per 16 bytes; steps 2g, 2g+1 share a lane (K even)
    f32x4 buf[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int g = tid + j * Lay::kLanes;
      if (g < groups) buf[j] = *reinterpret_cast<const f32x4u*>(src + 4 * g);
    }
    float ts = 0.0f, tc = 0.0f;
    const bool tail = (steps & 1) && tid == 0;
    if (tail) {
      ts = src[2 * (steps - 1)];
      tc = src[2 * (steps - 1) + 1];
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int g = tid + j * Lay::kLanes;
      if (g < groups) {
        const int slot = Lay::step_slot(2 * g);
        srow[slot] = buf[j].x;
        crow[slot] = buf[j].y;
        srow[slot + 1] = buf[j].z;
        crow[slot + 1] = buf[j].w;
      }
    }
    if (tail) {
      srow[Lay::step_slot(steps - 1)] = ts;
      crow[Lay::step_slot(steps - 1)] = tc;
    }
  } else {
    constexpr int kPer = (Lay::kCap + Lay::kLanes - 1) / Lay::kLanes;
    R bs[kPer], bc[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int s = tid + j * Lay::kLanes;
      if (s < steps) {
        bs[j] = widen(src[2 * s]);
        bc[j] = widen(src[2 * s + 1]);
      }
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int s = tid + j * Lay::kLanes;
      if (s < steps) {
        srow[Lay::step_slot(s)] = bs[j];
        crow[Lay::step_slot(s)] = bc[j];
      }
    }
  }
}

// Forward (torsion.cu:254-295).  With LossKind (fused_loss.h) it also reduces the chain's loss
// against target (its (points, 3) row) from the positions as stored: the sum of squares into
// loss[row], or the superposition sums into the chain's record (superpose_records_kernel
// follows).
template <typename T, int W, int K, int LossKind = kLossNone>
__global__ __launch_bounds__(64 * W) void torsion_forward_kernel(const T* __restrict__ raw_pairs, int64_t raw_stride,
                                                                 TorsionArgs cst, T* __restrict__ xyz, int points,
                                                                 const T* __restrict__ target = nullptr,
                                                                 T* __restrict__ loss = nullptr,
                                                                 double* __restrict__ record = nullptr) {
  constexpr bool Loss = LossKind != kLossNone;
  static_assert(K % 12 == 0, "torsion plans keep phases lane-invariant and segments 16-byte aligned");
  using R = compute_t<T>;
  using Lay = Layout<W, K, 1>;
  constexpr int kStage = 2 * Lay::kStepRow > Lay::kPointRow ? 2 * Lay::kStepRow : Lay::kPointRow;
  __shared__ __align__(16) R stage[kStage];
  __shared__ R wave_total[W][12];

  const int steps = points - 3;
  const int64_t row = blockIdx.x;
  const T* raw = raw_pairs + row * raw_stride;
  T* out = xyz + row * points * 3;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  load_pair_rows<Lay>(stage, stage + Lay::kStepRow, raw, steps, tid);
  const int s0 = tid * K;
  const int b0 = Lay::lane_step_base(tid);
  // Items past the chain's end take the pair (0, 1), a zero torsion, so that every lane runs
  // its K items without a guard (no exec-mask branches or register copies per item); their
  // positions are never stored.
  for (int i = steps - s0 > 0 ? steps - s0 : 0; i < K; ++i) {
    stage[b0 + i] = R(0);
    stage[Lay::kStepRow + b0 + i] = R(1);
  }
  const T* tgt = Loss ? target + row * points * 3 : nullptr;
  // The target of the lane's own points, loaded now so that the scan hides the latency.
  R tr[Loss ? 3 * K : 1];
  if constexpr (Loss) {
    const int count = steps - s0 < K ? (steps - s0 > 0 ? steps - s0 : 0) : K;
    load_run<3 * K>(tgt + 9 + 3 * s0, 3 * count, tr);
  }
  __syncthreads();

  // Serial part in double with the float64 bond-angle sin/cos (the reference rounds them to
  // the compute type, torsion.cu:226-227, which biases |M| per phase along the chain).
  Rigid<double> q = rigid_identity<double>();
  R y[K][3];
#pragma unroll
  for (int i = 0; i < K; ++i) {
    const int lp = (i + 2) % 3;  // torsion.cu:67-69
    const int ap = (i + 1) % 3;  // torsion.cu:71-73
    double S, C;
    pair_unit(stage[b0 + i], stage[Lay::kStepRow + b0 + i], S, C);
    step_forward(q.m, q.v, static_cast<double>(cst.length[lp]), cst.sin[ap], cst.cos[ap], S, C);
    y[i][0] = static_cast<R>(q.v[0]);
    y[i][1] = static_cast<R>(q.v[1]);
    y[i][2] = static_cast<R>(q.v[2]);
    __builtin_amdgcn_sched_barrier(0);  // one item per scheduling region: no hoisting across items
  }

  const Rigid<R> excl = lane_carry<R, W>(narrow_rigid<R>(q), wave_total, lane, wave);

  // Constant base (torsion.cu:149-166): x0 = 0, x1 = (l0,0,0), x2 = (l0 - l1 c0, l1 s0, 0),
  // F = [(-c0, s0, 0) | (-s0, -c0, 0) | (0, 0, 1)].
  const R s0a = static_cast<R>(cst.sin[0]), c0a = static_cast<R>(cst.cos[0]);
  const R l0 = static_cast<R>(cst.length[0]), l1 = static_cast<R>(cst.length[1]);
  const V3<R> p2 = {l0 - l1 * c0a, l1 * s0a, R(0)};
  R gm[9];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    gm[c] = -c0a * excl.m[c] - s0a * excl.m[3 + c];
    gm[3 + c] = s0a * excl.m[c] - c0a * excl.m[3 + c];
    gm[6 + c] = excl.m[6 + c];
  }
  const V3<R> gv = {p2.x + (-c0a * excl.v[0] - s0a * excl.v[1]), p2.y + (s0a * excl.v[0] - c0a * excl.v[1]),
                    p2.z + excl.v[2]};

  LossAccumulator<LossKind, R> lossacc;
  auto stored = [](V3<R> x) { return V3<R>{widen(narrow<T>(x.x)), widen(narrow<T>(x.y)), widen(narrow<T>(x.z))}; };
  // Superposed sums about the stored x2 and the target's point 2 for the chain, the thread's
  // first point and its target for the thread.
  if constexpr (LossKind == kLossSuperposed) lossacc.chain_shift(stored(p2), V3<R>{widen(tgt[6]), widen(tgt[7]), widen(tgt[8])});
  const int o0 = Lay::lane_point_base(tid);
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (s0 + i < steps) {
      // gv as the addend of the first fma: three issues per coordinate, not four.
      const V3<R> x = {fma(gm[2], y[i][2], fma(gm[1], y[i][1], fma(gm[0], y[i][0], gv.x))),
                       fma(gm[5], y[i][2], fma(gm[4], y[i][1], fma(gm[3], y[i][0], gv.y))),
                       fma(gm[8], y[i][2], fma(gm[7], y[i][1], fma(gm[6], y[i][0], gv.z)))};
      if constexpr (Loss) {
        const V3<R> xs = stored(x);
        if constexpr (LossKind == kLossSuperposed) {
          if (i == 0) lossacc.local_shift(xs, V3<R>{tr[0], tr[1], tr[2]});
        }
        lossacc.add(xs, V3<R>{tr[3 * i], tr[3 * i + 1], tr[3 * i + 2]});
      }
      stage[o0 + 3 * i] = x.x;
      stage[o0 + 3 * i + 1] = x.y;
      stage[o0 + 3 * i + 2] = x.z;
    }
  }
  if (tid == 0) {
    stage[0] = R(0); stage[1] = R(0); stage[2] = R(0);
    stage[3] = l0;   stage[4] = R(0); stage[5] = R(0);
    stage[6] = p2.x; stage[7] = p2.y; stage[8] = p2.z;
    if constexpr (Loss) {
      const V3<R> h[3] = {{R(0), R(0), R(0)}, {l0, R(0), R(0)}, p2};
#pragma unroll
      for (int j = 0; j < 3; ++j)
        lossacc.add(stored(h[j]), V3<R>{widen(tgt[3 * j]), widen(tgt[3 * j + 1]), widen(tgt[3 * j + 2])});
    }
  }
  if constexpr (Loss) {
    lossacc.template finish<T, W>(loss != nullptr ? loss + row : nullptr,
                                  record != nullptr ? record + row * kSuperposeRecord : nullptr, lane, wave, tid);
  } else {
    __syncthreads();
  }
  store_point_row<Lay>(out, stage, points, tid);
}

// Backward (torsion.cu:297-381) over the saved positions:
//   dphi_k = (1/l_{(k+1)%3}) (x_{k+2} - x_{k+1}) . (M_{k+3} - x_{k+2} x F_{k+3}),
//   raw grad = dphi (rc, -rs) / max(rs^2 + rc^2, 1e-16) (torsion.cu:173-182),
// with positions relative to x2 (the moments are translation invariant).  No LDS staging:
// each lane moves its own contiguous runs (points s0 .. s0+K+2, their gradients, its raw
// pairs and its raw-pair gradients) straight between HBM and registers; only the wave sums
// of the suffix scan go through LDS.  With K = 3 (the smallest multiple of the phase period)
// a workgroup per chain holds up to eight waves per SIMD, where staging whole rows through
// LDS held one or two.
//
// With LossKind (fused_loss.h) grad_xyz is the loss's target row instead, and the gradient of
// each point is formed from its position and target as the lane loads them (grad_loss: the
// upstream weight per chain, or NULL for ones; record: the superposed kinds' records).
template <typename T, int W, int K, int LossKind = kLossNone>
__global__ __launch_bounds__(64 * W) void torsion_backward_kernel(const T* __restrict__ raw_pairs, int64_t raw_stride,
                                                                  const T* __restrict__ xyz, const T* __restrict__ grad_xyz,
                                                                  T* __restrict__ grad_raw, int64_t grad_raw_stride,
                                                                  TorsionArgs cst, int points,
                                                                  const T* __restrict__ grad_loss = nullptr,
                                                                  const double* __restrict__ record = nullptr,
                                                                  int squared = 0) {
  static_assert(K % 3 == 0, "torsion plans keep phases lane-invariant");
  using R = compute_t<T>;
  __shared__ R wave_sum[W][6];

  const int steps = points - 3;
  const int64_t row = blockIdx.x;
  const T* raw = raw_pairs + row * raw_stride;
  const T* Xr = xyz + row * points * 3;
  const T* Gr = grad_xyz + row * points * 3;
  T* graw = grad_raw + row * grad_raw_stride;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int s0 = tid * K;
  const int count = steps - s0 < K ? (steps - s0 > 0 ? steps - s0 : 0) : K;
  const int last = count - 1;

  R xr[3 * K + 9], gr[3 * K], pr[2 * K];
  load_run<3 * K + 9>(Xr + 3 * s0, count > 0 ? 3 * (count + 3) : 0, xr);
  load_run<3 * K>(Gr + 9 + 3 * s0, 3 * count, gr);
  load_run<2 * K>(raw + 2 * s0, 2 * count, pr);
  if constexpr (LossKind != kLossNone) {  // gr holds the target: form each point's gradient
    const R w = grad_loss != nullptr ? widen(grad_loss[row]) : R(1);
    const auto res = make_residual<LossKind>(w, record != nullptr ? record + row * kSuperposeRecord : nullptr, points,
                                             squared);
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const V3<R> g = res(V3<R>{xr[9 + 3 * i], xr[10 + 3 * i], xr[11 + 3 * i]},
                          V3<R>{gr[3 * i], gr[3 * i + 1], gr[3 * i + 2]});
      gr[3 * i] = g.x;
      gr[3 * i + 1] = g.y;
      gr[3 * i + 2] = g.z;
    }
  }
  const V3<R> c = {widen(Xr[6]), widen(Xr[7]), widen(Xr[8])};
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

  V3<R> F = tail.f, M = tail.m;
  const R eps2 = static_cast<R>(1.0e-8f * 1.0e-8f);
  R go[2 * K];
#pragma unroll
  for (int i = K - 1; i >= 0; --i) {
    go[2 * i] = go[2 * i + 1] = R(0);
    if (i <= last) {
      const V3<R> xa = pos(i + 3), xb = pos(i + 2), xc = pos(i + 1);
      const V3<R> g = {gr[3 * i], gr[3 * i + 1], gr[3 * i + 2]};
      F = F + g;
      M = M + cross(xa, g);
      const R dphi = static_cast<R>(cst.inv_length[(i + 1) % 3]) * dot(xb - xc, M - cross(xb, F));
      const R rs = pr[2 * i], rc = pr[2 * i + 1];
      const R n2 = rs * rs + rc * rc;
      const R scale = dphi / (n2 < eps2 ? eps2 : n2);
      go[2 * i] = rc * scale;
      go[2 * i + 1] = -rs * scale;
    }
  }
  store_run<2 * K>(graw + 2 * s0, 2 * count, go);  // per-lane runs: nontemporal measured slower
}

}  // namespace cufk_amd
