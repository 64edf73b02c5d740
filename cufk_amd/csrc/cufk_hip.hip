// HIP kernels and C ABI for NeRF chain reconstruction on MI355X (gfx950).
//
// One workgroup of W wave64s reconstructs one chain.  Lane t owns the K consecutive steps
// [t*K, t*K + K) (blocked arrangement, as in the reference block.cu:187), so each lane runs
// a serial scan of K NeRF steps in registers and only lane totals cross lanes: a wave64
// DPP scan of 3x4 rigid transforms, then an LDS carry across the W waves.  Inputs and
// outputs pass through LDS so every global access is a coalesced row stream; LDS rows are
// padded by one word per lane so the per-lane (stride K+1 / 3K+1) accesses are free of
// bank conflicts.
#include "chain_ops.h"
#include "cufk_hip.h"

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

namespace cufk_amd {

constexpr int kMaxSteps = 2048;  // block.cu:88, torsion.cu:97 (512 threads x 4 items)

template <int W, int K> struct Layout {
  static constexpr int kLanes = 64 * W;
  static constexpr int kCap = kLanes * K;                    // steps per chain
  static constexpr int kParamRow = kLanes * (K + 1);         // one padded per-step row
  static constexpr int kPointRow = 9 + kLanes * (3 * K + 1); // padded (N, 3) row
  __device__ __forceinline__ static int param_slot(int s) { return s + s / K; }
  // Flat xyz element e = 3*point + component -> padded LDS slot.  Points 0..2 sit first;
  // point s+3 belongs to lane s/K.
  __device__ __forceinline__ static int point_slot(int e) {
    if (e < 9) return e;
    const int t = e - 9;
    return 9 + (t / (3 * K)) * (3 * K + 1) + t % (3 * K);
  }
};

template <typename R> __device__ __forceinline__ V3<R> load3(const R* p) { return {p[0], p[1], p[2]}; }

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
// Contains one __syncthreads(); must be called by every thread of the workgroup.
template <typename R, int W>
__device__ __forceinline__ Rigid<R> lane_carry(const Rigid<R>& lane_total, R (&wave_total)[W][12], int lane, int wave) {
  const Rigid<R> incl = wave_prefix(lane_total);
  if (lane == 63) store_rigid(wave_total, wave, incl);
  Rigid<R> excl = wave_shift_up(incl, lane);
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

// ============================================================================ reconstruct

// Forward (block.cu:157-204): x0 = p0, x1, x2 from the first frame, x_{k+3} = p2 + F P_k.v.
template <typename T, int W, int K>
__global__ __launch_bounds__(64 * W) void reconstruct_forward_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    T* __restrict__ xyz, int points) {
  using R = compute_t<T>;
  using Lay = Layout<W, K>;
  constexpr int kStage = 3 * Lay::kParamRow > Lay::kPointRow ? 3 * Lay::kParamRow : Lay::kPointRow;
  __shared__ R stage[kStage];
  __shared__ R wave_total[W][12];

  const int steps = points - 3;
  const int64_t row = blockIdx.x;
  const T* Lr = lengths + row * (points - 1);
  const T* Ar = angles + row * (points - 2);
  const T* Dr = dihedrals + row * (points - 3);
  T* out = xyz + row * points * 3;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  for (int s = tid; s < steps; s += Lay::kLanes) {
    const int slot = Lay::param_slot(s);
    stage[slot] = widen(Lr[s + 2]);
    stage[Lay::kParamRow + slot] = widen(Ar[s + 1]);
    stage[2 * Lay::kParamRow + slot] = widen(Dr[s]);
  }
  const FirstFrame<R> ff = first_frame<T>(widen(Lr[0]), widen(Lr[1]), widen(Ar[0]), p0, first_direction, initial_normal);
  __syncthreads();

  // Lane-local serial scan in double (rounding only at the lane boundary); y[i] = translation
  // of the local prefix after item i.
  Rigid<double> q = rigid_identity<double>();
  R y[K][3];
  const int s0 = tid * K;
  const int b0 = tid * (K + 1);
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (s0 + i < steps) {
      const R l = stage[b0 + i];
      const R th = stage[Lay::kParamRow + b0 + i];
      const R ph = stage[2 * Lay::kParamRow + b0 + i];
      double s, c, S, C;
      sin_cos_wide(th, s, c);
      sin_cos_wide(ph, S, C);
      step_forward(q.m, q.v, static_cast<double>(l), s, c, S, C);
    }
    y[i][0] = static_cast<R>(q.v[0]);
    y[i][1] = static_cast<R>(q.v[1]);
    y[i][2] = static_cast<R>(q.v[2]);
  }

  const Rigid<R> excl = lane_carry<R, W>(narrow_rigid<R>(q), wave_total, lane, wave);

  // World transform at the lane start: (F, p2) o excl.
  R gm[9], gv[3];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c)
      gm[3 * r + c] = ff.frame[3 * r] * excl.m[c] + ff.frame[3 * r + 1] * excl.m[3 + c] + ff.frame[3 * r + 2] * excl.m[6 + c];
  }
  const V3<R> ev = rot_apply(ff.frame, V3<R>{excl.v[0], excl.v[1], excl.v[2]});
  gv[0] = ff.p2.x + ev.x;
  gv[1] = ff.p2.y + ev.y;
  gv[2] = ff.p2.z + ev.z;

  // The output row aliases the parameter rows: every parameter read precedes the
  // barrier inside lane_carry.
  const int o0 = 9 + tid * (3 * K + 1);
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (s0 + i < steps) {
#pragma unroll
      for (int r = 0; r < 3; ++r)
        stage[o0 + 3 * i + r] = gv[r] + gm[3 * r] * y[i][0] + gm[3 * r + 1] * y[i][1] + gm[3 * r + 2] * y[i][2];
    }
  }
  if (tid == 0) {
    stage[0] = ff.p0.x; stage[1] = ff.p0.y; stage[2] = ff.p0.z;
    stage[3] = ff.p1.x; stage[4] = ff.p1.y; stage[5] = ff.p1.z;
    stage[6] = ff.p2.x; stage[7] = ff.p2.y; stage[8] = ff.p2.z;
  }
  __syncthreads();
  const int total = 3 * points;
  for (int e = tid; e < total; e += Lay::kLanes) out[e] = narrow<T>(stage[Lay::point_slot(e)]);
}

// Backward: world-frame adjoint with exact frame axes, recomputing the forward scan.
//   F_i = sum_{j>=i} g_j,  M_i = sum_{j>=i} x_j x g_j,  tau = M_{k+3} - x_{k+2} x F_{k+3}
//   dL/dL[k+2] = R_k[:,0].F_{k+3},  dL/dA[k+1] = -R_k[:,2].tau,  dL/dD[k] = R_{k-1}[:,0].tau
// with R_k the world rotation after step k; first-frame terms as block.cu:206-228.
// Positions are taken relative to x2 (the moments are translation invariant).
template <typename T, int W, int K>
__global__ __launch_bounds__(64 * W) void reconstruct_backward_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    const T* __restrict__ grad_xyz, T* __restrict__ grad_lengths, T* __restrict__ grad_angles,
    T* __restrict__ grad_dihedrals, int points) {
  using R = compute_t<T>;
  using Lay = Layout<W, K>;
  __shared__ R pstage[3 * Lay::kParamRow];  // parameters in, their gradients out
  __shared__ R gstage[Lay::kPointRow];      // upstream gradient
  __shared__ R wave_total[W][12];
  __shared__ R wave_sum[W][6];

  const int steps = points - 3;
  const int64_t row = blockIdx.x;
  const T* Lr = lengths + row * (points - 1);
  const T* Ar = angles + row * (points - 2);
  const T* Dr = dihedrals + row * (points - 3);
  const T* Gr = grad_xyz + row * points * 3;
  T* gLr = grad_lengths + row * (points - 1);
  T* gAr = grad_angles + row * (points - 2);
  T* gDr = grad_dihedrals + row * (points - 3);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  for (int s = tid; s < steps; s += Lay::kLanes) {
    const int slot = Lay::param_slot(s);
    pstage[slot] = widen(Lr[s + 2]);
    pstage[Lay::kParamRow + slot] = widen(Ar[s + 1]);
    pstage[2 * Lay::kParamRow + slot] = widen(Dr[s]);
  }
  const int total = 3 * points;
  for (int e = tid; e < total; e += Lay::kLanes) gstage[Lay::point_slot(e)] = widen(Gr[e]);
  const FirstFrame<R> ff = first_frame<T>(widen(Lr[0]), widen(Lr[1]), widen(Ar[0]), p0, first_direction, initial_normal);
  __syncthreads();

  // Pass 1: lane-local scan (double); keep sin/cos; accumulate Y = sum_i y_i g_i^T and sum_i g_i.
  Rigid<double> qd = rigid_identity<double>();
  R sc[K][4];
  R Y[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) Y[i] = R(0);
  V3<R> gsum = {R(0), R(0), R(0)};
  const int s0 = tid * K;
  const int b0 = tid * (K + 1);
  const int o0 = 9 + tid * (3 * K + 1);
#pragma unroll
  for (int i = 0; i < K; ++i) {
    sc[i][0] = sc[i][1] = sc[i][2] = sc[i][3] = R(0);
    if (s0 + i < steps) {
      const R l = pstage[b0 + i];
      const R th = pstage[Lay::kParamRow + b0 + i];
      const R ph = pstage[2 * Lay::kParamRow + b0 + i];
      double s, c, S, C;
      sin_cos_wide(th, s, c);
      sin_cos_wide(ph, S, C);
      sc[i][0] = static_cast<R>(s);
      sc[i][1] = static_cast<R>(c);
      sc[i][2] = static_cast<R>(S);
      sc[i][3] = static_cast<R>(C);
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

  const Rigid<R> q = narrow_rigid<R>(qd);
  const Rigid<R> excl = lane_carry<R, W>(q, wave_total, lane, wave);

  // World frame at the lane start, origin at x2: R0 = F excl.m, X0 = F excl.v.
  R R0[9];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c)
      R0[3 * r + c] = ff.frame[3 * r] * excl.m[c] + ff.frame[3 * r + 1] * excl.m[3 + c] + ff.frame[3 * r + 2] * excl.m[6 + c];
  }
  const V3<R> X0 = rot_apply(ff.frame, V3<R>{excl.v[0], excl.v[1], excl.v[2]});

  // Lane moment: sum_i (X0 + R0 y_i) x g_i = X0 x gsum + skew part of R0 Y.
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

  // Pass 3: walk the lane's steps backwards.
  V3<R> F = tail.f, M = tail.m;
#pragma unroll
  for (int i = K - 1; i >= 0; --i) {
    if (s0 + i < steps) {
      const V3<R> g = load3(&gstage[o0 + 3 * i]);
      F = F + g;
      M = M + cross(x, g);
      const R l = pstage[b0 + i];
      const V3<R> col0 = {Rm[0], Rm[3], Rm[6]};
      const V3<R> col2 = {Rm[2], Rm[5], Rm[8]};
      const V3<R> xp = x - l * col0;
      const V3<R> tau = M - cross(xp, F);
      const R gl = dot(col0, F);
      const R ga = -dot(col2, tau);
      step_backward(Rm, sc[i][0], sc[i][1], sc[i][2], sc[i][3]);
      const R gd = dot(V3<R>{Rm[0], Rm[3], Rm[6]}, tau);
      pstage[b0 + i] = gl;
      pstage[Lay::kParamRow + b0 + i] = ga;
      pstage[2 * Lay::kParamRow + b0 + i] = gd;
      x = xp;
    }
  }
  if (tid == 0) {
    // First-frame parameters (block.cu:206-228): x2 is the origin, so M_2 = M_3.
    const V3<R> g1 = load3(&gstage[3]);
    const V3<R> g2 = load3(&gstage[6]);
    const V3<R> F2 = F + g2;
    const V3<R> x1 = ff.p1 - ff.p2;
    const V3<R> tau2 = M - cross(x1, F2);
    gLr[0] = narrow<T>(dot(ff.d0, F2 + g1));
    gLr[1] = narrow<T>(dot(ff.d1, F2));
    gAr[0] = narrow<T>(-dot(cross(ff.d0, ff.t0), tau2));
  }
  __syncthreads();
  for (int s = tid; s < steps; s += Lay::kLanes) {
    const int slot = Lay::param_slot(s);
    gLr[s + 2] = narrow<T>(pstage[slot]);
    gAr[s + 1] = narrow<T>(pstage[Lay::kParamRow + slot]);
    gDr[s] = narrow<T>(pstage[2 * Lay::kParamRow + slot]);
  }
}

// ============================================================================ torsion

struct TorsionArgs {
  float length[3];
  double sin[3];
  double cos[3];
  float inv_length[3];  // 1.0f / length (torsion.cu:216)
};

// Forward (torsion.cu:254-295).  K is a multiple of 3, so item i of every lane has phase i%3.
template <typename T, int W, int K>
__global__ __launch_bounds__(64 * W) void torsion_forward_kernel(const T* __restrict__ raw_pairs, int64_t raw_stride,
                                                                 TorsionArgs cst, T* __restrict__ xyz, int points) {
  static_assert(K % 3 == 0, "torsion plans keep phases lane-invariant");
  using R = compute_t<T>;
  using Lay = Layout<W, K>;
  constexpr int kStage = 2 * Lay::kParamRow > Lay::kPointRow ? 2 * Lay::kParamRow : Lay::kPointRow;
  __shared__ R stage[kStage];
  __shared__ R wave_total[W][12];

  const int steps = points - 3;
  const int64_t row = blockIdx.x;
  const T* raw = raw_pairs + row * raw_stride;
  T* out = xyz + row * points * 3;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  for (int e = tid; e < 2 * steps; e += Lay::kLanes)
    stage[(e & 1) * Lay::kParamRow + Lay::param_slot(e >> 1)] = widen(raw[e]);
  __syncthreads();

  // Serial part in double with the float64 bond-angle sin/cos (the reference rounds them to
  // the compute type, torsion.cu:226-227, which biases |M| per phase).
  Rigid<double> q = rigid_identity<double>();
  R y[K][3];
  const int s0 = tid * K;
  const int b0 = tid * (K + 1);
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (s0 + i < steps) {
      const int lp = (i + 2) % 3;  // torsion.cu:67-69
      const int ap = (i + 1) % 3;  // torsion.cu:71-73
      double S, C;
      pair_unit(stage[b0 + i], stage[Lay::kParamRow + b0 + i], S, C);
      step_forward(q.m, q.v, static_cast<double>(cst.length[lp]), cst.sin[ap], cst.cos[ap], S, C);
    }
    y[i][0] = static_cast<R>(q.v[0]);
    y[i][1] = static_cast<R>(q.v[1]);
    y[i][2] = static_cast<R>(q.v[2]);
  }

  const Rigid<R> excl = lane_carry<R, W>(narrow_rigid<R>(q), wave_total, lane, wave);

  // Constant base (torsion.cu:149-166): x0 = 0, x1 = (l0,0,0), x2 = (l0 - l1 c0, l1 s0, 0),
  // F = [(-c0, s0, 0) | (-s0, -c0, 0) | (0, 0, 1)].
  const R s0a = static_cast<R>(cst.sin[0]), c0a = static_cast<R>(cst.cos[0]);
  const R l0 = static_cast<R>(cst.length[0]), l1 = static_cast<R>(cst.length[1]);
  const V3<R> p2 = {l0 - l1 * c0a, l1 * s0a, R(0)};
  // World at lane start: rows of F applied to excl.
  R gm[9];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    gm[c] = -c0a * excl.m[c] - s0a * excl.m[3 + c];
    gm[3 + c] = s0a * excl.m[c] - c0a * excl.m[3 + c];
    gm[6 + c] = excl.m[6 + c];
  }
  const R gv[3] = {p2.x + (-c0a * excl.v[0] - s0a * excl.v[1]), p2.y + (s0a * excl.v[0] - c0a * excl.v[1]),
                   p2.z + excl.v[2]};

  const int o0 = 9 + tid * (3 * K + 1);
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (s0 + i < steps) {
#pragma unroll
      for (int r = 0; r < 3; ++r)
        stage[o0 + 3 * i + r] = gv[r] + gm[3 * r] * y[i][0] + gm[3 * r + 1] * y[i][1] + gm[3 * r + 2] * y[i][2];
    }
  }
  if (tid == 0) {
    stage[0] = R(0); stage[1] = R(0); stage[2] = R(0);
    stage[3] = l0;   stage[4] = R(0); stage[5] = R(0);
    stage[6] = p2.x; stage[7] = p2.y; stage[8] = p2.z;
  }
  __syncthreads();
  const int total = 3 * points;
  for (int e = tid; e < total; e += Lay::kLanes) out[e] = narrow<T>(stage[Lay::point_slot(e)]);
}

// Backward (torsion.cu:297-381): reverse force/moment scan over the saved positions,
// dphi_k = (1/l_{(k+1)%3}) (x_{k+2} - x_{k+1}).(M_{k+3} - x_{k+2} x F_{k+3}),
// raw grad = dphi (rc, -rs) / max(rs^2 + rc^2, 1e-16) (torsion.cu:173-182).
template <typename T, int W, int K>
__global__ __launch_bounds__(64 * W) void torsion_backward_kernel(const T* __restrict__ raw_pairs, int64_t raw_stride,
                                                                  const T* __restrict__ xyz, const T* __restrict__ grad_xyz,
                                                                  T* __restrict__ grad_raw, int64_t grad_raw_stride,
                                                                  TorsionArgs cst, int points) {
  static_assert(K % 3 == 0, "torsion plans keep phases lane-invariant");
  using R = compute_t<T>;
  using Lay = Layout<W, K>;
  __shared__ R xstage[Lay::kPointRow];
  __shared__ R gstage[Lay::kPointRow];
  __shared__ R rstage[2 * Lay::kParamRow];  // raw pairs in, their gradients out
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

  const int total = 3 * points;
  for (int e = tid; e < total; e += Lay::kLanes) {
    const int slot = Lay::point_slot(e);
    xstage[slot] = widen(Xr[e]);
    gstage[slot] = widen(Gr[e]);
  }
  for (int e = tid; e < 2 * steps; e += Lay::kLanes)
    rstage[(e & 1) * Lay::kParamRow + Lay::param_slot(e >> 1)] = widen(raw[e]);
  __syncthreads();

  const int s0 = tid * K;
  const int b0 = tid * (K + 1);
  const int o0 = 9 + tid * (3 * K + 1);
  ForceMoment<R> lane_sum = {{R(0), R(0), R(0)}, {R(0), R(0), R(0)}};
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (s0 + i < steps) {
      const V3<R> xp = load3(&xstage[o0 + 3 * i]);
      const V3<R> g = load3(&gstage[o0 + 3 * i]);
      lane_sum.f = lane_sum.f + g;
      lane_sum.m = lane_sum.m + cross(xp, g);
    }
  }
  const ForceMoment<R> tail = lane_suffix<R, W>(lane_sum, wave_sum, lane, wave);

  V3<R> F = tail.f, M = tail.m;
  const R eps2 = static_cast<R>(1.0e-8f * 1.0e-8f);
#pragma unroll
  for (int i = K - 1; i >= 0; --i) {
    const int s = s0 + i;
    if (s < steps) {
      const V3<R> xk = load3(&xstage[o0 + 3 * i]);
      const V3<R> g = load3(&gstage[o0 + 3 * i]);
      F = F + g;
      M = M + cross(xk, g);
      const V3<R> pivot = load3(&xstage[Lay::point_slot(3 * (s + 2))]);
      const V3<R> prev = s == 0 ? V3<R>{static_cast<R>(cst.length[0]), R(0), R(0)}
                                : load3(&xstage[Lay::point_slot(3 * (s + 1))]);
      const R inv_len = static_cast<R>(cst.inv_length[(i + 1) % 3]);
      const R dphi = inv_len * dot(pivot - prev, M - cross(pivot, F));
      const R rs = rstage[b0 + i];
      const R rc = rstage[Lay::kParamRow + b0 + i];
      const R n2 = rs * rs + rc * rc;
      const R scale = dphi / (n2 < eps2 ? eps2 : n2);
      rstage[b0 + i] = rc * scale;
      rstage[Lay::kParamRow + b0 + i] = -rs * scale;
    }
  }
  __syncthreads();
  for (int e = tid; e < 2 * steps; e += Lay::kLanes)
    graw[e] = narrow<T>(rstage[(e & 1) * Lay::kParamRow + Lay::param_slot(e >> 1)]);
}

// ============================================================================ launch plans

// Plans are (waves W, items per lane K); capacity 64*W*K steps.  The smallest plan that
// holds the chain is used.
struct PlanChoice {
  int waves;
  int items;
};

inline PlanChoice reconstruct_plan(int steps) {
  if (steps <= 256) return {1, 4};
  if (steps <= 512) return {1, 8};
  if (steps <= 1024) return {2, 8};
  return {4, 8};
}

inline PlanChoice torsion_plan(int steps) {
  if (steps <= 192) return {1, 3};
  if (steps <= 384) return {1, 6};
  if (steps <= 768) return {2, 6};
  if (steps <= 1536) return {4, 6};
  return {4, 9};
}

// Workgroups per launch: HIP's grid x extent counts work-items in 32 bits.
inline int64_t max_blocks_per_launch(int threads) { return (int64_t{UINT32_MAX} / threads); }

template <typename Fn> int launch_chunks(int64_t batch, int threads, Fn fn) {
  const int64_t chunk = max_blocks_per_launch(threads);
  for (int64_t done = 0; done < batch; done += chunk) {
    const int64_t n = batch - done < chunk ? batch - done : chunk;
    fn(done, static_cast<unsigned>(n));
    if (hipGetLastError() != hipSuccess) return CUFK_ERR_LAUNCH;
  }
  return CUFK_OK;
}

template <typename T, int W, int K>
int launch_reconstruct_fwd(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz, int64_t B,
                           int N, hipStream_t stream) {
  return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
    hipLaunchKernelGGL((reconstruct_forward_kernel<T, W, K>), dim3(n), dim3(64 * W), 0, stream, L + off * (N - 1),
                       A + off * (N - 2), D + off * (N - 3), p0, fd, n0, xyz + off * N * 3, N);
  });
}

template <typename T, int W, int K>
int launch_reconstruct_bwd(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* g, T* gL,
                           T* gA, T* gD, int64_t B, int N, hipStream_t stream) {
  return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
    hipLaunchKernelGGL((reconstruct_backward_kernel<T, W, K>), dim3(n), dim3(64 * W), 0, stream, L + off * (N - 1),
                       A + off * (N - 2), D + off * (N - 3), p0, fd, n0, g + off * N * 3, gL + off * (N - 1),
                       gA + off * (N - 2), gD + off * (N - 3), N);
  });
}

template <typename T, int W, int K>
int launch_torsion_fwd(const T* raw, int64_t rs, const TorsionArgs& c, T* xyz, int64_t B, int N, hipStream_t stream) {
  return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
    hipLaunchKernelGGL((torsion_forward_kernel<T, W, K>), dim3(n), dim3(64 * W), 0, stream, raw + off * rs, rs, c,
                       xyz + off * N * 3, N);
  });
}

template <typename T, int W, int K>
int launch_torsion_bwd(const T* raw, int64_t rs, const T* xyz, const T* g, T* graw, int64_t gs, const TorsionArgs& c,
                       int64_t B, int N, hipStream_t stream) {
  return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
    hipLaunchKernelGGL((torsion_backward_kernel<T, W, K>), dim3(n), dim3(64 * W), 0, stream, raw + off * rs, rs,
                       xyz + off * N * 3, g + off * N * 3, graw + off * gs, gs, c, N);
  });
}

template <typename T>
int reconstruct_fwd_typed(const void* L, const void* A, const void* D, const void* p0, const void* fd, const void* n0,
                          void* xyz, int64_t B, int N, hipStream_t st) {
  auto* l = static_cast<const T*>(L);
  auto* a = static_cast<const T*>(A);
  auto* d = static_cast<const T*>(D);
  auto* p = static_cast<const T*>(p0);
  auto* f = static_cast<const T*>(fd);
  auto* n = static_cast<const T*>(n0);
  auto* x = static_cast<T*>(xyz);
  const PlanChoice pc = reconstruct_plan(N - 3);
  if (pc.waves == 1 && pc.items == 4) return launch_reconstruct_fwd<T, 1, 4>(l, a, d, p, f, n, x, B, N, st);
  if (pc.waves == 1 && pc.items == 8) return launch_reconstruct_fwd<T, 1, 8>(l, a, d, p, f, n, x, B, N, st);
  if (pc.waves == 2) return launch_reconstruct_fwd<T, 2, 8>(l, a, d, p, f, n, x, B, N, st);
  return launch_reconstruct_fwd<T, 4, 8>(l, a, d, p, f, n, x, B, N, st);
}

template <typename T>
int reconstruct_bwd_typed(const void* L, const void* A, const void* D, const void* p0, const void* fd, const void* n0,
                          const void* g, void* gL, void* gA, void* gD, int64_t B, int N, hipStream_t st) {
  auto* l = static_cast<const T*>(L);
  auto* a = static_cast<const T*>(A);
  auto* d = static_cast<const T*>(D);
  auto* p = static_cast<const T*>(p0);
  auto* f = static_cast<const T*>(fd);
  auto* n = static_cast<const T*>(n0);
  auto* gx = static_cast<const T*>(g);
  auto* ol = static_cast<T*>(gL);
  auto* oa = static_cast<T*>(gA);
  auto* od = static_cast<T*>(gD);
  const PlanChoice pc = reconstruct_plan(N - 3);
  if (pc.waves == 1 && pc.items == 4) return launch_reconstruct_bwd<T, 1, 4>(l, a, d, p, f, n, gx, ol, oa, od, B, N, st);
  if (pc.waves == 1 && pc.items == 8) return launch_reconstruct_bwd<T, 1, 8>(l, a, d, p, f, n, gx, ol, oa, od, B, N, st);
  if (pc.waves == 2) return launch_reconstruct_bwd<T, 2, 8>(l, a, d, p, f, n, gx, ol, oa, od, B, N, st);
  return launch_reconstruct_bwd<T, 4, 8>(l, a, d, p, f, n, gx, ol, oa, od, B, N, st);
}

template <typename T>
int torsion_fwd_typed(const void* raw, int64_t rs, const TorsionArgs& c, void* xyz, int64_t B, int N, hipStream_t st) {
  auto* r = static_cast<const T*>(raw);
  auto* x = static_cast<T*>(xyz);
  const PlanChoice pc = torsion_plan(N - 3);
  if (pc.waves == 1 && pc.items == 3) return launch_torsion_fwd<T, 1, 3>(r, rs, c, x, B, N, st);
  if (pc.waves == 1 && pc.items == 6) return launch_torsion_fwd<T, 1, 6>(r, rs, c, x, B, N, st);
  if (pc.waves == 2) return launch_torsion_fwd<T, 2, 6>(r, rs, c, x, B, N, st);
  if (pc.items == 6) return launch_torsion_fwd<T, 4, 6>(r, rs, c, x, B, N, st);
  return launch_torsion_fwd<T, 4, 9>(r, rs, c, x, B, N, st);
}

template <typename T>
int torsion_bwd_typed(const void* raw, int64_t rs, const void* xyz, const void* g, void* graw, int64_t gs,
                      const TorsionArgs& c, int64_t B, int N, hipStream_t st) {
  auto* r = static_cast<const T*>(raw);
  auto* x = static_cast<const T*>(xyz);
  auto* gx = static_cast<const T*>(g);
  auto* o = static_cast<T*>(graw);
  const PlanChoice pc = torsion_plan(N - 3);
  if (pc.waves == 1 && pc.items == 3) return launch_torsion_bwd<T, 1, 3>(r, rs, x, gx, o, gs, c, B, N, st);
  if (pc.waves == 1 && pc.items == 6) return launch_torsion_bwd<T, 1, 6>(r, rs, x, gx, o, gs, c, B, N, st);
  if (pc.waves == 2) return launch_torsion_bwd<T, 2, 6>(r, rs, x, gx, o, gs, c, B, N, st);
  if (pc.items == 6) return launch_torsion_bwd<T, 4, 6>(r, rs, x, gx, o, gs, c, B, N, st);
  return launch_torsion_bwd<T, 4, 9>(r, rs, x, gx, o, gs, c, B, N, st);
}

// Shape validation shared by every entry point (extension_utils.cuh:119-130).
inline int check_chain(int64_t batch, int64_t points) {
  if (batch < 0 || batch > INT32_MAX || points > INT32_MAX) return CUFK_ERR_SHAPE;
  if (points < 4) return CUFK_ERR_POINTS;
  if (points - 3 > kMaxSteps) return CUFK_ERR_STEPS;
  return CUFK_OK;
}

inline bool valid_dtype(int dtype) { return dtype >= CUFK_FLOAT32 && dtype <= CUFK_BFLOAT16; }

inline TorsionArgs torsion_args(const cufk_torsion_consts& c) {
  TorsionArgs a;
  for (int i = 0; i < 3; ++i) {
    a.length[i] = c.length[i];
    a.sin[i] = c.sin[i];
    a.cos[i] = c.cos[i];
    a.inv_length[i] = 1.0f / c.length[i];
  }
  return a;
}

}  // namespace cufk_amd

using namespace cufk_amd;

extern "C" {

int cufk_reconstruct_fwd(int dtype, const void* lengths, const void* angles, const void* dihedrals, const void* p0,
                         const void* first_direction, const void* initial_normal, void* xyz, int64_t batch,
                         int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !xyz) return CUFK_ERR_NULL;
  const int N = static_cast<int>(points);
  auto st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case CUFK_FLOAT32: return reconstruct_fwd_typed<float>(lengths, angles, dihedrals, p0, first_direction, initial_normal, xyz, batch, N, st);
    case CUFK_FLOAT64: return reconstruct_fwd_typed<double>(lengths, angles, dihedrals, p0, first_direction, initial_normal, xyz, batch, N, st);
    case CUFK_FLOAT16: return reconstruct_fwd_typed<_Float16>(lengths, angles, dihedrals, p0, first_direction, initial_normal, xyz, batch, N, st);
    default: return reconstruct_fwd_typed<__bf16>(lengths, angles, dihedrals, p0, first_direction, initial_normal, xyz, batch, N, st);
  }
}

int cufk_reconstruct_bwd(int dtype, const void* lengths, const void* angles, const void* dihedrals, const void* p0,
                         const void* first_direction, const void* initial_normal, const void* grad_xyz,
                         void* grad_lengths, void* grad_angles, void* grad_dihedrals, int64_t batch, int64_t points,
                         void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !grad_xyz || !grad_lengths ||
      !grad_angles || !grad_dihedrals)
    return CUFK_ERR_NULL;
  const int N = static_cast<int>(points);
  auto st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case CUFK_FLOAT32: return reconstruct_bwd_typed<float>(lengths, angles, dihedrals, p0, first_direction, initial_normal, grad_xyz, grad_lengths, grad_angles, grad_dihedrals, batch, N, st);
    case CUFK_FLOAT64: return reconstruct_bwd_typed<double>(lengths, angles, dihedrals, p0, first_direction, initial_normal, grad_xyz, grad_lengths, grad_angles, grad_dihedrals, batch, N, st);
    case CUFK_FLOAT16: return reconstruct_bwd_typed<_Float16>(lengths, angles, dihedrals, p0, first_direction, initial_normal, grad_xyz, grad_lengths, grad_angles, grad_dihedrals, batch, N, st);
    default: return reconstruct_bwd_typed<__bf16>(lengths, angles, dihedrals, p0, first_direction, initial_normal, grad_xyz, grad_lengths, grad_angles, grad_dihedrals, batch, N, st);
  }
}

int cufk_torsion_fwd(int dtype, const void* raw_pairs, int64_t raw_stride, const cufk_torsion_consts* consts, void* xyz,
                     int64_t batch, int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (raw_stride < 0) return CUFK_ERR_STRIDE;
  if (!consts) return CUFK_ERR_NULL;
  if (batch == 0) return CUFK_OK;
  if (!raw_pairs || !xyz) return CUFK_ERR_NULL;
  const TorsionArgs args = torsion_args(*consts);
  const int N = static_cast<int>(points);
  auto st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case CUFK_FLOAT32: return torsion_fwd_typed<float>(raw_pairs, raw_stride, args, xyz, batch, N, st);
    case CUFK_FLOAT64: return torsion_fwd_typed<double>(raw_pairs, raw_stride, args, xyz, batch, N, st);
    case CUFK_FLOAT16: return torsion_fwd_typed<_Float16>(raw_pairs, raw_stride, args, xyz, batch, N, st);
    default: return torsion_fwd_typed<__bf16>(raw_pairs, raw_stride, args, xyz, batch, N, st);
  }
}

int cufk_torsion_bwd(int dtype, const void* raw_pairs, int64_t raw_stride, const void* xyz, const void* grad_xyz,
                     void* grad_raw, int64_t grad_raw_stride, const cufk_torsion_consts* consts, int64_t batch,
                     int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (raw_stride < 0 || grad_raw_stride < 0) return CUFK_ERR_STRIDE;
  if (!consts) return CUFK_ERR_NULL;
  if (batch == 0) return CUFK_OK;
  if (!raw_pairs || !xyz || !grad_xyz || !grad_raw) return CUFK_ERR_NULL;
  const TorsionArgs args = torsion_args(*consts);
  const int N = static_cast<int>(points);
  auto st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case CUFK_FLOAT32: return torsion_bwd_typed<float>(raw_pairs, raw_stride, xyz, grad_xyz, grad_raw, grad_raw_stride, args, batch, N, st);
    case CUFK_FLOAT64: return torsion_bwd_typed<double>(raw_pairs, raw_stride, xyz, grad_xyz, grad_raw, grad_raw_stride, args, batch, N, st);
    case CUFK_FLOAT16: return torsion_bwd_typed<_Float16>(raw_pairs, raw_stride, xyz, grad_xyz, grad_raw, grad_raw_stride, args, batch, N, st);
    default: return torsion_bwd_typed<__bf16>(raw_pairs, raw_stride, xyz, grad_xyz, grad_raw, grad_raw_stride, args, batch, N, st);
  }
}

int cufk_max_steps(int dtype, int direction, int device) {
  (void)device;
  if (!valid_dtype(dtype)) return -CUFK_ERR_DTYPE;
  if (direction != CUFK_FORWARD && direction != CUFK_BACKWARD) return -CUFK_ERR_DTYPE;
  return kMaxSteps;
}

const char* cufk_error_string(int status) {
  switch (status) {
    case CUFK_OK: return "success";
    case CUFK_ERR_DTYPE: return "unsupported dtype";
    case CUFK_ERR_POINTS: return "point_count must be >= 4";
    case CUFK_ERR_SHAPE: return "shape exceeds int32 kernel limits";
    case CUFK_ERR_STEPS: return "too many local transforms";
    case CUFK_ERR_NULL: return "null pointer argument";
    case CUFK_ERR_STRIDE: return "negative row stride";
    case CUFK_ERR_LAUNCH: return "kernel launch failed";
    case CUFK_ERR_DEVICE: return "device query failed";
    default: return "unknown status";
  }
}

const char* cufk_version(void) { return "0.1.0"; }

}  // extern "C"
