// Short chains, several per wave (the reference runs one chain per CTA at every length,
// block.cu:319-365; small-N packing has no counterpart there).
//
// A workgroup of W waves reconstructs C = 64W/G consecutive chains, G lanes each (G a power of
// two <= 16, so a chain's lanes sit inside one 16-lane DPP row), K steps per lane: chains of
// up to G*K steps.  Lane tid serves chain c = tid / G as its lane t = tid % G and owns that
// chain's steps [tK, tK+K).  Scans run inside each group of G lanes (DPP row_shr rounds masked
// at group starts), so no chain pays a full 64-lane scan or a workgroup barrier per scan, and
// one wave carries 64/G chains instead of one.
//
// The rows of C consecutive chains are contiguous in HBM and stay in that flat order in LDS,
// with one pad word per Gap elements (Gap = K for parameter and output rows, 3K for point
// rows) so that lanes reading their K-item runs hit distinct banks: element e of a flat range
// sits at e + e / Gap.  Rows move between HBM and LDS as 16-byte windows with no per-element
// index arithmetic beyond that slot.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "chain_ops.h"
#include "reconstruct_kernels.h"
#include "staging.h"

namespace cufk_amd {

// ---------------------------------------------------------------------------- group primitives

template <int Ctrl, int D, int G, typename R>
__device__ __forceinline__ Rigid<R> group_scan_round(const Rigid<R>& x, int t) {
  Rigid<R> y = dpp_rigid<Ctrl, 0xf>(x);  // identity where the source lies outside the row
  if constexpr (G < 16) {
    if (t < D) y = rigid_identity<R>();  // source in the previous group of the same row
  }
  return compose(y, x);
}

// Exclusive ordered product over each group of G lanes (identity in the group's first lane).
template <int G, typename R> __device__ __forceinline__ Rigid<R> group_exclusive(Rigid<R> x, int lane) {
  static_assert(G >= 1 && G <= 16 && (G & (G - 1)) == 0, "groups are powers of two inside one DPP row");
  const int t = lane & (G - 1);
  if constexpr (G == 1) {
    return rigid_identity<R>();
  } else if constexpr (std::is_same_v<R, float>) {
    // The fused DPP levels (group_prefix: 51 VALU issues and at most 12 selects per level,
    // against about 75 for the rounds below), then the shift by one lane: mov_dpp needs no
    // old value, since every lane without a source (a row start) is a group start and takes
    // the identity.
    x = group_prefix<G>(x, t);
    Rigid<R> y;
#pragma unroll
    for (int i = 0; i < 9; ++i) {
      const R v = __builtin_bit_cast(R, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x.m[i]), kRowShr1, 0xf, 0xf, true));
      y.m[i] = t == 0 ? ((i % 4 == 0) ? R(1) : R(0)) : v;
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const R v = __builtin_bit_cast(R, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x.v[i]), kRowShr1, 0xf, 0xf, true));
      y.v[i] = t == 0 ? R(0) : v;
    }
    return y;
  } else {
    x = group_scan_round<kRowShr1, 1, G>(x, t);
    if constexpr (G >= 4) x = group_scan_round<kRowShr2, 2, G>(x, t);
    if constexpr (G >= 8) x = group_scan_round<kRowShr4, 4, G>(x, t);
    if constexpr (G >= 16) x = group_scan_round<kRowShr8, 8, G>(x, t);
    // Shift by one lane inside the row (row_shr:1); a group's first lane takes the identity.
    Rigid<R> y;
#pragma unroll
    for (int i = 0; i < 9; ++i) {
      const R id = (i % 4 == 0) ? R(1) : R(0);
      const R v = dpp_move<kRowShr1, 0xf>(id, x.m[i]);
      y.m[i] = t == 0 ? id : v;
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const R v = dpp_move<kRowShr1, 0xf>(R(0), x.v[i]);
      y.v[i] = t == 0 ? R(0) : v;
    }
    return y;
  }
}

// x of lane + D inside the group (row_shl:D; groups lie inside one DPP row), else 0.
template <int D, int G, typename R> __device__ __forceinline__ R group_down(R x, int t) {
  const R y = dpp_move<0x100 + D, 0xf>(R(0), x);
  return t + D < G ? y : R(0);
}

// Exclusive suffix sum over each group (zero in the group's last lane).
template <int G, typename R> __device__ __forceinline__ ForceMoment<R> group_suffix(ForceMoment<R> a, int lane) {
  const int t = lane & (G - 1);
  auto round = [&]<int D>() {
    if constexpr (D < G) {
      a.f = {a.f.x + group_down<D, G>(a.f.x, t), a.f.y + group_down<D, G>(a.f.y, t), a.f.z + group_down<D, G>(a.f.z, t)};
      a.m = {a.m.x + group_down<D, G>(a.m.x, t), a.m.y + group_down<D, G>(a.m.y, t), a.m.z + group_down<D, G>(a.m.z, t)};
    }
  };
  round.template operator()<1>();
  round.template operator()<2>();
  round.template operator()<4>();
  round.template operator()<8>();
  ForceMoment<R> e;
  if constexpr (G == 1) {
    e = {{R(0), R(0), R(0)}, {R(0), R(0), R(0)}};
  } else {
    e.f = {group_down<1, G>(a.f.x, t), group_down<1, G>(a.f.y, t), group_down<1, G>(a.f.z, t)};
    e.m = {group_down<1, G>(a.m.x, t), group_down<1, G>(a.m.y, t), group_down<1, G>(a.m.z, t)};
  }
  return e;
}

// Reductions over each group of G lanes (aligned, G <= 16) by swizzled exchanges.
template <int G, typename V, typename Op> __device__ __forceinline__ V group_reduce(V x, Op op) {
  auto round = [&]<int D>() {
    if constexpr (D < G) x = op(x, lane_xor<D>(x));
  };
  round.template operator()<1>();
  round.template operator()<2>();
  round.template operator()<4>();
  round.template operator()<8>();
  return x;
}
template <int G> __device__ __forceinline__ bool group_all(bool p) {
  return group_reduce<G>(p ? 1 : 0, [](int a, int b) { return a & b; }) != 0;
}
template <int G, typename R> __device__ __forceinline__ R group_min(R x) {
  return group_reduce<G>(x, [](R a, R b) { return fmin(a, b); });
}
template <int G, typename R> __device__ __forceinline__ R group_max(R x) {
  return group_reduce<G>(x, [](R a, R b) { return fmax(a, b); });
}

// ---------------------------------------------------------------------------- flat staging

template <int Gap> __device__ __forceinline__ int fslot(int e) { return e + e / Gap; }
// LDS words for a flat range of n elements (plus `over` elements read past its end).
constexpr int flat_words(int n, int gap, int over = 0) { return n + over + (n + over) / gap + 1; }

// [src, src + total) moves as RowSplit: whole 16-byte windows (E = 16 / sizeof(T) elements),
// head and tail elements one per thread.  A window of E <= Gap elements crosses at most one
// segment end, so its slots follow from one division.
constexpr int flat_windows(int elems, int elem_bytes, int lanes) {
  const int e = 16 / elem_bytes;
  return ((elems + 2 * e - 2) / e + lanes - 1) / lanes;
}
// fslot<Gap>(f0 + k) for 0 <= k < 2 Gap: a shift per element for a power-of-two Gap, else from
// one division per run (q = f0 / Gap, off = f0 % Gap, unsigned so that the compiler knows
// off < Gap and drops the compare that cannot hold for a constant k).
template <int Gap> struct FlatRun {
  static constexpr bool kPow2 = (Gap & (Gap - 1)) == 0;
  int base;      // f0 for a power-of-two Gap, else fslot(f0) = f0 + q
  unsigned off;  // f0 % Gap (unused for a power-of-two Gap)
  __device__ __forceinline__ explicit FlatRun(int f0) {
    if constexpr (kPow2) {
      base = f0;
      off = 0;
    } else {
      const unsigned u = static_cast<unsigned>(f0);
      base = f0 + static_cast<int>(u / Gap);
      off = u % Gap;
    }
  }
  __device__ __forceinline__ int slot(int k) const {
    if constexpr (kPow2)
      return fslot<Gap>(base + k);
    else
      return base + k + (off + k >= Gap ? 1 : 0) + (off + k >= 2 * Gap ? 1 : 0);
  }
};

// dst[fslot<Gap>(f)] = src[f] for f in [0, total).  All of a thread's loads are issued before
// its first LDS write; MaxWin bounds the windows per thread.  Returns whether any element lies
// beyond the polynomial range of sin_cos_wide (when `range`).
template <int Lanes, int MaxWin, int Gap, typename T>
__device__ __forceinline__ bool stage_flat(compute_t<T>* dst, const T* __restrict__ src, int total, int tid,
                                           bool range) {
  using R = compute_t<T>;
  constexpr int E = 16 / sizeof(T);
  static_assert(E <= Gap, "a window crosses at most one segment end");
  const RowSplit sp = block_split(src, total);
  uint4 buf[MaxWin];
#pragma unroll
  for (int j = 0; j < MaxWin; ++j) {
    const int g = tid + j * Lanes;
    if (g < sp.windows) buf[j] = *reinterpret_cast<const uint4*>(src + sp.head + E * g);
  }
  T head_v, tail_v;
  if (tid < sp.head) head_v = src[tid];
  if (tid < sp.tail) tail_v = src[total - sp.tail + tid];
  bool wide = false;
#pragma unroll
  for (int j = 0; j < MaxWin; ++j) {
    const int g = tid + j * Lanes;
    if (g < sp.windows) {
      const FlatRun<Gap> run(sp.head + E * g);
      T v[E];
      __builtin_memcpy(v, &buf[j], 16);
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const R x = widen(v[k]);
        dst[run.slot(k)] = x;
        if (range) wide = wide || beyond_wide_reduce(x);
      }
    }
  }
  if (tid < sp.head) {
    const R x = widen(head_v);
    dst[fslot<Gap>(tid)] = x;
    if (range) wide = wide || beyond_wide_reduce(x);
  }
  if (tid < sp.tail) {
    const R x = widen(tail_v);
    dst[fslot<Gap>(total - sp.tail + tid)] = x;
    if (range) wide = wide || beyond_wide_reduce(x);
  }
  return wide;
}

// dst[f] = src[fslot<Gap>(f)] for f in [0, total); Stream as for global_store.
template <int Lanes, int Gap, bool Stream = false, typename T>
__device__ __forceinline__ void store_flat(T* __restrict__ dst, const compute_t<T>* src, int total, int tid) {
  constexpr int E = 16 / sizeof(T);
  static_assert(E <= Gap, "a window crosses at most one segment end");
  const RowSplit sp = block_split(dst, total);
  for (int g = tid; g < sp.windows; g += Lanes) {
    const int f0 = sp.head + E * g;
    const FlatRun<Gap> run(f0);
    T v[E];
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = narrow<T>(src[run.slot(k)]);
    u32x4 w;
    __builtin_memcpy(&w, v, 16);
    global_store<Stream>(reinterpret_cast<u32x4*>(dst + f0), w);
  }
  if (tid < sp.head) global_store<Stream>(dst + tid, narrow<T>(src[fslot<Gap>(tid)]));
  if (tid < sp.tail) {
    const int f = total - sp.tail + tid;
    global_store<Stream>(dst + f, narrow<T>(src[fslot<Gap>(f)]));
  }
}

template <int W, int G, int K> struct Packed {
  static constexpr int kLanes = 64 * W;
  static constexpr int kGroup = G;
  static constexpr int kChains = kLanes / G;
  static constexpr int kCap = G * K;  // steps per chain
  static constexpr int kStepGap = K;
  static constexpr int kPointGap = 3 * K;
  // One parameter or output row of kChains chains (at most kCap + 2 elements each).
  static constexpr int kStepWords = flat_words(kChains * (kCap + 2), kStepGap);
  // One point row (3 * kCap + 9 elements per chain); lanes read up to 9 elements past the
  // last chain's row, which are never used.
  static constexpr int kPointWords = flat_words(kChains * (3 * kCap + 9), kPointGap, 16);
  template <typename T> static constexpr int kStepWin = flat_windows(kChains * (kCap + 2), sizeof(T), kLanes);
  template <typename T> static constexpr int kPointWin = flat_windows(kChains * (3 * kCap + 9), sizeof(T), kLanes);
};

// Lane geometry: chain c = tid / G (of nc in this workgroup), steps [s0, s0 + count).
template <int G, int K> struct PackedLane {
  int c, s0, count;
  bool leader, live;
  __device__ __forceinline__ PackedLane(int tid, int nc, int steps) {
    c = tid / G;
    s0 = (tid & (G - 1)) * K;
    live = c < nc;
    leader = live && (tid & (G - 1)) == 0;
    count = live ? (steps - s0 < K ? steps - s0 : K) : 0;  // may be <= 0
    if (!live) c = 0;  // idle lanes read chain 0's slots and contribute nothing
  }
};

// Parameter rows of the workgroup's chains, flat: lengths (N-1 per chain), angles (N-2),
// dihedrals (N-3).
template <typename P, typename R> struct ParamRows {
  R* L;
  R* A;
  R* D;
  __device__ __forceinline__ explicit ParamRows(R* base) : L(base), A(base + P::kStepWords), D(base + 2 * P::kStepWords) {}
};

template <typename P, typename T>
__device__ __forceinline__ bool stage_params(const ParamRows<P, compute_t<T>>& rows, const T* L, const T* A, const T* D,
                                             int nc, int points, int tid) {
  bool w = stage_flat<P::kLanes, P::template kStepWin<T>, P::kStepGap>(rows.L, L, nc * (points - 1), tid, false);
  w = stage_flat<P::kLanes, P::template kStepWin<T>, P::kStepGap>(rows.A, A, nc * (points - 2), tid, true) || w;
  w = stage_flat<P::kLanes, P::template kStepWin<T>, P::kStepGap>(rows.D, D, nc * (points - 3), tid, true) || w;
  return w;
}

// Lane-serial scan in double over the lane's steps (as forward_chain's): y[i] is the
// translation of the lane-local prefix after item i.  The hot instance runs every item
// unguarded: items past the chain's last step read the next chain's slots of the flat rows (or
// the rows' unused tail: lane runs end at most kCap + 1 elements into a chain's kCap + 2 slots)
// and feed only positions that are never stored and the lane total of the chain's last lane,
// which no lane of the chain consumes; the regularity tests mask them.  The instance with the
// library sin/cos stays guarded (unguarded it needs more registers).  With Table, float angles
// take sin/cos from the LDS table (table), otherwise from sin_cos_wide.
template <typename T, typename P, int K, bool Table>
__device__ __forceinline__ void packed_serial(const ParamRows<P, compute_t<T>>& rows, const PackedLane<P::kGroup, K>& ln,
                                              int points, const SinCosEntry* table, bool wide, Rigid<double>& q,
                                              compute_t<T> (&y)[K][3], bool& ok, compute_t<T>& lmin) {
  using R = compute_t<T>;
  const int el = ln.c * (points - 1) + 2 + ln.s0;
  const int ea = ln.c * (points - 2) + 1 + ln.s0;
  const int ed = ln.c * (points - 3) + ln.s0;
  auto run = [&]<bool Checked, bool Guard>() {
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const bool in = i < ln.count;
      if (!Guard || in) {
        const R l = rows.L[fslot<P::kStepGap>(el + i)];
        double s, c, S, C;
        if constexpr (Table && sizeof(R) == 4) {
          sin_cos_tab<Checked>(rows.A[fslot<P::kStepGap>(ea + i)], table, s, c);
          sin_cos_tab<Checked>(rows.D[fslot<P::kStepGap>(ed + i)], table, S, C);
        } else {
          sin_cos_wide<Checked>(rows.A[fslot<P::kStepGap>(ea + i)], s, c);
          sin_cos_wide<Checked>(rows.D[fslot<P::kStepGap>(ed + i)], S, C);
        }
        if (i == 0)
          step_first(q.m, q.v, static_cast<double>(l), s, c, S, C);
        else
          step_forward(q.m, q.v, static_cast<double>(l), s, c, S, C);
        ok = ok && (!in || (l > R(0) && s >= FastPath<R>::kSinMin));
        lmin = in ? min_positive(lmin, l) : lmin;
      }
      y[i][0] = static_cast<R>(q.v[0]);
      y[i][1] = static_cast<R>(q.v[1]);
      y[i][2] = static_cast<R>(q.v[2]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if (wide)
    run.template operator()<true, true>();
  else
    run.template operator()<false, false>();
}

// ---------------------------------------------------------------------------- forward

// Forward for kChains chains per workgroup; regular[b] as reconstruct_forward_kernel's.
template <typename T, int W, int G, int K>
__global__ __launch_bounds__(64 * W) void packed_forward_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    T* __restrict__ xyz, uint8_t* __restrict__ regular, int64_t batch, int points) {
  using R = compute_t<T>;
  using P = Packed<W, G, K>;
  constexpr int C = P::kChains;
  constexpr int kStage = 3 * P::kStepWords > P::kPointWords ? 3 * P::kStepWords : P::kPointWords;
  __shared__ __align__(16) R stage[kStage];  // parameter rows, then the point row
  __shared__ R base[C * 12];                 // first-frame rotation (row-major) and p2
  __shared__ int wide_vote[W];
  __shared__ SinCosEntry sc_table[kSinCosTable];

  const int steps = points - 3;
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * C;
  const int nc = batch - b0 < C ? static_cast<int>(batch - b0) : C;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const PackedLane<G, K> ln(tid, nc, steps);
  const ParamRows<P, R> rows(stage);

  bool wide = stage_params<P>(rows, lengths + b0 * (points - 1), angles + b0 * (points - 2),
                              dihedrals + b0 * (points - 3), nc, points, tid);
  if constexpr (sizeof(R) == 4) sin_cos_table_init(sc_table, tid, 64 * W);
  wide = block_any<W>(wide, wide_vote, lane, wave);  // barrier: rows and table visible

  Rigid<double> q = rigid_identity<double>();
  R y[K][3];
  bool ok = true;
  R lmin = R(1.0e30);
  packed_serial<T, P, K, sizeof(R) == 4>(rows, ln, points, sc_table, wide, q, y, ok, lmin);

  // Each chain's first frame (block.cu:113-148), by its leader, after the lane scan: it is
  // then not live across the scan, and the barrier below publishes it.
  FirstFrame<R> ff;
  if (ln.leader) {
    ff = first_frame<T>(rows.L[fslot<P::kStepGap>(ln.c * (points - 1))],
                        rows.L[fslot<P::kStepGap>(ln.c * (points - 1) + 1)],
                        rows.A[fslot<P::kStepGap>(ln.c * (points - 2))], p0, first_direction, initial_normal);
#pragma unroll
    for (int i = 0; i < 9; ++i) base[ln.c * 12 + i] = ff.frame[i];
    base[ln.c * 12 + 9] = ff.p2.x;
    base[ln.c * 12 + 10] = ff.p2.y;
    base[ln.c * 12 + 11] = ff.p2.z;
  }
  const Rigid<R> excl = group_exclusive<G>(narrow_rigid<R>(q), lane);
  __syncthreads();  // base published; every read of the parameter rows retired

  R xmax = R(0);
  if (ln.count > 0) {
    R F[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) F[i] = base[ln.c * 12 + i];
    const V3<R> p2 = {base[ln.c * 12 + 9], base[ln.c * 12 + 10], base[ln.c * 12 + 11]};
    R gm[9];
#pragma unroll
    for (int r = 0; r < 3; ++r) {
#pragma unroll
      for (int cc = 0; cc < 3; ++cc)
        gm[3 * r + cc] = F[3 * r] * excl.m[cc] + F[3 * r + 1] * excl.m[3 + cc] + F[3 * r + 2] * excl.m[6 + cc];
    }
    const V3<R> gv = p2 + rot_apply(F, V3<R>{excl.v[0], excl.v[1], excl.v[2]});
    const FlatRun<P::kPointGap> run(ln.c * 3 * points + 9 + 3 * ln.s0);
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (i < ln.count) {
        // gv as the addend of the first fma: three issues per coordinate, not four.
        const V3<R> x = {fma(gm[2], y[i][2], fma(gm[1], y[i][1], fma(gm[0], y[i][0], gv.x))),
                         fma(gm[5], y[i][2], fma(gm[4], y[i][1], fma(gm[3], y[i][0], gv.y))),
                         fma(gm[8], y[i][2], fma(gm[7], y[i][1], fma(gm[6], y[i][0], gv.z)))};
        stage[run.slot(3 * i)] = x.x;
        stage[run.slot(3 * i + 1)] = x.y;
        stage[run.slot(3 * i + 2)] = x.z;
        xmax = abs_max3(xmax, x);
      }
    }
  }
  if (ln.leader) {
    const V3<R> h[3] = {ff.p0, ff.p1, ff.p2};
    const FlatRun<P::kPointGap> run(ln.c * 3 * points);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      stage[run.slot(3 * j)] = h[j].x;
      stage[run.slot(3 * j + 1)] = h[j].y;
      stage[run.slot(3 * j + 2)] = h[j].z;
    }
  }
  if constexpr (FastPath<T>::kEnabled) {
    if (regular != nullptr) {
      const bool all_ok = group_all<G>(ok);
      const R m = group_min<G>(lmin);
      const R xm = group_max<G>(xmax);
      if (ln.leader) {
        bool reg = all_ok && ff.L0 > R(0) && ff.L1 > R(0) && ff.sinA0 >= FastPath<T>::kSinMin;
        const R mm = fmin(m, fmin(ff.L0, ff.L1));
        const R x = fmax(xm, abs_max3(abs_max3(abs_max3(R(0), ff.p0), ff.p1), ff.p2));
        reg = reg && fast_extent_ok<FastPath<T>>(x, mm);
        regular[b0 + ln.c] = reg ? 1 : 0;
      }
    }
  } else {
    if (regular != nullptr && ln.leader) regular[b0 + ln.c] = 0;
  }
  __syncthreads();
  store_flat<P::kLanes, P::kPointGap>(xyz + b0 * points * 3, stage, nc * 3 * points, tid);
}

// ---------------------------------------------------------------------------- backward

// Outputs of a lane's steps, later written in output-row order.
template <typename R, int K> struct LaneGrads {
  R l[K], a[K], d[K];
  R head[3];  // dL0, dL1, dA0 (chain leaders)
};

// Position-based adjoint (position_adjoint) for one lane, positions and gradients in flat
// point rows (xs, gs).  Positions are taken relative to the chain's x2.
template <typename T, typename P, int G, int K>
__device__ __forceinline__ void packed_position_adjoint(const compute_t<T>* xs, const compute_t<T>* gs,
                                                        const PackedLane<G, K>& ln, int points, int lane,
                                                        LaneGrads<compute_t<T>, K>& out, double* anchor) {
  using R = compute_t<T>;
  const int last = ln.count - 1;
  static_assert(3 * K + 9 <= 2 * P::kPointGap, "a lane's run crosses at most two pad words");
  // Point s0: the three points before the lane's run, then the run.
  const FlatRun<P::kPointGap> run(ln.c * 3 * points + 3 * ln.s0);
  const FlatRun<P::kPointGap> chain(ln.c * 3 * points);  // the chain's points 0..2
  R xr[3 * K + 9], gr[3 * K];
#pragma unroll
  for (int i = 0; i < 3 * K + 9; ++i) xr[i] = xs[run.slot(i)];
#pragma unroll
  for (int i = 0; i < 3 * K; ++i) gr[i] = gs[run.slot(9 + i)];
  const V3<R> ctr = {xs[chain.slot(6)], xs[chain.slot(7)], xs[chain.slot(8)]};
  auto pos = [&](int j) { return V3<R>{xr[3 * j], xr[3 * j + 1], xr[3 * j + 2]} - ctr; };

  ForceMoment<R> lane_sum = {{R(0), R(0), R(0)}, {R(0), R(0), R(0)}};
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (i <= last) {
      const V3<R> g = {gr[3 * i], gr[3 * i + 1], gr[3 * i + 2]};
      lane_sum.f = lane_sum.f + g;
      lane_sum.m = lane_sum.m + cross(pos(i + 3), g);
    }
  }
  const ForceMoment<R> tail = group_suffix<G>(lane_sum, threadIdx.x & 63);

  V3<R> F = tail.f, M = tail.m;
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
      out.l[i] = dot(b1, F) * rsqrt_bond(dot(b1, b1));
      out.a[i] = dot(n, Tq) * rsqrt_bond(dot(n, n));
      out.d[i] = dot(b2, Tq) * rsqrt_bond(dot(b2, b2));
    }
  }
  if (ln.leader) {  // s0 = 0: xr holds points 0, 1, 2 first
    const V3<R> x0 = pos(0), x1 = pos(1), x2 = pos(2);
    const V3<R> g1 = {gs[chain.slot(3)], gs[chain.slot(4)], gs[chain.slot(5)]};
    const V3<R> g2 = {gs[chain.slot(6)], gs[chain.slot(7)], gs[chain.slot(8)]};
    if (anchor != nullptr) {
      const V3<R> g0 = {gs[chain.slot(0)], gs[chain.slot(1)], gs[chain.slot(2)]};
      store_anchor_sums(anchor, F, M, x0, x1, g0, g1, g2);
    }
    F = F + g2;
    const V3<R> Tq = M - cross(x1, F);
    const V3<R> b1 = x2 - x1;
    const V3<R> b0 = x1 - x0;
    const V3<R> n = cross(b1, b0);
    out.head[0] = dot(b0, F + g1) * rsqrt_bond(dot(b0, b0));
    out.head[1] = dot(b1, F) * rsqrt_bond(dot(b1, b1));
    out.head[2] = dot(n, Tq) * rsqrt_bond(dot(n, n));
  }
}

// Exact adjoint (exact_chain) for one lane: parameters in flat rows, gradients in the flat
// point row gs, the chain's first-frame rotation in base (published before the call).
template <typename T, typename P, int G, int K>
__device__ __forceinline__ void packed_exact_adjoint(const ParamRows<P, compute_t<T>>& rows, const compute_t<T>* gs,
                                                     const compute_t<T>* base, const FirstFrame<compute_t<T>>& ff,
                                                     const PackedLane<G, K>& ln, int points, bool wide,
                                                     LaneGrads<compute_t<T>, K>& out, double* anchor) {
  using R = compute_t<T>;
  const int lane = threadIdx.x & 63;
  const int el = ln.c * (points - 1) + 2 + ln.s0;
  const int ea = ln.c * (points - 2) + 1 + ln.s0;
  const int ed = ln.c * (points - 3) + ln.s0;
  const FlatRun<P::kPointGap> grun(ln.c * 3 * points + 9 + 3 * ln.s0);

  Rigid<double> qd = rigid_identity<double>();
  R Y[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) Y[i] = R(0);
  V3<R> gsum = {R(0), R(0), R(0)};
  auto pass1 = [&]<bool Checked>() {
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (i < ln.count) {
        const R l = rows.L[fslot<P::kStepGap>(el + i)];
        double s, c, S, C;
        sin_cos_wide<Checked>(rows.A[fslot<P::kStepGap>(ea + i)], s, c);
        sin_cos_wide<Checked>(rows.D[fslot<P::kStepGap>(ed + i)], S, C);
        step_forward(qd.m, qd.v, static_cast<double>(l), s, c, S, C);
        const V3<R> g = {gs[grun.slot(3 * i)], gs[grun.slot(3 * i + 1)], gs[grun.slot(3 * i + 2)]};
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
  const Rigid<R> excl = group_exclusive<G>(q, lane);
  R Fm[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) Fm[i] = base[ln.c * 12 + i];
  R R0[9];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int cc = 0; cc < 3; ++cc)
      R0[3 * r + cc] = Fm[3 * r] * excl.m[cc] + Fm[3 * r + 1] * excl.m[3 + cc] + Fm[3 * r + 2] * excl.m[6 + cc];
  }
  const V3<R> X0 = rot_apply(Fm, V3<R>{excl.v[0], excl.v[1], excl.v[2]});
  R Z[9];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int cc = 0; cc < 3; ++cc) Z[3 * r + cc] = R0[3 * r] * Y[cc] + R0[3 * r + 1] * Y[3 + cc] + R0[3 * r + 2] * Y[6 + cc];
  }
  ForceMoment<R> lane_sum;
  lane_sum.f = gsum;
  lane_sum.m = cross(X0, gsum) + V3<R>{Z[5] - Z[7], Z[6] - Z[2], Z[1] - Z[3]};
  R Rm[9];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int cc = 0; cc < 3; ++cc)
      Rm[3 * r + cc] = R0[3 * r] * q.m[cc] + R0[3 * r + 1] * q.m[3 + cc] + R0[3 * r + 2] * q.m[6 + cc];
  }
  V3<R> x = X0 + rot_apply(R0, V3<R>{q.v[0], q.v[1], q.v[2]});
  const ForceMoment<R> tail = group_suffix<G>(lane_sum, lane);

  V3<R> Fs = tail.f, Ms = tail.m;
  auto pass2 = [&]<bool Checked>() {
#pragma unroll
    for (int i = K - 1; i >= 0; --i) {
      if (i < ln.count) {
        const V3<R> g = {gs[grun.slot(3 * i)], gs[grun.slot(3 * i + 1)], gs[grun.slot(3 * i + 2)]};
        Fs = Fs + g;
        Ms = Ms + cross(x, g);
        const R l = rows.L[fslot<P::kStepGap>(el + i)];
        const V3<R> col0 = {Rm[0], Rm[3], Rm[6]};
        const V3<R> col2 = {Rm[2], Rm[5], Rm[8]};
        const V3<R> xp = x - l * col0;
        const V3<R> tau = Ms - cross(xp, Fs);
        out.l[i] = dot(col0, Fs);
        out.a[i] = -dot(col2, tau);
        double s, c, S, C;
        sin_cos_wide<Checked>(rows.A[fslot<P::kStepGap>(ea + i)], s, c);
        sin_cos_wide<Checked>(rows.D[fslot<P::kStepGap>(ed + i)], S, C);
        step_backward(Rm, static_cast<R>(s), static_cast<R>(c), static_cast<R>(S), static_cast<R>(C));
        out.d[i] = dot(V3<R>{Rm[0], Rm[3], Rm[6]}, tau);
        x = xp;
      }
    }
  };
  if (wide)
    pass2.template operator()<true>();
  else
    pass2.template operator()<false>();
  if (ln.leader) {
    const FlatRun<P::kPointGap> chain(ln.c * 3 * points);
    const V3<R> g1 = {gs[chain.slot(3)], gs[chain.slot(4)], gs[chain.slot(5)]};
    const V3<R> g2 = {gs[chain.slot(6)], gs[chain.slot(7)], gs[chain.slot(8)]};
    const V3<R> F2 = Fs + g2;
    const V3<R> x1 = ff.p1 - ff.p2;
    const V3<R> tau2 = Ms - cross(x1, F2);
    if (anchor != nullptr) {
      const V3<R> g0 = {gs[chain.slot(0)], gs[chain.slot(1)], gs[chain.slot(2)]};
      store_anchor_sums(anchor, Fs, Ms, ff.p0 - ff.p2, x1, g0, g1, g2);
    }
    out.head[0] = dot(ff.d0, F2 + g1);
    out.head[1] = dot(ff.d1, F2);
    out.head[2] = -dot(cross(ff.d0, ff.t0), tau2);
  }
}

// Backward for kChains chains per workgroup.  Saved: positions from the forward's output,
// position-based when every chain of the workgroup is flagged regular, exact otherwise.
// Without Saved (no output, or float16/bfloat16): the forward scan is rerun in registers and
// the position-based adjoint runs on those positions when every chain passes the regularity
// test of the compute type, exact otherwise.
template <typename T, int W, int G, int K, bool Saved>
__global__ __launch_bounds__(64 * W) void packed_backward_kernel(
    const T* __restrict__ lengths, const T* __restrict__ angles, const T* __restrict__ dihedrals,
    const T* __restrict__ p0, const T* __restrict__ first_direction, const T* __restrict__ initial_normal,
    const T* __restrict__ xyz, const uint8_t* __restrict__ regular, const T* __restrict__ grad_xyz,
    T* __restrict__ grad_lengths, T* __restrict__ grad_angles, T* __restrict__ grad_dihedrals, int64_t batch,
    int points, double* __restrict__ anchor = nullptr) {
  using R = compute_t<T>;
  using P = Packed<W, G, K>;
  constexpr int C = P::kChains;
  constexpr int kA = 3 * P::kStepWords > P::kPointWords ? 3 * P::kStepWords : P::kPointWords;
  __shared__ __align__(16) R region_a[kA];              // parameter rows or positions, then the outputs
  __shared__ __align__(16) R region_b[P::kPointWords];  // gradients
  __shared__ R base[C * 12];
  __shared__ int vote[W];

  const int steps = points - 3;
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * C;
  const int nc = batch - b0 < C ? static_cast<int>(batch - b0) : C;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const PackedLane<G, K> ln(tid, nc, steps);
  const ParamRows<P, R> rows(region_a);

  stage_flat<P::kLanes, P::template kPointWin<T>, P::kPointGap>(region_b, grad_xyz + b0 * points * 3, nc * 3 * points,
                                                                 tid, false);
  auto stage_rows_here = [&]() {
    return stage_params<P>(rows, lengths + b0 * (points - 1), angles + b0 * (points - 2), dihedrals + b0 * (points - 3),
                           nc, points, tid);
  };
  auto frame = [&](FirstFrame<R>& ff) {  // leaders: first frame of the chain, rotation to base
    ff = first_frame<T>(rows.L[fslot<P::kStepGap>(ln.c * (points - 1))],
                        rows.L[fslot<P::kStepGap>(ln.c * (points - 1) + 1)],
                        rows.A[fslot<P::kStepGap>(ln.c * (points - 2))], p0, first_direction, initial_normal);
#pragma unroll
    for (int i = 0; i < 9; ++i) base[ln.c * 12 + i] = ff.frame[i];
  };

  bool positions;  // every chain of the workgroup takes the position-based adjoint
  bool wide = false;
  FirstFrame<R> ff;
  if constexpr (Saved) {
    positions = !block_any<W>(ln.leader && regular[b0 + ln.c] == 0, vote, lane, wave);
    if (positions) {
      stage_flat<P::kLanes, P::template kPointWin<T>, P::kPointGap>(region_a, xyz + b0 * points * 3, nc * 3 * points,
                                                                     tid, false);
    } else {
      wide = block_any<W>(stage_rows_here(), vote, lane, wave);
      if (ln.leader) frame(ff);
    }
  } else {
    // Rerun the forward scan, positions relative to each chain's x2 (recompute_chain's).
    using Fast = FastPath<R>;
    wide = block_any<W>(stage_rows_here(), vote, lane, wave);
    if (ln.leader) frame(ff);
    Rigid<double> q = rigid_identity<double>();
    R y[K][3];
    bool ok = true;
    R lmin = R(1.0e30);
    packed_serial<T, P, K, false>(rows, ln, points, nullptr, wide, q, y, ok, lmin);
    const Rigid<R> excl = group_exclusive<G>(narrow_rigid<R>(q), lane);
    __syncthreads();  // base published
    R Fm[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) Fm[i] = base[ln.c * 12 + i];
    R R0[9];
#pragma unroll
    for (int r = 0; r < 3; ++r) {
#pragma unroll
      for (int cc = 0; cc < 3; ++cc)
        R0[3 * r + cc] = Fm[3 * r] * excl.m[cc] + Fm[3 * r + 1] * excl.m[3 + cc] + Fm[3 * r + 2] * excl.m[6 + cc];
    }
    const V3<R> X0 = rot_apply(Fm, V3<R>{excl.v[0], excl.v[1], excl.v[2]});
    V3<R> x[K];
    R xmax = R(0);
#pragma unroll
    for (int i = 0; i < K; ++i) {
      x[i] = X0 + rot_apply(R0, V3<R>{y[i][0], y[i][1], y[i][2]});
      if (i < ln.count) xmax = abs_max3(xmax, x[i]);
    }
    const bool all_ok = group_all<G>(ok);
    const R m = group_min<G>(lmin);
    const R xm = group_max<G>(xmax);
    bool irregular = false;
    if (ln.leader) {
      const V3<R> a = ff.p0 - ff.p2, bb = ff.p1 - ff.p2;
      const bool reg = all_ok && ff.L0 > R(0) && ff.L1 > R(0) && ff.sinA0 >= static_cast<R>(Fast::kSinMin);
      const R mm = fmin(m, fmin(ff.L0, ff.L1));
      const R xx = fmax(xm, abs_max3(abs_max3(R(0), a), bb));
      irregular = !(reg && fast_extent_ok<Fast>(xx, mm));
    }
    positions = !block_any<W>(irregular, vote, lane, wave);  // barrier: parameter reads retired
    if (positions) {
      if (ln.count > 0) {
        const FlatRun<P::kPointGap> run(ln.c * 3 * points + 9 + 3 * ln.s0);
#pragma unroll
        for (int i = 0; i < K; ++i) {
          if (i < ln.count) {
            region_a[run.slot(3 * i)] = x[i].x;
            region_a[run.slot(3 * i + 1)] = x[i].y;
            region_a[run.slot(3 * i + 2)] = x[i].z;
          }
        }
      }
      if (ln.leader) {
        const V3<R> h[3] = {ff.p0 - ff.p2, ff.p1 - ff.p2, {R(0), R(0), R(0)}};
        const FlatRun<P::kPointGap> run(ln.c * 3 * points);
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          region_a[run.slot(3 * j)] = h[j].x;
          region_a[run.slot(3 * j + 1)] = h[j].y;
          region_a[run.slot(3 * j + 2)] = h[j].z;
        }
      }
    }
  }
  __syncthreads();  // staged rows (and positions, base) visible
  LaneGrads<R, K> out;
  double* const an = anchor != nullptr && ln.leader ? anchor + (b0 + ln.c) * 6 : nullptr;
  if (positions)
    packed_position_adjoint<T, P, G, K>(region_a, region_b, ln, points, lane, out, an);
  else
    packed_exact_adjoint<T, P, G, K>(rows, region_b, base, ff, ln, points, wide, out, an);
  __syncthreads();  // every read of region_a retired: the outputs replace it

  // Outputs in output-row order: lengths (N-1 per chain), angles (N-2), dihedrals (N-3).
  R* ol = region_a;
  R* oa = region_a + P::kStepWords;
  R* od = region_a + 2 * P::kStepWords;
  {
    const int el = ln.c * (points - 1) + 2 + ln.s0;
    const int ea = ln.c * (points - 2) + 1 + ln.s0;
    const int ed = ln.c * (points - 3) + ln.s0;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (i < ln.count) {
        ol[fslot<P::kStepGap>(el + i)] = out.l[i];
        oa[fslot<P::kStepGap>(ea + i)] = out.a[i];
        od[fslot<P::kStepGap>(ed + i)] = out.d[i];
      }
    }
    if (ln.leader) {
      ol[fslot<P::kStepGap>(ln.c * (points - 1))] = out.head[0];
      ol[fslot<P::kStepGap>(ln.c * (points - 1) + 1)] = out.head[1];
      oa[fslot<P::kStepGap>(ln.c * (points - 2))] = out.head[2];
    }
  }
  __syncthreads();
  store_flat<P::kLanes, P::kStepGap, true>(grad_lengths + b0 * (points - 1), ol, nc * (points - 1), tid);
  store_flat<P::kLanes, P::kStepGap, true>(grad_angles + b0 * (points - 2), oa, nc * (points - 2), tid);
  store_flat<P::kLanes, P::kStepGap, true>(grad_dihedrals + b0 * (points - 3), od, nc * (points - 3), tid);
}

}  // namespace cufk_amd
