// LDS staging of chain rows.
//
// Global rows are streamed with 16-byte vector accesses (coalesced across the workgroup) into
// LDS layouts in which every lane's K steps (or K points) are contiguous, padded by Pad words
// per lane:
//   step layout:  step s        -> slot s + Pad*(s/K)              (lane stride K+Pad)
//   point layout: flat xyz e>=9 -> slot 12 + e' + Pad*(e'/(3K))    (e' = e-9, lane stride 3K+Pad)
//                 e < 9 (points 0..2) -> slot e
// Lane t owns steps [tK, tK+K) and points [3+tK, 3+tK+K).
//   Pad = 4 (K a multiple of 4): lane runs are 16-byte aligned and the strides are 4 mod 32
//     words, so ds_read_b128 / ds_write_b128 by the lanes hit disjoint banks.
//   Pad = 1: odd strides, so one 32-bit access per lane hits 64 distinct banks; every access
//     is a 32-bit one and the layout is 3/4 the size of Pad = 4 at K = 8 (more workgroups per
//     CU where LDS bounds occupancy).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "chain_ops.h"

namespace cufk_amd {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4u __attribute__((ext_vector_type(4), aligned(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
typedef double f64x2u __attribute__((ext_vector_type(2), aligned(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// A global store with the nontemporal hint, for rows that no later kernel of the step reads
// (gradients, and the half-type output whose float copy the backward reads instead): steps at
// the C4 shape 211 -> 198 us, loss 124 -> 119 us, long 180 -> 174 us, short 121 -> 118 us.
// The forward's positions stay plain: the backward that follows finds part of them in the
// last-level cache, which nontemporal stores would give up (C2: forward 48.4 -> 45 us,
// backward 49 -> 57 us).  Loads stay plain too (C2 and torsion measured slower with
// nontemporal loads), and so do the torsion backward's per-lane runs (73.6 -> 75.4 us).
template <bool Stream, typename V> __device__ __forceinline__ void global_store(V* p, V v) {
  if constexpr (Stream)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}
// The element-aligned vectors take overloads of their own: deducing V from an f32x4u* would
// drop the typedef's alignment and store through a 16-byte-aligned vector type, which rows at
// any float offset are not.
template <bool Stream> __device__ __forceinline__ void global_store(f32x4u* p, f32x4u v) {
  if constexpr (Stream)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}
template <bool Stream> __device__ __forceinline__ void global_store(f64x2u* p, f64x2u v) {
  if constexpr (Stream)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}

template <int W, int K, int Pad = 4> struct Layout {
  static_assert(K % 4 == 0, "lane segments must be whole 16-byte groups");
  static_assert(Pad == 4 || Pad == 1, "padding is 4 words (vector LDS access) or 1 word");
  static constexpr int kWaves = W;
  static constexpr int kItems = K;
  static constexpr int kPad = Pad;
  static constexpr int kLanes = 64 * W;
  static constexpr int kCap = kLanes * K;  // steps per chain
  static constexpr bool kVec = Pad == 4;    // lane runs 16-byte aligned
  static constexpr int kStepStride = K + Pad;
  static constexpr int kStepRow = kLanes * kStepStride;
  static constexpr int kPointStride = 3 * K + Pad;
  static constexpr int kPointRow = 12 + kLanes * kPointStride;
  __device__ __forceinline__ static int step_slot(int s) { return s + Pad * (s / K); }
  __device__ __forceinline__ static int point_slot(int e) {
    if (e < 9) return e;
    const int t = e - 9;
    return 12 + t + Pad * (t / (3 * K));
  }
  __device__ __forceinline__ static int lane_step_base(int tid) { return tid * kStepStride; }
  __device__ __forceinline__ static int lane_point_base(int tid) { return 12 + tid * kPointStride; }
};

// Where the elements x of a row live in LDS.  slot(x) gives one slot; run(x) gives slot(x) and
// x's offset within its lane segment (kSeg elements), from which run_slot gives the slots of
// the following elements (kStride apart, plus the layout's padding for each segment end
// crossed) without a division per element.
struct SlotRun {
  int slot;
  int off;
};
template <typename Lay> struct StepRowMap {  // step rows: element s at step_slot(s)
  static constexpr int kSeg = Lay::kItems;
  static constexpr int kStride = 1;
  static constexpr int kPad = Lay::kPad;
  __device__ __forceinline__ static int slot(int s) { return Lay::step_slot(s); }
  __device__ __forceinline__ static SlotRun run(int s) { return {Lay::step_slot(s), s % kSeg}; }
};
template <typename Lay> struct PointRowMap {  // flat (points, 3) rows, elements x >= 9
  static constexpr int kSeg = 3 * Lay::kItems;
  static constexpr int kStride = 1;
  static constexpr int kPad = Lay::kPad;
  __device__ __forceinline__ static int slot(int x) { return Lay::point_slot(x); }
  __device__ __forceinline__ static SlotRun run(int x) {
    const int t = x - 9;
    const int q = t / kSeg;
    return {12 + t + kPad * q, t - q * kSeg};
  }
};
template <typename Lay> struct StepPointMap {  // step s at the first point slot of point s+3
  static constexpr int kSeg = Lay::kItems;
  static constexpr int kStride = 3;
  static constexpr int kPad = Lay::kPad;
  __device__ __forceinline__ static int slot(int s) { return Lay::point_slot(9 + 3 * s); }
  __device__ __forceinline__ static SlotRun run(int s) { return {Lay::point_slot(9 + 3 * s), s % kSeg}; }
};
// Slot of element x + k, for r = Map::run(x) and 0 <= k < 8.
template <typename Map> __device__ __forceinline__ int run_slot(SlotRun r, int k) {
  if constexpr (Map::kSeg >= 8)  // at most one segment end within 8 elements
    return r.slot + Map::kStride * k + (r.off + k >= Map::kSeg ? Map::kPad : 0);
  else
    return r.slot + Map::kStride * k + Map::kPad * ((r.off + k) / Map::kSeg);
}

// 16-byte global access unit for T: 4 floats or 2 doubles (dword-aligned rows suffice);
// float16/bfloat16 rows are only 2-byte aligned and move in windows (below).
template <typename T> struct Unit {
  static constexpr int kElems = 1;
};
template <> struct Unit<float> {
  static constexpr int kElems = 4;
  typedef f32x4u Global;
  typedef f32x4 Local;
};
template <> struct Unit<double> {
  static constexpr int kElems = 2;
  typedef f64x2u Global;
  typedef f64x2 Local;
};

// A row of n elements that is only element-aligned splits at its 16-byte block boundaries:
// `head` elements before the first boundary, `windows` whole 16-byte windows of 16/sizeof(T)
// elements, and `tail` elements after the last boundary (head, tail < 16/sizeof(T)).  Windows
// move as one 16-byte access each, head and tail elements one per thread, so no access touches
// bytes outside the row.  float16/bfloat16 rows (2-byte aligned) always move this way.
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
struct RowSplit {
  int head;
  int windows;
  int tail;
};
template <typename T> __device__ __forceinline__ RowSplit block_split(const T* row, int n) {
  constexpr int E = 16 / sizeof(T);
  const int lead = static_cast<int>((reinterpret_cast<uintptr_t>(row) / sizeof(T)) & (E - 1));
  const int head = min((E - lead) & (E - 1), max(n, 0));
  const int windows = (max(n, 0) - head) / E;
  return {head, windows, max(n, 0) - head - E * windows};
}

// dst[e] = src[Map::slot(x0 + e)] rounded to T, for e in [0, n), by the Lanes threads of a
// workgroup (RowSplit): each window takes its slots from one Map::run.
template <int Lanes, typename Map, bool Stream = false, typename T>
__device__ __forceinline__ void store_windows(T* __restrict__ dst, const compute_t<T>* __restrict__ src, int x0, int n,
                                              int tid) {
  const RowSplit sp = block_split(dst, n);
  for (int g = tid; g < sp.windows; g += Lanes) {
    const int e0 = sp.head + 8 * g;
    const SlotRun r = Map::run(x0 + e0);
    u16x8 v;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const T x = narrow<T>(src[run_slot<Map>(r, k)]);
      v[k] = __builtin_bit_cast(unsigned short, x);
    }
    global_store<Stream>(reinterpret_cast<u16x8*>(dst + e0), v);
  }
  if (tid < sp.head) global_store<Stream>(dst + tid, narrow<T>(src[Map::slot(x0 + tid)]));
  if (tid < sp.tail) {
    const int e = n - sp.tail + tid;
    global_store<Stream>(dst + e, narrow<T>(src[Map::slot(x0 + e)]));
  }
}

// A 16-byte group of consecutive LDS slots: one vector read when the layout keeps lane runs
// 16-byte aligned, element reads otherwise.
template <typename Lay, typename V, typename S> __device__ __forceinline__ V lds_vec(const S* p) {
  if constexpr (Lay::kVec) {
    return *reinterpret_cast<const V*>(p);
  } else {
    V v;
#pragma unroll
    for (int e = 0; e < static_cast<int>(sizeof(V) / sizeof(S)); ++e) v[e] = p[e];
    return v;
  }
}

// One thread's share of NR rows moved into LDS, in two phases: fetch() issues the thread's
// global loads of src[r][first, first + n) into registers; commit() writes them to
// dst[r][Map::slot(first + e)] and returns whether any element of a row in RangeRows (bit r
// for row r) lies beyond the polynomial range of sin_cos_wide.  MaxN bounds n at compile time.
// A 16-byte group never straddles a lane segment, so its elements land in consecutive slots;
// Vec writes it with one vector LDS store (slots 16-byte aligned), otherwise element by
// element.
template <int NR, int MaxN, int Lanes, typename T, bool Half = sizeof(T) == 2> struct RowFetch {  // float, double
  using R = compute_t<T>;
  static constexpr int E = Unit<T>::kElems;
  static constexpr int kPer = (MaxN / E + Lanes - 1) / Lanes;
  typename Unit<T>::Local buf[NR][kPer];
  R tail[NR];
  int first, n, groups, te;

  __device__ __forceinline__ void fetch(const T* const (&src)[NR], int first_, int n_, int tid) {
    first = first_;
    n = n_;
    groups = n / E;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int g = tid + j * Lanes;
      if (g < groups) {
#pragma unroll
        for (int r = 0; r < NR; ++r) buf[r][j] = *reinterpret_cast<const typename Unit<T>::Global*>(src[r] + first + E * g);
      }
    }
    te = E * groups + tid;  // at most E-1 tail elements, one per low thread
    if (te < n) {
#pragma unroll
      for (int r = 0; r < NR; ++r) tail[r] = src[r][first + te];
    }
  }

  template <bool Vec, unsigned RangeRows, typename Map>
  __device__ __forceinline__ bool commit(R* const (&dst)[NR], int tid) const {
    bool wide = false;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int g = tid + j * Lanes;
      if (g < groups) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          R* const d = dst[r] + Map::slot(first + E * g);
          if constexpr (Vec) {
            *reinterpret_cast<typename Unit<T>::Local*>(d) = buf[r][j];
          } else {
#pragma unroll
            for (int e = 0; e < E; ++e) d[e] = buf[r][j][e];
          }
          if ((RangeRows >> r) & 1u) {
#pragma unroll
            for (int e = 0; e < E; ++e) wide = wide || beyond_wide_reduce(buf[r][j][e]);
          }
        }
      }
    }
    if (te < n) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        dst[r][Map::slot(first + te)] = tail[r];
        if ((RangeRows >> r) & 1u) wide = wide || beyond_wide_reduce(tail[r]);
      }
    }
    return wide;
  }
};

// float16/bfloat16 rows move in 16-byte windows (above).
template <int NR, int MaxN, int Lanes, typename T> struct RowFetch<NR, MaxN, Lanes, T, true> {
  using R = compute_t<T>;
  static constexpr int kPer = (MaxN / 8 + Lanes - 1) / Lanes;
  u16x8 buf[NR][kPer];
  T head_v[NR], tail_v[NR];  // this thread's element of the head and of the tail, if any
  RowSplit sp[NR];
  int first, n;

  __device__ __forceinline__ void fetch(const T* const (&src)[NR], int first_, int n_, int tid) {
    first = first_;
    n = n_;
#pragma unroll
    for (int r = 0; r < NR; ++r) sp[r] = block_split(src[r] + first, n);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int g = tid + j * Lanes;
#pragma unroll
      for (int r = 0; r < NR; ++r)
        if (g < sp[r].windows) buf[r][j] = *reinterpret_cast<const u16x8*>(src[r] + first + sp[r].head + 8 * g);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (tid < sp[r].head) head_v[r] = src[r][first + tid];
      if (tid < sp[r].tail) tail_v[r] = src[r][first + n - sp[r].tail + tid];
    }
  }

  template <bool Vec, unsigned RangeRows, typename Map>
  __device__ __forceinline__ bool commit(R* const (&dst)[NR], int tid) const {
    bool wide = false;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int g = tid + j * Lanes;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if (g < sp[r].windows) {
          const SlotRun run = Map::run(first + sp[r].head + 8 * g);
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            // Through a scalar: a bit cast of the vector element itself reads element 0.
            const unsigned short bits = buf[r][j][k];
            const R v = widen(__builtin_bit_cast(T, bits));
            dst[r][run_slot<Map>(run, k)] = v;
            if ((RangeRows >> r) & 1u) wide = wide || beyond_wide_reduce(v);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (tid < sp[r].head) {
        const R v = widen(head_v[r]);
        dst[r][Map::slot(first + tid)] = v;
        if ((RangeRows >> r) & 1u) wide = wide || beyond_wide_reduce(v);
      }
      if (tid < sp[r].tail) {
        const R v = widen(tail_v[r]);
        dst[r][Map::slot(first + n - sp[r].tail + tid)] = v;
        if ((RangeRows >> r) & 1u) wide = wide || beyond_wide_reduce(v);
      }
    }
    return wide;
  }
};

// Rows of NR arrays into LDS: dst[r][slot(first + e)] = src[r][first + e] for e in [0, n).
// Every global load of the thread is issued into registers before the first LDS write, so a
// workgroup pays one memory latency per staging phase, not one per group.  Returns whether
// any element this thread staged from a row in RangeRows lies beyond the polynomial range of
// sin_cos_wide (RowFetch).
template <int NR, int MaxN, int Lanes, bool Vec, typename Map, unsigned RangeRows = 0, typename T>
__device__ __forceinline__ bool stage_rows(compute_t<T>* const (&dst)[NR], const T* const (&src)[NR], int first, int n,
                                           int tid) {
  RowFetch<NR, MaxN, Lanes, T> rows;
  rows.fetch(src, first, n, tid);
  return rows.template commit<Vec, RangeRows, Map>(dst, tid);
}

// NR step rows (n <= kCap elements each) into step layouts; see stage_rows for RangeRows.
template <typename Lay, int NR, unsigned RangeRows = 0, typename T>
__device__ __forceinline__ bool load_step_rows(compute_t<T>* const (&dst)[NR], const T* const (&src)[NR], int n, int tid) {
  return stage_rows<NR, Lay::kCap, Lay::kLanes, Lay::kVec, StepRowMap<Lay>, RangeRows, T>(dst, src, 0, n, tid);
}

// NR (points, 3) rows into point layouts.
template <typename Lay, int NR, typename T>
__device__ __forceinline__ void load_point_rows(compute_t<T>* const (&dst)[NR], const T* const (&src)[NR], int points,
                                                int tid) {
  if (tid < 9) {
#pragma unroll
    for (int r = 0; r < NR; ++r) dst[r][tid] = widen(src[r][tid]);
  }
  stage_rows<NR, 3 * Lay::kCap, Lay::kLanes, Lay::kVec, PointRowMap<Lay>, 0u, T>(dst, src, 9, 3 * points - 9, tid);
}

// Two (points, 3) rows of different element types (float positions, the gradients of a
// float16/bfloat16 chain) into point layouts, both rows' global loads issued before the first
// LDS write.
template <typename Lay, typename TA, typename TB>
__device__ __forceinline__ void load_point_rows_pair(compute_t<TA>* da, const TA* __restrict__ sa, compute_t<TB>* db,
                                                     const TB* __restrict__ sb, int points, int tid) {
  if (tid < 9) {
    da[tid] = widen(sa[tid]);
    db[tid] = widen(sb[tid]);
  }
  const TA* const src_a[1] = {sa};
  const TB* const src_b[1] = {sb};
  compute_t<TA>* const dst_a[1] = {da};
  compute_t<TB>* const dst_b[1] = {db};
  RowFetch<1, 3 * Lay::kCap, Lay::kLanes, TA> a;
  RowFetch<1, 3 * Lay::kCap, Lay::kLanes, TB> b;
  a.fetch(src_a, 9, 3 * points - 9, tid);
  b.fetch(src_b, 9, 3 * points - 9, tid);
  a.template commit<Lay::kVec, 0u, PointRowMap<Lay>>(dst_a, tid);
  b.template commit<Lay::kVec, 0u, PointRowMap<Lay>>(dst_b, tid);
}

// One lane's run of n <= N consecutive elements between global memory and registers, in
// 16-byte vectors where the run allows (dword alignment suffices for float and double rows)
// and element by element for the remainder and for float16/bfloat16.
template <int N, typename T>
__device__ __forceinline__ void load_run(const T* __restrict__ src, int n, compute_t<T> (&dst)[N]) {
  constexpr int E = Unit<T>::kElems;
  if constexpr (E > 1) {
#pragma unroll
    for (int j = 0; j + E <= N; j += E) {
      if (j + E <= n) {
        const typename Unit<T>::Local v = *reinterpret_cast<const typename Unit<T>::Global*>(src + j);
#pragma unroll
        for (int e = 0; e < E; ++e) dst[j + e] = v[e];
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e)
          if (j + e < n) dst[j + e] = src[j + e];
      }
    }
  }
  constexpr int kTail = E > 1 ? (N / E) * E : 0;  // first element not covered by a vector
#pragma unroll
  for (int j = kTail; j < N; ++j)
    if (j < n) dst[j] = widen(src[j]);
}
template <int N, bool Stream = false, typename T>
__device__ __forceinline__ void store_run(T* __restrict__ dst, int n, const compute_t<T> (&src)[N]) {
  constexpr int E = Unit<T>::kElems;
  if constexpr (E > 1) {
#pragma unroll
    for (int j = 0; j + E <= N; j += E) {
      if (j + E <= n) {
        typename Unit<T>::Local v;
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = src[j + e];
        global_store<Stream>(reinterpret_cast<typename Unit<T>::Global*>(dst + j), typename Unit<T>::Global(v));
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e)
          if (j + e < n) global_store<Stream>(dst + j + e, src[j + e]);
      }
    }
  }
  constexpr int kTail = E > 1 ? (N / E) * E : 0;
#pragma unroll
  for (int j = kTail; j < N; ++j)
    if (j < n) global_store<Stream>(dst + j, narrow<T>(src[j]));
}

// dst[s] = src[step_slot(s)] for s in [0, n).
template <typename Lay, typename T>
__device__ __forceinline__ void store_step_row(T* __restrict__ dst, const compute_t<T>* __restrict__ src, int n, int tid) {
  if constexpr (std::is_same_v<T, float>) {
    const int groups = n >> 2;
    for (int g = tid; g < groups; g += Lay::kLanes)
      *reinterpret_cast<f32x4u*>(dst + 4 * g) = lds_vec<Lay, f32x4>(src + Lay::step_slot(4 * g));
    for (int s = 4 * groups + tid; s < n; s += Lay::kLanes) dst[s] = src[Lay::step_slot(s)];
  } else if constexpr (std::is_same_v<T, double>) {
    const int groups = n >> 1;
    for (int g = tid; g < groups; g += Lay::kLanes)
      *reinterpret_cast<f64x2u*>(dst + 2 * g) = lds_vec<Lay, f64x2>(src + Lay::step_slot(2 * g));
    if ((n & 1) && tid == 0) dst[n - 1] = src[Lay::step_slot(n - 1)];
  } else {
    for (int s = tid; s < n; s += Lay::kLanes) dst[s] = narrow<T>(src[Lay::step_slot(s)]);
  }
}

// dst[e] = src[point_slot(e)] for e in [0, 3*points); without `head`, points 0..2 are left alone.
template <typename Lay, bool Stream = false, typename T>
__device__ __forceinline__ void store_point_row(T* __restrict__ dst, const compute_t<T>* __restrict__ src, int points,
                                                int tid, bool head = true) {
  const int n = 3 * points - 9;
  if (head && tid < 9) global_store<Stream>(dst + tid, narrow<T>(src[tid]));
  if constexpr (std::is_same_v<T, float>) {
    const int groups = n >> 2;
    for (int g = tid; g < groups; g += Lay::kLanes)
      global_store<Stream>(reinterpret_cast<f32x4u*>(dst + 9 + 4 * g), f32x4u(lds_vec<Lay, f32x4>(src + Lay::point_slot(9 + 4 * g))));
    for (int e = 4 * groups + tid; e < n; e += Lay::kLanes) global_store<Stream>(dst + 9 + e, src[Lay::point_slot(9 + e)]);
  } else if constexpr (std::is_same_v<T, double>) {
    const int groups = n >> 1;
    for (int g = tid; g < groups; g += Lay::kLanes)
      global_store<Stream>(reinterpret_cast<f64x2u*>(dst + 9 + 2 * g), f64x2u(lds_vec<Lay, f64x2>(src + Lay::point_slot(9 + 2 * g))));
    if ((n & 1) && tid == 0) global_store<Stream>(dst + 9 + n - 1, src[Lay::point_slot(9 + n - 1)]);
  } else {
    store_windows<Lay::kLanes, PointRowMap<Lay>, Stream>(dst + 9, src, 9, n, tid);
  }
}

// Three step-indexed gradient rows written interleaved into the point layout: the outputs of
// step s (lane t, item i) occupy slots lane_point_base(t) + 3i + {0,1,2}, i.e. exactly the
// upstream-gradient slots of point s+3, which the owning lane has consumed by then.
//   a[s + offset_a] for s in [0, steps), likewise b and c.
template <typename Lay, typename T>
__device__ __forceinline__ void store_interleaved_rows(T* __restrict__ a, T* __restrict__ b, T* __restrict__ c,
                                                       const compute_t<T>* __restrict__ src, int steps, int tid) {
  if constexpr (std::is_same_v<T, float>) {
    const int groups = steps >> 2;  // 4 steps never straddle a lane (K % 4 == 0)
    for (int g = tid; g < groups; g += Lay::kLanes) {
      const float* p = src + Lay::point_slot(9 + 12 * g);
      const f32x4 v0 = lds_vec<Lay, f32x4>(p);
      const f32x4 v1 = lds_vec<Lay, f32x4>(p + 4);
      const f32x4 v2 = lds_vec<Lay, f32x4>(p + 8);
      global_store<true>(reinterpret_cast<f32x4u*>(a + 4 * g), f32x4u{v0.x, v0.w, v1.z, v2.y});
      global_store<true>(reinterpret_cast<f32x4u*>(b + 4 * g), f32x4u{v0.y, v1.x, v1.w, v2.z});
      global_store<true>(reinterpret_cast<f32x4u*>(c + 4 * g), f32x4u{v0.z, v1.y, v2.x, v2.w});
    }
    for (int s = 4 * groups + tid; s < steps; s += Lay::kLanes) {
      const float* p = src + Lay::point_slot(9 + 3 * s);
      global_store<true>(a + s, p[0]);
      global_store<true>(b + s, p[1]);
      global_store<true>(c + s, p[2]);
    }
  } else if constexpr (sizeof(T) == 2) {
    store_windows<Lay::kLanes, StepPointMap<Lay>, true>(a, src, 0, steps, tid);
    store_windows<Lay::kLanes, StepPointMap<Lay>, true>(b, src + 1, 0, steps, tid);
    store_windows<Lay::kLanes, StepPointMap<Lay>, true>(c, src + 2, 0, steps, tid);
  } else {
    for (int s = tid; s < steps; s += Lay::kLanes) {
      const compute_t<T>* p = src + Lay::point_slot(9 + 3 * s);
      global_store<true>(a + s, narrow<T>(p[0]));
      global_store<true>(b + s, narrow<T>(p[1]));
      global_store<true>(c + s, narrow<T>(p[2]));
    }
  }
}

// Same for two interleaved rows written as (x0, y0, -, x1, y1, -, ...) into point slots,
// stored to a[2s], a[2s+1] (torsion raw-pair gradients).
template <typename Lay, typename T>
__device__ __forceinline__ void store_interleaved_pairs(T* __restrict__ out, const compute_t<T>* __restrict__ src,
                                                        int steps, int tid) {
  for (int s = tid; s < steps; s += Lay::kLanes) {
    const compute_t<T>* p = src + Lay::point_slot(9 + 3 * s);
    out[2 * s] = narrow<T>(p[0]);
    out[2 * s + 1] = narrow<T>(p[1]);
  }
}

}  // namespace cufk_amd
