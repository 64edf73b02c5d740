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

// Where the elements x of a row live in LDS: slot(x) for the row's elements (x >= 9 for point
// rows), consecutive elements kStride slots apart within a lane segment of kSeg elements.
template <typename Lay> struct StepRowMap {  // step rows: element s at step_slot(s)
  static constexpr int kSeg = Lay::kItems;
  static constexpr int kStride = 1;
  __device__ __forceinline__ static int slot(int s) { return Lay::step_slot(s); }
};
template <typename Lay> struct PointRowMap {  // flat (points, 3) rows, elements x >= 9
  static constexpr int kSeg = 3 * Lay::kItems;
  static constexpr int kStride = 1;
  __device__ __forceinline__ static int slot(int x) {
    const int t = x - 9;
    return 12 + t + Lay::kPad * (t / kSeg);
  }
};
template <typename Lay> struct StepPointMap {  // step s at the first point slot of point s+3
  static constexpr int kSeg = Lay::kItems;
  static constexpr int kStride = 3;
  __device__ __forceinline__ static int slot(int s) { return 12 + 3 * s + Lay::kPad * (s / kSeg); }
};

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
// bytes outside the row (the packed kernels' flat rows).
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
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

// float16/bfloat16 rows through a slot map move in windows of V = half_window<Map>()
// consecutive elements, V the largest of 8 and 4 that divides the map's lane segment.  Window g
// covers the elements x0 + V*g .. x0 + V*g + V-1 with x0 the map's first element (a segment
// start), so it lies inside one lane segment and its slots are Map::slot(x0 + V*g) +
// kStride*k: no per-element slot arithmetic.  A window is one 2V-byte global access at the
// row's own 2-byte alignment, which gfx950 serves as it stands (its global accesses need no
// alignment, and hipcc itself emits them for 2-byte-aligned vectors); the n mod V elements past
// the last whole window move one per thread.  No access touches bytes outside the row.
// 16-byte-aligned windows, which straddle lane segments, cost 4 VALU per element for the slot
// alone: at the C4 shape (bfloat16, B = 16384, N = 1026) the forward took 114.5 us against
// 99.3 us in these windows, the backward 92.8 against 85.1 us.
typedef unsigned short u16x8u __attribute__((ext_vector_type(8), aligned(2)));
typedef unsigned short u16x4u __attribute__((ext_vector_type(4), aligned(2)));
template <typename Map> constexpr int half_window() {
  static_assert(Map::kSeg % 4 == 0, "lane segments hold whole 4-element windows");
  return Map::kSeg % 8 == 0 ? 8 : 4;
}
template <int V> struct HalfWindow;
template <> struct HalfWindow<8> {
  typedef u16x8u Global;
  typedef u16x8 Local;
};
template <> struct HalfWindow<4> {
  typedef u16x4u Global;
  typedef u16x4 Local;
};
template <int V> struct HalfPairs {  // a window's V/2 dwords as pairs of 16-bit lanes
  u16x2 p[V / 2];
};
// Overloads of their own, like f32x4u's: deduction would drop the 2-byte alignment.
template <bool Stream> __device__ __forceinline__ void global_store(u16x8u* p, u16x8u v) {
  if constexpr (Stream)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}
template <bool Stream> __device__ __forceinline__ void global_store(u16x4u* p, u16x4u v) {
  if constexpr (Stream)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}

// dst[e] = src[Map::slot(x0 + e)] rounded to T, for e in [0, n), by the Lanes threads of a
// workgroup, in the windows above (x0 the map's first element).
template <int Lanes, typename Map, bool Stream = false, typename T>
__device__ __forceinline__ void store_windows(T* __restrict__ dst, const compute_t<T>* __restrict__ src, int x0, int n,
                                              int tid) {
  constexpr int V = half_window<Map>();
  using Win = HalfWindow<V>;
  const int windows = n / V;
  for (int g = tid; g < windows; g += Lanes) {
    const compute_t<T>* const p = src + Map::slot(x0 + V * g);
    typename Win::Local v;
#pragma unroll
    for (int k = 0; k < V; ++k) v[k] = __builtin_bit_cast(unsigned short, narrow<T>(p[Map::kStride * k]));
    global_store<Stream>(reinterpret_cast<typename Win::Global*>(dst + V * g), typename Win::Global(v));
  }
  const int e = V * windows + tid;
  if (e < n) global_store<Stream>(dst + e, narrow<T>(src[Map::slot(x0 + e)]));
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
template <int NR, int MaxN, int Lanes, typename T, typename Map, bool Half = sizeof(T) == 2>
struct RowFetch {  // float, double
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

  template <bool Vec, unsigned RangeRows>
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

// float16/bfloat16 rows move in the windows of store_windows (first the map's first element).
// The range test runs on the bit patterns: the magnitude bits of a float16/bfloat16 order like
// the magnitudes, so one compare of the window's largest against the largest magnitude within
// kWideReduceMax (bfloat16 0x4780 = 65536; float16 0x7bff = 65504, its largest finite value)
// replaces one per element.  NaN patterns count as beyond, which changes nothing: the checked
// sin/cos form gives NaN the unchecked form's result.
template <typename T> inline constexpr unsigned short kWideReduceBits = 0;
template <> inline constexpr unsigned short kWideReduceBits<__bf16> = 0x4780;
template <> inline constexpr unsigned short kWideReduceBits<_Float16> = 0x7bff;

template <int NR, int MaxN, int Lanes, typename T, typename Map> struct RowFetch<NR, MaxN, Lanes, T, Map, true> {
  using R = compute_t<T>;
  static constexpr int V = half_window<Map>();
  using Win = HalfWindow<V>;
  static constexpr int kPer = (MaxN / V + Lanes - 1) / Lanes;
  typename Win::Local buf[NR][kPer];
  T tail_v[NR];  // this thread's element past the last whole window, if any
  int first, n, windows, te;

  __device__ __forceinline__ void fetch(const T* const (&src)[NR], int first_, int n_, int tid) {
    first = first_;
    n = n_;
    windows = n / V;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int g = tid + j * Lanes;
      if (g < windows) {
#pragma unroll
        for (int r = 0; r < NR; ++r) buf[r][j] = *reinterpret_cast<const typename Win::Global*>(src[r] + first + V * g);
      }
    }
    te = V * windows + tid;
    if (te < n) {
#pragma unroll
      for (int r = 0; r < NR; ++r) tail_v[r] = src[r][first + te];
    }
  }

  template <bool Vec, unsigned RangeRows>
  __device__ __forceinline__ bool commit(R* const (&dst)[NR], int tid) const {
    // Largest magnitude patterns staged from the rows in RangeRows, two lanes of 16 bits: the
    // windows' dwords are masked and maximised whole (v_pk_max_u16).
    u16x2 mag = {0, 0};
    constexpr u16x2 kMagnitude = {0x7fff, 0x7fff};
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int g = tid + j * Lanes;
      if (g < windows) {
        const int s = Map::slot(first + V * g);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
#pragma unroll
          for (int k = 0; k < V; ++k) {
            // Through a scalar: a bit cast of the vector element itself reads element 0.
            const unsigned short bits = buf[r][j][k];
            dst[r][s + Map::kStride * k] = widen(__builtin_bit_cast(T, bits));
          }
          if ((RangeRows >> r) & 1u) {
            const HalfPairs<V> w = __builtin_bit_cast(HalfPairs<V>, buf[r][j]);
#pragma unroll
            for (int d = 0; d < V / 2; ++d) mag = __builtin_elementwise_max(mag, w.p[d] & kMagnitude);
          }
        }
      }
    }
    if (te < n) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        dst[r][Map::slot(first + te)] = widen(tail_v[r]);
        if ((RangeRows >> r) & 1u)
          mag = __builtin_elementwise_max(mag, u16x2{__builtin_bit_cast(unsigned short, tail_v[r]), 0} & kMagnitude);
      }
    }
    return max(mag.x, mag.y) > kWideReduceBits<T>;
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
  RowFetch<NR, MaxN, Lanes, T, Map> rows;
  rows.fetch(src, first, n, tid);
  return rows.template commit<Vec, RangeRows>(dst, tid);
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
  RowFetch<1, 3 * Lay::kCap, Lay::kLanes, TA, PointRowMap<Lay>> a;
  RowFetch<1, 3 * Lay::kCap, Lay::kLanes, TB, PointRowMap<Lay>> b;
  a.fetch(src_a, 9, 3 * points - 9, tid);
  b.fetch(src_b, 9, 3 * points - 9, tid);
  a.template commit<Lay::kVec, 0u>(dst_a, tid);
  b.template commit<Lay::kVec, 0u>(dst_b, tid);
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
