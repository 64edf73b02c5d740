// Typed kernel launchers: launch plans, grid chunking and the launches themselves.
//
// This file is compiled once per (dtype, kernel family), selected by two macros:
//   CUFK_DTYPE   a cufk_dtype code (include/cufk_hip.h);
//   CUFK_FAMILY  one of the CUFK_FAMILY_* values below.
// Each unit instantiates only its family's launchers for its dtype, so only those kernels are
// compiled into it, and the units build in parallel (cufk_amd/_build.py).  The C ABI
// (cufk_hip.hip) calls the launchers through their declarations in launch.h.
//
// One workgroup of W wave64s reconstructs one chain; lane t owns the K consecutive steps
// [tK, tK+K) (blocked arrangement, as in the reference block.cu:187), runs them as a serial
// scan in registers and only lane totals cross lanes (wave64 DPP scan, then an LDS carry across
// waves).  Rows move between HBM and LDS as coalesced 16-byte streams.
#include "launch.h"

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "chain_ops.h"
#include "reconstruct_kernels.h"
#include "staging.h"
#include "torsion_kernels.h"

#define CUFK_FAMILY_FORWARD 0
#define CUFK_FAMILY_RECOMPUTE 1
#define CUFK_FAMILY_SAVED 2
#define CUFK_FAMILY_PACKED 3
#define CUFK_FAMILY_LOSS 4
#define CUFK_FAMILY_LONG 5
#define CUFK_FAMILY_TORSION 6

#if !defined(CUFK_DTYPE) || !defined(CUFK_FAMILY)
#error "compile launchers.hip with -DCUFK_DTYPE=<cufk_dtype> -DCUFK_FAMILY=<CUFK_FAMILY_*>"
#endif

#if CUFK_DTYPE == 0
#define CUFK_T float
#elif CUFK_DTYPE == 1
#define CUFK_T double
#elif CUFK_DTYPE == 2
#define CUFK_T _Float16
#elif CUFK_DTYPE == 3
#define CUFK_T __bf16
#else
#error "unknown CUFK_DTYPE"
#endif
// float32 and float64 keep the position-based backward over the saved output; float16 and
// bfloat16 outputs are too coarse for it (FastPath<T>::kEnabled), and take it over a float
// copy of their positions instead (shadow_*_typed).
#define CUFK_SAVED_BACKWARD (CUFK_DTYPE == 0 || CUFK_DTYPE == 1)

// Explicit instantiation of one launcher, its signature taken from its declaration.
#define CUFK_INSTANTIATE(...) template decltype(__VA_ARGS__) __VA_ARGS__;

namespace cufk_amd {

// ---------------------------------------------------------------------------- plans

// (waves W, items per lane K), capacity 64*W*K steps; the smallest plan holding the chain.
// Eight items per lane measured fastest at N = 2049 for both the forward and the
// position-based backward (K = 16 runs out of registers and waves, K = 4 pays the lane scan
// on too few items).  The exact backward uses the same plans.  The kernels stage rows with one
// word of padding per lane: at (4, 8) that lets five forward workgroups (three backward)
// share a CU instead of four (two).
//
// Small grids (`groups` workgroups of one chain each, at most kLatencyWaves waves under the
// eight-item plan, four per SIMD) run latency-bound: a lone wave per SIMD waits on every
// dependent instruction.  There the chain takes twice the waves with four items per lane,
// halving each lane's serial scan.  Measured on MI355X (forward + position-based backward,
// back-to-back launches): B=1024, N=384: 13.6 against 15.1 us; B=512, N=384: 11.4 against
// 12.5 us; B=2048, N=700: 30.1 against 33.2 us.
constexpr int kScanPad = 1;
constexpr int64_t kLatencyWaves = 4096;
//
// Every plan gives each of its waves some of the chain's steps (a wave past the chain would still
// run the lane scan, lane_scan_chain): where four waves of four or eight steps would leave the
// last one idle (513-768 and 1025-1536 steps), the chain takes three.
template <typename Fn> int with_scan_plan(int64_t groups, int steps, Fn&& fn) {
  if (steps <= 256) return fn.template operator()<1, 4>();
  if (steps <= 512) {
    if (groups <= kLatencyWaves) return fn.template operator()<2, 4>();
    return fn.template operator()<1, 8>();
  }
  if (steps <= 1024) {
    if (2 * groups <= kLatencyWaves) {
      if (steps <= 768) return fn.template operator()<3, 4>();
      return fn.template operator()<4, 4>();
    }
    return fn.template operator()<2, 8>();
  }
  if (steps <= 1536) return fn.template operator()<3, 8>();
  return fn.template operator()<4, 8>();
}

// Torsion plans: K a multiple of 12.
template <typename Fn> int with_torsion_plan(int steps, Fn&& fn) {
  if (steps <= 768) return fn.template operator()<1, 12>();
  if (steps <= 1536) return fn.template operator()<2, 12>();
  return fn.template operator()<3, 12>();
}

// Torsion backward plans: three steps per lane (no LDS staging, see torsion_backward_kernel).
template <typename Fn> int with_torsion_bwd_plan(int steps, Fn&& fn) {
  if (steps <= 192) return fn.template operator()<1, 3>();
  if (steps <= 384) return fn.template operator()<2, 3>();
  if (steps <= 768) return fn.template operator()<4, 3>();
  if (steps <= 1536) return fn.template operator()<8, 3>();
  return fn.template operator()<11, 3>();
}

// HIP's grid x extent counts work-items in 32 bits: launch one-chain-per-workgroup kernels
// in chunks of at most UINT32_MAX / threads workgroups.
template <typename Fn> int launch_chunks(int64_t batch, int threads, Fn&& fn) {
  const int64_t chunk = int64_t{UINT32_MAX} / threads;
  for (int64_t done = 0; done < batch; done += chunk) {
    const int64_t n = batch - done < chunk ? batch - done : chunk;
    fn(done, static_cast<unsigned>(n));
    if (hipGetLastError() != hipSuccess) return CUFK_ERR_LAUNCH;
  }
  return CUFK_OK;
}

// Packed plans (launch.h: when the packed kernels run): 64W/G chains per workgroup of
// kPackedWaves waves.
constexpr int kPackedWaves = 2;
template <int MaxG = 16, typename Fn> int with_packed_plan(int steps, Fn&& fn) {
  if (steps <= 8) return fn.template operator()<1>();
  if (steps <= 16) return fn.template operator()<2>();
  if (steps <= 32) return fn.template operator()<4>();
  if (MaxG == 8 || steps <= 64) return fn.template operator()<8>();
  if constexpr (MaxG >= 16) return fn.template operator()<16>();
  return CUFK_ERR_STEPS;
}
// Launch a packed kernel over B chains, C per workgroup, in grid chunks that keep the grid's
// work-item count within 32 bits.
template <typename Fn> int launch_packed(int64_t B, int C, Fn&& fn) {
  const int64_t threads = 64 * kPackedWaves;
  const int64_t chunk = (int64_t{UINT32_MAX} / threads) * C;
  for (int64_t done = 0; done < B; done += chunk) {
    const int64_t n = B - done < chunk ? B - done : chunk;
    fn(done, n, static_cast<unsigned>((n + C - 1) / C));
    if (hipGetLastError() != hipSuccess) return CUFK_ERR_LAUNCH;
  }
  return CUFK_OK;
}

// The superposed losses' second launch: one thread per chain solves its record.
template <typename T> int solve_records(double* record, T* loss, int64_t B, int N, int squared, hipStream_t st) {
  const int64_t groups = (B + kSolveThreads - 1) / kSolveThreads;
  for (int64_t done = 0; done < groups; done += INT32_MAX) {
    const int64_t g = groups - done < INT32_MAX ? groups - done : INT32_MAX;
    const int64_t off = done * kSolveThreads;
    hipLaunchKernelGGL(superpose_records_kernel<T>, dim3(static_cast<unsigned>(g)), dim3(kSolveThreads), 0, st,
                       record + off * kSuperposeRecord, loss + off, B - off, N, squared);
    if (hipGetLastError() != hipSuccess) return CUFK_ERR_LAUNCH;
  }
  return CUFK_OK;
}

}  // namespace cufk_amd

#if CUFK_FAMILY == CUFK_FAMILY_FORWARD
namespace cufk_amd {

template <typename T>
int reconstruct_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz,
                          uint8_t* regular, int64_t B, int N, hipStream_t st) {
  if (use_packed_fwd(B, N - 3)) return packed_fwd_typed<T>(L, A, D, p0, fd, n0, xyz, regular, B, N, st);
  return with_scan_plan(B, N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((reconstruct_forward_kernel<T, W, K, kScanPad>), dim3(n), dim3(64 * W), 0, st, L + off * (N - 1),
                         A + off * (N - 2), D + off * (N - 3), p0, fd, n0, xyz + off * N * 3,
                         regular ? regular + off : nullptr, N);
    });
  });
}

template <typename T>
int shadow_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz, float* pos,
                     uint8_t* regular, int64_t B, int N, hipStream_t st) {
  if (!use_shadow(B, N - 3)) return reconstruct_fwd_typed<T>(L, A, D, p0, fd, n0, xyz, nullptr, B, N, st);
  return with_scan_plan(B, N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((reconstruct_forward_shadow_kernel<T, W, K, kScanPad>), dim3(n), dim3(64 * W), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, xyz + off * N * 3,
                         pos + off * N * 3, regular + off, N);
    });
  });
}

CUFK_INSTANTIATE(reconstruct_fwd_typed<CUFK_T>)
#if !CUFK_SAVED_BACKWARD
CUFK_INSTANTIATE(shadow_fwd_typed<CUFK_T>)
#endif

}  // namespace cufk_amd
#endif

#if CUFK_FAMILY == CUFK_FAMILY_RECOMPUTE
namespace cufk_amd {

template <typename T>
int reconstruct_bwd_recompute_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0,
                                    const T* g, T* gL, T* gA, T* gD, int64_t B, int N, hipStream_t st,
                                    double* anchor) {
  if (use_packed_bwd(B, N - 3))
    return packed_bwd_typed<T, false>(L, A, D, p0, fd, n0, nullptr, nullptr, g, gL, gA, gD, B, N, st, anchor);
  return with_scan_plan(B, N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((reconstruct_backward_recompute_kernel<T, W, K, kScanPad>), dim3(n), dim3(64 * W), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, g + off * N * 3,
                         gL + off * (N - 1), gA + off * (N - 2), gD + off * (N - 3), N,
                         anchor != nullptr ? anchor + off * 6 : nullptr);
    });
  });
}

CUFK_INSTANTIATE(reconstruct_bwd_recompute_typed<CUFK_T>)

}  // namespace cufk_amd
#endif

#if CUFK_FAMILY == CUFK_FAMILY_SAVED
namespace cufk_amd {

template <typename T>
int reconstruct_bwd_saved_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0,
                                const T* xyz, const uint8_t* regular, const T* g, T* gL, T* gA, T* gD, int64_t B, int N,
                                hipStream_t st, double* anchor) {
  if (use_packed_bwd(B, N - 3))
    return packed_bwd_typed<T, true>(L, A, D, p0, fd, n0, xyz, regular, g, gL, gA, gD, B, N, st, anchor);
  return with_scan_plan(B, N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 2 * 64 * W, [&](int64_t off, unsigned n) {  // room for the front workgroups
      const unsigned grid = n + static_cast<unsigned>(front_groups(n));
      hipLaunchKernelGGL((reconstruct_backward_saved_kernel<T, W, K, kScanPad>), dim3(grid), dim3(64 * W), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, xyz + off * N * 3,
                         regular + off, g + off * N * 3, gL + off * (N - 1), gA + off * (N - 2), gD + off * (N - 3), N,
                         int64_t{n}, anchor != nullptr ? anchor + off * 6 : nullptr);
    });
  });
}

template <typename T>
int shadow_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const float* pos,
                     const uint8_t* regular, const T* g, T* gL, T* gA, T* gD, int64_t B, int N, hipStream_t st) {
  if (!use_shadow(B, N - 3)) return reconstruct_bwd_recompute_typed<T>(L, A, D, p0, fd, n0, g, gL, gA, gD, B, N, st);
  return with_scan_plan(B, N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 2 * 64 * W, [&](int64_t off, unsigned n) {  // room for the front workgroups
      const unsigned grid = n + static_cast<unsigned>(front_groups(n));
      hipLaunchKernelGGL((reconstruct_backward_saved_kernel<T, W, K, kScanPad, float>), dim3(grid), dim3(64 * W), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, pos + off * N * 3,
                         regular + off, g + off * N * 3, gL + off * (N - 1), gA + off * (N - 2), gD + off * (N - 3), N,
                         int64_t{n}, nullptr);
    });
  });
}

template <typename T>
int anchor_grads_typed(const double* anchor, int64_t B, const T* fd, const T* n0, T* grad_p0, T* grad_fd, T* grad_n0,
                       hipStream_t st) {
  hipLaunchKernelGGL(anchor_gradients_kernel<T>, dim3(1), dim3(kAnchorThreads), 0, st, anchor, B, fd, n0, grad_p0,
                     grad_fd, grad_n0);
  return hipGetLastError() == hipSuccess ? CUFK_OK : CUFK_ERR_LAUNCH;
}

#if CUFK_SAVED_BACKWARD
CUFK_INSTANTIATE(reconstruct_bwd_saved_typed<CUFK_T>)
#else
CUFK_INSTANTIATE(shadow_bwd_typed<CUFK_T>)
#endif
CUFK_INSTANTIATE(anchor_grads_typed<CUFK_T>)

}  // namespace cufk_amd
#endif

#if CUFK_FAMILY == CUFK_FAMILY_PACKED
#include "packed_kernels.h"
namespace cufk_amd {

template <typename T>
int packed_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz,
                     uint8_t* regular, int64_t B, int N, hipStream_t st) {
  return with_packed_plan(N - 3, [&]<int G>() {
    constexpr int C = 64 * kPackedWaves / G;
    return launch_packed(B, C, [&](int64_t off, int64_t n, unsigned groups) {
      hipLaunchKernelGGL((packed_forward_kernel<T, kPackedWaves, G, 8>), dim3(groups), dim3(64 * kPackedWaves), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, xyz + off * N * 3,
                         regular ? regular + off : nullptr, n, N);
    });
  });
}

template <typename T, bool Saved>
int packed_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* xyz,
                     const uint8_t* regular, const T* g, T* gL, T* gA, T* gD, int64_t B, int N, hipStream_t st,
                     double* anchor) {
  static_assert(kPackedBwdMaxSteps <= 64, "the packed backward is compiled for up to 8 lanes per chain");
  return with_packed_plan<8>(N - 3, [&]<int G>() {
    constexpr int C = 64 * kPackedWaves / G;
    return launch_packed(B, C, [&](int64_t off, int64_t n, unsigned groups) {
      hipLaunchKernelGGL((packed_backward_kernel<T, kPackedWaves, G, 8, Saved>), dim3(groups), dim3(64 * kPackedWaves),
                         0, st, L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0,
                         Saved ? xyz + off * N * 3 : nullptr, Saved ? regular + off : nullptr, g + off * N * 3,
                         gL + off * (N - 1), gA + off * (N - 2), gD + off * (N - 3), n, N,
                         anchor != nullptr ? anchor + off * 6 : nullptr);
    });
  });
}

CUFK_INSTANTIATE(packed_fwd_typed<CUFK_T>)
CUFK_INSTANTIATE(packed_bwd_typed<CUFK_T, false>)
#if CUFK_SAVED_BACKWARD
CUFK_INSTANTIATE(packed_bwd_typed<CUFK_T, true>)
#endif

}  // namespace cufk_amd
#endif

#if CUFK_FAMILY == CUFK_FAMILY_LOSS
namespace cufk_amd {

template <typename T>
int loss_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* target, T* xyz,
                   uint8_t* regular, T* loss, int64_t B, int N, hipStream_t st) {
  return with_scan_plan(B, N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((reconstruct_loss_forward_kernel<T, W, K, kScanPad>), dim3(n), dim3(64 * W), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, target + off * N * 3,
                         xyz + off * N * 3, regular + off, loss + off, N);
    });
  });
}

template <typename T>
int loss_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* xyz,
                   const uint8_t* regular, const T* target, const T* grad_loss, T* gL, T* gA, T* gD, int64_t B, int N,
                   hipStream_t st, double* anchor) {
  return with_scan_plan(B, N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 2 * 64 * W, [&](int64_t off, unsigned n) {  // room for the front workgroups
      const unsigned grid = FastPath<T>::kEnabled ? n + static_cast<unsigned>(front_groups(n)) : n;
      hipLaunchKernelGGL((reconstruct_loss_backward_kernel<T, W, K, kScanPad>), dim3(grid), dim3(64 * W), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, xyz + off * N * 3,
                         regular + off, target + off * N * 3, grad_loss != nullptr ? grad_loss + off : nullptr,
                         gL + off * (N - 1), gA + off * (N - 2), gD + off * (N - 3), N, int64_t{n}, nullptr, 0,
                         anchor != nullptr ? anchor + off * 6 : nullptr);
    });
  });
}

template <typename T>
int superposed_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* target,
                         T* xyz, uint8_t* regular, T* loss, double* record, int squared, int64_t B, int N,
                         hipStream_t st) {
  const int rc = with_scan_plan(B, N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((reconstruct_superposed_forward_kernel<T, W, K, kScanPad>), dim3(n), dim3(64 * W), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, target + off * N * 3,
                         xyz + off * N * 3, regular + off, record + off * kSuperposeRecord, N);
    });
  });
  if (rc != CUFK_OK) return rc;
  return solve_records<T>(record, loss, B, N, squared, st);
}

template <typename T>
int superposed_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* xyz,
                         const uint8_t* regular, const T* target, const double* record, const T* grad_loss,
                         int squared, T* gL, T* gA, T* gD, int64_t B, int N, hipStream_t st) {
  return with_scan_plan(B, N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 2 * 64 * W, [&](int64_t off, unsigned n) {  // room for the front workgroups
      const unsigned grid = FastPath<T>::kEnabled ? n + static_cast<unsigned>(front_groups(n)) : n;
      hipLaunchKernelGGL((reconstruct_loss_backward_kernel<T, W, K, kScanPad, kLossSuperposed>), dim3(grid),
                         dim3(64 * W), 0, st, L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0,
                         xyz + off * N * 3, regular + off, target + off * N * 3,
                         grad_loss != nullptr ? grad_loss + off : nullptr, gL + off * (N - 1), gA + off * (N - 2),
                         gD + off * (N - 3), N, int64_t{n}, record + off * kSuperposeRecord, squared);
    });
  });
}

CUFK_INSTANTIATE(loss_fwd_typed<CUFK_T>)
CUFK_INSTANTIATE(loss_bwd_typed<CUFK_T>)
CUFK_INSTANTIATE(superposed_fwd_typed<CUFK_T>)
CUFK_INSTANTIATE(superposed_bwd_typed<CUFK_T>)

}  // namespace cufk_amd
#endif

#if CUFK_FAMILY == CUFK_FAMILY_LONG
#include "long_chain_kernels.h"
namespace cufk_amd {

template <typename T>
int long_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz, double* state,
                   int64_t B, int N, int S, hipStream_t st) {
  const int segs = static_cast<int>(long_segments(N, S));
  uint8_t* const flags = reinterpret_cast<uint8_t*>(state + long_flag_offset(B, segs));
  T* const local = reinterpret_cast<T*>(state + long_local_offset(B, segs));
  const int rc = with_scan_plan(B * segs, S, [&]<int W, int K>() {
    hipLaunchKernelGGL((long_forward_segments_kernel<T, W, K, kScanPad>), dim3(static_cast<unsigned>(B * segs)),
                       dim3(64 * W), 0, st, L, A, D, p0, fd, n0, xyz, local, flags, state, N, S, segs);
    return hipGetLastError() == hipSuccess ? CUFK_OK : CUFK_ERR_LAUNCH;
  });
  if (rc != CUFK_OK) return rc;
  constexpr int64_t kChainsPerGroup = kLongThreads / 64;  // one wave per chain
  hipLaunchKernelGGL(long_forward_frames_kernel<T>, dim3(static_cast<unsigned>((B + kChainsPerGroup - 1) / kChainsPerGroup)),
                     dim3(kLongThreads), 0, st, L, A, p0, fd, n0, state, B, N, segs);
  if (segs > 1)
    hipLaunchKernelGGL(long_forward_place_kernel<T>, dim3(static_cast<unsigned>(B * (segs - 1))), dim3(kLongThreads), 0,
                       st, xyz, local, state, N, S, segs);
  return hipGetLastError() == hipSuccess ? CUFK_OK : CUFK_ERR_LAUNCH;
}

template <typename T>
int long_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* xyz,
                   const double* state, const T* g, double* work, T* gL, T* gA, T* gD, int64_t B, int N, int S,
                   hipStream_t st, double* anchor) {
  const int segs = static_cast<int>(long_segments(N, S));
  const uint8_t* const flags = reinterpret_cast<const uint8_t*>(state + long_flag_offset(B, segs));
  const T* const local = reinterpret_cast<const T*>(state + long_local_offset(B, segs));
  if (segs > 1)
    hipLaunchKernelGGL(long_backward_sums_kernel<T>, dim3(static_cast<unsigned>(B * (segs - 1))), dim3(kLongThreads), 0,
                       st, xyz, g, state, work, N, S, segs);
  constexpr int64_t kChainsPerGroup = kLongThreads / 64;  // one wave per chain
  hipLaunchKernelGGL(long_backward_carry_kernel, dim3(static_cast<unsigned>((B + kChainsPerGroup - 1) / kChainsPerGroup)),
                     dim3(kLongThreads), 0, st, state, work, B, segs);
  if (hipGetLastError() != hipSuccess) return CUFK_ERR_LAUNCH;
  return with_scan_plan(B * segs, S, [&]<int W, int K>() {
    hipLaunchKernelGGL((long_backward_segments_kernel<T, W, K, kScanPad>), dim3(static_cast<unsigned>(B * segs)),
                       dim3(64 * W), 0, st, L, A, D, p0, fd, n0, xyz, local, flags, g, gL, gA, gD, state, work, N,
                       S, segs, anchor);
    return hipGetLastError() == hipSuccess ? CUFK_OK : CUFK_ERR_LAUNCH;
  });
}

CUFK_INSTANTIATE(long_fwd_typed<CUFK_T>)
CUFK_INSTANTIATE(long_bwd_typed<CUFK_T>)

}  // namespace cufk_amd
#endif

#if CUFK_FAMILY == CUFK_FAMILY_TORSION
namespace cufk_amd {

template <typename T>
int torsion_fwd_typed(const T* raw, int64_t rs, const TorsionArgs& c, T* xyz, int64_t B, int N, hipStream_t st) {
  return with_torsion_plan(N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((torsion_forward_kernel<T, W, K>), dim3(n), dim3(64 * W), 0, st, raw + off * rs, rs, c,
                         xyz + off * N * 3, N);
    });
  });
}

template <typename T>
int torsion_bwd_typed(const T* raw, int64_t rs, const T* xyz, const T* g, T* graw, int64_t gs, const TorsionArgs& c,
                      int64_t B, int N, hipStream_t st) {
  return with_torsion_bwd_plan(N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((torsion_backward_kernel<T, W, K>), dim3(n), dim3(64 * W), 0, st, raw + off * rs, rs,
                         xyz + off * N * 3, g + off * N * 3, graw + off * gs, gs, c, N);
    });
  });
}

template <typename T>
int torsion_loss_fwd_typed(int kind, const T* raw, int64_t rs, const TorsionArgs& c, const T* target, T* xyz, T* loss,
                           double* record, int squared, int64_t B, int N, hipStream_t st) {
  const int rc = with_torsion_plan(N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      double* rec = record != nullptr ? record + off * kSuperposeRecord : nullptr;
      if (kind == kLossSuperposed)
        hipLaunchKernelGGL((torsion_forward_kernel<T, W, K, kLossSuperposed>), dim3(n), dim3(64 * W), 0, st,
                           raw + off * rs, rs, c, xyz + off * N * 3, N, target + off * N * 3, nullptr, rec);
      else
        hipLaunchKernelGGL((torsion_forward_kernel<T, W, K, kLossSquared>), dim3(n), dim3(64 * W), 0, st, raw + off * rs,
                           rs, c, xyz + off * N * 3, N, target + off * N * 3, loss + off, nullptr);
    });
  });
  if (rc != CUFK_OK || kind != kLossSuperposed) return rc;
  return solve_records<T>(record, loss, B, N, squared, st);
}

template <typename T>
int torsion_loss_bwd_typed(int kind, const T* raw, int64_t rs, const T* xyz, const T* target, const double* record,
                           const T* grad_loss, int squared, T* graw, int64_t gs, const TorsionArgs& c, int64_t B, int N,
                           hipStream_t st) {
  return with_torsion_bwd_plan(N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      const T* gl = grad_loss != nullptr ? grad_loss + off : nullptr;
      if (kind == kLossSuperposed)
        hipLaunchKernelGGL((torsion_backward_kernel<T, W, K, kLossSuperposed>), dim3(n), dim3(64 * W), 0, st,
                           raw + off * rs, rs, xyz + off * N * 3, target + off * N * 3, graw + off * gs, gs, c, N, gl,
                           record + off * kSuperposeRecord, squared);
      else
        hipLaunchKernelGGL((torsion_backward_kernel<T, W, K, kLossSquared>), dim3(n), dim3(64 * W), 0, st,
                           raw + off * rs, rs, xyz + off * N * 3, target + off * N * 3, graw + off * gs, gs, c, N, gl,
                           nullptr, 0);
    });
  });
}

CUFK_INSTANTIATE(torsion_fwd_typed<CUFK_T>)
CUFK_INSTANTIATE(torsion_bwd_typed<CUFK_T>)
CUFK_INSTANTIATE(torsion_loss_fwd_typed<CUFK_T>)
CUFK_INSTANTIATE(torsion_loss_bwd_typed<CUFK_T>)

}  // namespace cufk_amd
#endif
