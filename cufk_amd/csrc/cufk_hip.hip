// C ABI of the MI355X (gfx950) reconstruction library: launch plans and entry points.
//
// Kernels live in reconstruct_kernels.h and torsion_kernels.h.  One workgroup of W wave64s
// reconstructs one chain; lane t owns the K consecutive steps [tK, tK+K) (blocked
// arrangement, as in the reference block.cu:187), runs them as a serial scan in registers and
// only lane totals cross lanes (wave64 DPP scan, then an LDS carry across waves).  Rows move
// between HBM and LDS as coalesced 16-byte streams.
#include "cufk_hip.h"

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "chain_ops.h"
#include "long_chain_kernels.h"
#include "packed_kernels.h"
#include "reconstruct_kernels.h"
#include "staging.h"
#include "torsion_kernels.h"

namespace cufk_amd {

constexpr int kMaxSteps = 2048;  // block.cu:88, torsion.cu:97 (512 threads x 4 items)

// ---------------------------------------------------------------------------- plans

// (waves W, items per lane K), capacity 64*W*K steps; the smallest plan holding the chain.
// Eight items per lane measured fastest at N = 2049 for both the forward and the
// position-based backward (K = 16 runs out of registers and waves, K = 4 pays the lane scan
// on too few items).  The exact backward uses the same plans.  The kernels stage rows with one
// word of padding per lane: at (4, 8) that lets five forward workgroups (three backward)
// share a CU instead of four (two).
constexpr int kScanPad = 1;
template <typename Fn> int with_scan_plan(int steps, Fn&& fn) {
  if (steps <= 256) return fn.template operator()<1, 4>();
  if (steps <= 512) return fn.template operator()<1, 8>();
  if (steps <= 1024) return fn.template operator()<2, 8>();
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

// Short chains: G lanes per chain, 8 steps per lane, 64W/G chains per workgroup (packed
// kernels).  Measured on MI355X against one chain per workgroup: packing wins from about 4096
// chains up (at 8192 chains: forward 9.5-15.5 us against 19-21 us for 9-128 steps), loses
// below (fewer waves in flight), and its backward stops winning past 64 steps (at 128 steps
// and 32768 chains: 44 us against 34 us).
constexpr int kPackedFwdMaxSteps = 128;
constexpr int kPackedBwdMaxSteps = 64;
constexpr int64_t kPackedMinBatch = 4096;
constexpr int kPackedWaves = 2;
template <int MaxG = 16, typename Fn> int with_packed_plan(int steps, Fn&& fn) {
  if (steps <= 8) return fn.template operator()<1>();
  if (steps <= 16) return fn.template operator()<2>();
  if (steps <= 32) return fn.template operator()<4>();
  if (MaxG == 8 || steps <= 64) return fn.template operator()<8>();
  if constexpr (MaxG >= 16) return fn.template operator()<16>();
  return CUFK_ERR_STEPS;
}
inline bool use_packed_fwd(int64_t B, int steps) { return steps <= kPackedFwdMaxSteps && B >= kPackedMinBatch; }
inline bool use_packed_bwd(int64_t B, int steps) { return steps <= kPackedBwdMaxSteps && B >= kPackedMinBatch; }
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
                     double* anchor = nullptr) {
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

// ---------------------------------------------------------------------------- reconstruct

template <typename T>
int reconstruct_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz,
                          uint8_t* regular, int64_t B, int N, hipStream_t st) {
  if (use_packed_fwd(B, N - 3)) return packed_fwd_typed<T>(L, A, D, p0, fd, n0, xyz, regular, B, N, st);
  return with_scan_plan(N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((reconstruct_forward_kernel<T, W, K, kScanPad>), dim3(n), dim3(64 * W), 0, st, L + off * (N - 1),
                         A + off * (N - 2), D + off * (N - 3), p0, fd, n0, xyz + off * N * 3,
                         regular ? regular + off : nullptr, N);
    });
  });
}

// Backward without a saved output: the forward scan is rerun per chain, then the
// position-based adjoint (or the exact one for irregular chains).
template <typename T>
int reconstruct_bwd_recompute_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0,
                                    const T* g, T* gL, T* gA, T* gD, int64_t B, int N, hipStream_t st,
                                    double* anchor = nullptr) {
  if (use_packed_bwd(B, N - 3))
    return packed_bwd_typed<T, false>(L, A, D, p0, fd, n0, nullptr, nullptr, g, gL, gA, gD, B, N, st, anchor);
  return with_scan_plan(N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((reconstruct_backward_recompute_kernel<T, W, K, kScanPad>), dim3(n), dim3(64 * W), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, g + off * N * 3,
                         gL + off * (N - 1), gA + off * (N - 2), gD + off * (N - 3), N,
                         anchor != nullptr ? anchor + off * 6 : nullptr);
    });
  });
}

// Backward over the saved forward output: one launch, each chain taking the position-based
// or the exact path by its flag.
template <typename T>
int reconstruct_bwd_saved_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0,
                                const T* xyz, const uint8_t* regular, const T* g, T* gL, T* gA, T* gD, int64_t B, int N,
                                hipStream_t st, double* anchor = nullptr) {
  if (use_packed_bwd(B, N - 3))
    return packed_bwd_typed<T, true>(L, A, D, p0, fd, n0, xyz, regular, g, gL, gA, gD, B, N, st, anchor);
  return with_scan_plan(N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((reconstruct_backward_saved_kernel<T, W, K, kScanPad>), dim3(n), dim3(64 * W), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, xyz + off * N * 3,
                         regular + off, g + off * N * 3, gL + off * (N - 1), gA + off * (N - 2), gD + off * (N - 3), N,
                         anchor != nullptr ? anchor + off * 6 : nullptr);
    });
  });
}

// Fused coordinate loss: one workgroup per chain, the plans of the reconstruct kernels.
template <typename T>
int loss_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* target, T* xyz,
                   uint8_t* regular, T* loss, int64_t B, int N, hipStream_t st) {
  return with_scan_plan(N - 3, [&]<int W, int K>() {
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
                   hipStream_t st) {
  return with_scan_plan(N - 3, [&]<int W, int K>() {
    return launch_chunks(B, 64 * W, [&](int64_t off, unsigned n) {
      hipLaunchKernelGGL((reconstruct_loss_backward_kernel<T, W, K, kScanPad>), dim3(n), dim3(64 * W), 0, st,
                         L + off * (N - 1), A + off * (N - 2), D + off * (N - 3), p0, fd, n0, xyz + off * N * 3,
                         regular + off, target + off * N * 3, grad_loss != nullptr ? grad_loss + off : nullptr,
                         gL + off * (N - 1), gA + off * (N - 2), gD + off * (N - 3), N);
    });
  });
}

// ---------------------------------------------------------------------------- long chains

// Default segment length: the largest plan capacity (2048 steps) unless the grid would then
// hold fewer than ~4 workgroups per CU; halved down to 256 steps until it does.
constexpr int64_t kLongMinSegment = 256;
constexpr int64_t kLongTargetGroups = 1024;
// Grid extents of the long-chain launches count work-items in 32 bits.
constexpr int64_t kLongMaxGroups = int64_t{UINT32_MAX} / 256;

inline int64_t long_segments(int64_t points, int64_t seg_steps) { return (points - 3 + seg_steps - 1) / seg_steps; }

template <typename T>
int long_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz, double* state,
                   int64_t B, int N, int S, hipStream_t st) {
  const int segs = static_cast<int>(long_segments(N, S));
  const int rc = with_scan_plan(S, [&]<int W, int K>() {
    hipLaunchKernelGGL((long_forward_segments_kernel<T, W, K, kScanPad>), dim3(static_cast<unsigned>(B * segs)),
                       dim3(64 * W), 0, st, L, A, D, p0, fd, n0, xyz, state, N, S, segs);
    return hipGetLastError() == hipSuccess ? CUFK_OK : CUFK_ERR_LAUNCH;
  });
  if (rc != CUFK_OK) return rc;
  constexpr int64_t kChainsPerGroup = kLongThreads / 64;  // one wave per chain
  hipLaunchKernelGGL(long_forward_frames_kernel<T>, dim3(static_cast<unsigned>((B + kChainsPerGroup - 1) / kChainsPerGroup)),
                     dim3(kLongThreads), 0, st, L, A, p0, fd, n0, state, B, N, segs);
  if (segs > 1)
    hipLaunchKernelGGL(long_forward_place_kernel<T>, dim3(static_cast<unsigned>(B * (segs - 1))), dim3(kLongThreads), 0,
                       st, xyz, state, N, S, segs);
  return hipGetLastError() == hipSuccess ? CUFK_OK : CUFK_ERR_LAUNCH;
}

template <typename T>
int long_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* xyz,
                   const double* state, const T* g, double* work, T* gL, T* gA, T* gD, int64_t B, int N, int S,
                   hipStream_t st) {
  const int segs = static_cast<int>(long_segments(N, S));
  if (segs > 1)
    hipLaunchKernelGGL(long_backward_sums_kernel<T>, dim3(static_cast<unsigned>(B * (segs - 1))), dim3(kLongThreads), 0,
                       st, xyz, g, state, work, N, S, segs);
  constexpr int64_t kChainsPerGroup = kLongThreads / 64;  // one wave per chain
  hipLaunchKernelGGL(long_backward_carry_kernel, dim3(static_cast<unsigned>((B + kChainsPerGroup - 1) / kChainsPerGroup)),
                     dim3(kLongThreads), 0, st, state, work, B, segs);
  if (hipGetLastError() != hipSuccess) return CUFK_ERR_LAUNCH;
  return with_scan_plan(S, [&]<int W, int K>() {
    hipLaunchKernelGGL((long_backward_segments_kernel<T, W, K, kScanPad>), dim3(static_cast<unsigned>(B * segs)),
                       dim3(64 * W), 0, st, L, A, D, p0, fd, n0, g, gL, gA, gD, state, work, N, S, segs);
    return hipGetLastError() == hipSuccess ? CUFK_OK : CUFK_ERR_LAUNCH;
  });
}

// ---------------------------------------------------------------------------- torsion

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

// ---------------------------------------------------------------------------- dispatch helpers

// Shape validation shared by every entry point (extension_utils.cuh:119-130).
inline int check_chain(int64_t batch, int64_t points) {
  if (batch < 0 || batch > INT32_MAX || points > INT32_MAX) return CUFK_ERR_SHAPE;
  if (points < 4) return CUFK_ERR_POINTS;
  if (points - 3 > kMaxSteps) return CUFK_ERR_STEPS;
  return CUFK_OK;
}

// Long chains: no step cap, but in-row element offsets stay in int32 and the segment grid
// within one launch.
inline int check_long(int64_t batch, int64_t points, int64_t seg_steps) {
  if (batch < 0 || batch > INT32_MAX || points > INT32_MAX / 3) return CUFK_ERR_SHAPE;
  if (points < 4) return CUFK_ERR_POINTS;
  if (seg_steps < 1 || seg_steps > kMaxSteps) return CUFK_ERR_SEGMENT;
  if (batch * long_segments(points, seg_steps) > kLongMaxGroups) return CUFK_ERR_SHAPE;
  return CUFK_OK;
}

inline bool valid_dtype(int dtype) { return dtype >= CUFK_FLOAT32 && dtype <= CUFK_BFLOAT16; }

template <typename Fn> int dispatch(int dtype, Fn&& fn) {
  switch (dtype) {
    case CUFK_FLOAT32: return fn.template operator()<float>();
    case CUFK_FLOAT64: return fn.template operator()<double>();
    case CUFK_FLOAT16: return fn.template operator()<_Float16>();
    case CUFK_BFLOAT16: return fn.template operator()<__bf16>();
    default: return CUFK_ERR_DTYPE;
  }
}

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

template <typename T> const T* cp(const void* p) { return static_cast<const T*>(p); }
template <typename T> T* mp(void* p) { return static_cast<T*>(p); }

}  // namespace cufk_amd

using namespace cufk_amd;

extern "C" {

int cufk_reconstruct_fwd_flagged(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                 const void* p0, const void* first_direction, const void* initial_normal, void* xyz,
                                 uint8_t* chain_regular, int64_t batch, int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !xyz) return CUFK_ERR_NULL;
  const int N = static_cast<int>(points);
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    return reconstruct_fwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0), cp<T>(first_direction),
                                    cp<T>(initial_normal), mp<T>(xyz), chain_regular, batch, N, st);
  });
}

int cufk_reconstruct_fwd(int dtype, const void* lengths, const void* angles, const void* dihedrals, const void* p0,
                         const void* first_direction, const void* initial_normal, void* xyz, int64_t batch,
                         int64_t points, void* stream) {
  return cufk_reconstruct_fwd_flagged(dtype, lengths, angles, dihedrals, p0, first_direction, initial_normal, xyz,
                                      nullptr, batch, points, stream);
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
  return dispatch(dtype, [&]<typename T>() {
    return reconstruct_bwd_recompute_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0),
                                              cp<T>(first_direction), cp<T>(initial_normal), cp<T>(grad_xyz),
                                              mp<T>(grad_lengths), mp<T>(grad_angles), mp<T>(grad_dihedrals), batch, N,
                                              st);
  });
}

int cufk_reconstruct_bwd_saved(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                               const void* p0, const void* first_direction, const void* initial_normal,
                               const void* xyz, const uint8_t* chain_regular, const void* grad_xyz, void* grad_lengths,
                               void* grad_angles, void* grad_dihedrals, int64_t batch, int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !xyz || !chain_regular ||
      !grad_xyz || !grad_lengths || !grad_angles || !grad_dihedrals)
    return CUFK_ERR_NULL;
  const int N = static_cast<int>(points);
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    if constexpr (FastPath<T>::kEnabled) {
      return reconstruct_bwd_saved_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0),
                                            cp<T>(first_direction), cp<T>(initial_normal), cp<T>(xyz), chain_regular,
                                            cp<T>(grad_xyz), mp<T>(grad_lengths), mp<T>(grad_angles),
                                            mp<T>(grad_dihedrals), batch, N, st);
    } else {
      // float16 / bfloat16 outputs are too coarse for the position-based adjoint; the
      // positions are recomputed in float instead.
      return reconstruct_bwd_recompute_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0),
                                                cp<T>(first_direction), cp<T>(initial_normal), cp<T>(grad_xyz),
                                                mp<T>(grad_lengths), mp<T>(grad_angles), mp<T>(grad_dihedrals), batch,
                                                N, st);
    }
  });
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
  return dispatch(dtype, [&]<typename T>() {
    return torsion_fwd_typed<T>(cp<T>(raw_pairs), raw_stride, args, mp<T>(xyz), batch, N, st);
  });
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
  return dispatch(dtype, [&]<typename T>() {
    return torsion_bwd_typed<T>(cp<T>(raw_pairs), raw_stride, cp<T>(xyz), cp<T>(grad_xyz), mp<T>(grad_raw),
                                grad_raw_stride, args, batch, N, st);
  });
}

int cufk_reconstruct_bwd_anchored(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                  const void* p0, const void* first_direction, const void* initial_normal,
                                  const void* xyz, const uint8_t* chain_regular, const void* grad_xyz,
                                  void* grad_lengths, void* grad_angles, void* grad_dihedrals, double* anchor_work,
                                  void* grad_p0, void* grad_first_direction, void* grad_initial_normal, int64_t batch,
                                  int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (!p0 || !first_direction || !initial_normal || !grad_p0 || !grad_first_direction || !grad_initial_normal)
    return CUFK_ERR_NULL;
  if (batch > 0 && (!lengths || !angles || !dihedrals || (xyz && !chain_regular) || !grad_xyz || !grad_lengths ||
                    !grad_angles || !grad_dihedrals || !anchor_work))
    return CUFK_ERR_NULL;
  const int N = static_cast<int>(points);
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    int r = CUFK_OK;
    if (batch > 0) {
      if (xyz != nullptr && FastPath<T>::kEnabled) {
        r = reconstruct_bwd_saved_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0),
                                           cp<T>(first_direction), cp<T>(initial_normal), cp<T>(xyz), chain_regular,
                                           cp<T>(grad_xyz), mp<T>(grad_lengths), mp<T>(grad_angles),
                                           mp<T>(grad_dihedrals), batch, N, st, anchor_work);
      } else {
        r = reconstruct_bwd_recompute_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0),
                                               cp<T>(first_direction), cp<T>(initial_normal), cp<T>(grad_xyz),
                                               mp<T>(grad_lengths), mp<T>(grad_angles), mp<T>(grad_dihedrals), batch,
                                               N, st, anchor_work);
      }
      if (r != CUFK_OK) return r;
    }
    hipLaunchKernelGGL(anchor_gradients_kernel<T>, dim3(1), dim3(kAnchorThreads), 0, st, anchor_work, batch,
                       cp<T>(first_direction), cp<T>(initial_normal), mp<T>(grad_p0), mp<T>(grad_first_direction),
                       mp<T>(grad_initial_normal));
    return hipGetLastError() == hipSuccess ? int{CUFK_OK} : int{CUFK_ERR_LAUNCH};
  });
}

int cufk_reconstruct_loss_fwd(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                              const void* p0, const void* first_direction, const void* initial_normal,
                              const void* target, void* xyz, uint8_t* chain_regular, void* loss, int64_t batch,
                              int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !target || !xyz ||
      !chain_regular || !loss)
    return CUFK_ERR_NULL;
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    return loss_fwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0), cp<T>(first_direction),
                             cp<T>(initial_normal), cp<T>(target), mp<T>(xyz), chain_regular, mp<T>(loss), batch,
                             static_cast<int>(points), st);
  });
}

int cufk_reconstruct_loss_bwd(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                              const void* p0, const void* first_direction, const void* initial_normal, const void* xyz,
                              const uint8_t* chain_regular, const void* target, const void* grad_loss,
                              void* grad_lengths, void* grad_angles, void* grad_dihedrals, int64_t batch,
                              int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !xyz || !chain_regular ||
      !target || !grad_lengths || !grad_angles || !grad_dihedrals)
    return CUFK_ERR_NULL;
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    return loss_bwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0), cp<T>(first_direction),
                             cp<T>(initial_normal), cp<T>(xyz), chain_regular, cp<T>(target), cp<T>(grad_loss),
                             mp<T>(grad_lengths), mp<T>(grad_angles), mp<T>(grad_dihedrals), batch,
                             static_cast<int>(points), st);
  });
}

int64_t cufk_long_segment_steps(int64_t batch, int64_t points) {
  if (batch < 0 || points < 4) return 0;
  int64_t S = kMaxSteps;
  while (S > kLongMinSegment && batch * long_segments(points, S) < kLongTargetGroups) S /= 2;
  return S;
}

int64_t cufk_long_state_doubles(int64_t batch, int64_t points, int64_t segment_steps) {
  if (check_long(batch, points, segment_steps) != CUFK_OK) return -1;
  return batch * long_segments(points, segment_steps) * kLongStateDoubles;
}

int64_t cufk_long_work_doubles(int64_t batch, int64_t points, int64_t segment_steps) {
  if (check_long(batch, points, segment_steps) != CUFK_OK) return -1;
  return batch * long_segments(points, segment_steps) * kLongWorkDoubles;
}

int cufk_reconstruct_long_fwd(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                              const void* p0, const void* first_direction, const void* initial_normal, void* xyz,
                              double* state, int64_t batch, int64_t points, int64_t segment_steps, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_long(batch, points, segment_steps);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !xyz || !state)
    return CUFK_ERR_NULL;
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    return long_fwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0), cp<T>(first_direction),
                             cp<T>(initial_normal), mp<T>(xyz), state, batch, static_cast<int>(points),
                             static_cast<int>(segment_steps), st);
  });
}

int cufk_reconstruct_long_bwd(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                              const void* p0, const void* first_direction, const void* initial_normal, const void* xyz,
                              const double* state, const void* grad_xyz, double* work, void* grad_lengths,
                              void* grad_angles, void* grad_dihedrals, int64_t batch, int64_t points,
                              int64_t segment_steps, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_long(batch, points, segment_steps);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !xyz || !state ||
      !grad_xyz || !work || !grad_lengths || !grad_angles || !grad_dihedrals)
    return CUFK_ERR_NULL;
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    return long_bwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0), cp<T>(first_direction),
                             cp<T>(initial_normal), cp<T>(xyz), state, cp<T>(grad_xyz), work, mp<T>(grad_lengths),
                             mp<T>(grad_angles), mp<T>(grad_dihedrals), batch, static_cast<int>(points),
                             static_cast<int>(segment_steps), st);
  });
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
    case CUFK_ERR_SEGMENT: return "segment length must be in [1, 2048] local transforms";
    default: return "unknown status";
  }
}

const char* cufk_version(void) { return "0.1.0"; }

}  // extern "C"
