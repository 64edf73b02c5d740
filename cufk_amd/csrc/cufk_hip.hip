// C ABI of the MI355X (gfx950) reconstruction library: argument checks and dtype dispatch.
//
// The typed launchers it calls are declared in launch.h and defined in launchers.hip, which is
// compiled once per (dtype, kernel family); this unit instantiates no kernel.
#include "cufk_hip.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cstdint>
#include <cstring>
#include <mutex>

#include "launch.h"

namespace cufk_amd {

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

// Raw-pair row strides: reading rows that overlap is harmless, but gradient rows that overlap
// (a stride shorter than the row's 2(N-3) values, more than one chain) would have workgroups
// writing each other's elements.
inline int check_pair_strides(int64_t raw_stride, int64_t grad_raw_stride, int64_t batch, int64_t points) {
  if (raw_stride < 0 || grad_raw_stride < 0) return CUFK_ERR_STRIDE;
  if (batch > 1 && grad_raw_stride < 2 * (points - 3)) return CUFK_ERR_STRIDE;
  return CUFK_OK;
}

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

// ---------------------------------------------------------------------------- static scratch

// Scratch of cufk_reconstruct_bwd_anchored_noalloc: the per-chain force and torque sums that
// cufk_reconstruct_bwd_anchored keeps in its anchor_work argument, six doubles per chain.  Every
// GPU the library runs on holds one copy (3 MiB) until the process ends.  In host code the name
// `scratch` is a stand-in, not a device address: kernels get the address that
// hipGetSymbolAddress returns for the current device, looked up once per device.
constexpr int64_t kNoAllocMaxChains = CUFK_NOALLOC_MAX_CHAINS;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) double scratch[6 * kNoAllocMaxChains];

// The device address of `scratch` on the current device, or a status.  The first call on a
// device looks it up (this allocates nothing; the array is part of the loaded code object).
inline int scratch_on_current_device(double** out) {
  static std::mutex mutex;
  static double* address[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return CUFK_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(mutex);
  if (address[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return CUFK_ERR_DEVICE;
    address[dev] = static_cast<double*>(p);
  }
  *out = address[dev];
  return CUFK_OK;
}

// Whether `device` is a present HIP device of the one architecture this library carries code
// for (gfx950).  Cached per device index: the torch binding asks on every call.
bool device_supported(int device) {
  constexpr int kMaxDevices = 64;
  static std::atomic<signed char> known[kMaxDevices] = {};  // 0 unknown, 1 supported, -1 not
  if (device < 0 || device >= kMaxDevices) return false;
  const signed char k = known[device].load(std::memory_order_relaxed);
  if (k != 0) return k > 0;
  int count = 0;
  bool ok = hipGetDeviceCount(&count) == hipSuccess && device < count;
  if (ok) {
    hipDeviceProp_t prop;
    ok = hipGetDeviceProperties(&prop, device) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
         (prop.gcnArchName[6] == '\0' || prop.gcnArchName[6] == ':');
  }
  known[device].store(ok ? 1 : -1, std::memory_order_relaxed);
  return ok;
}

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

int64_t cufk_reconstruct_shadow_floats(int64_t batch, int64_t points) {
  if (check_chain(batch, points) != CUFK_OK) return -1;
  return use_shadow(batch, points - 3) ? batch * points * 3 : 0;
}

int cufk_reconstruct_fwd_shadow(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                const void* p0, const void* first_direction, const void* initial_normal, void* xyz,
                                float* positions, uint8_t* chain_regular, int64_t batch, int64_t points,
                                void* stream) {
  if (dtype != CUFK_FLOAT16 && dtype != CUFK_BFLOAT16) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !xyz) return CUFK_ERR_NULL;
  if (use_shadow(batch, points - 3) && (!positions || !chain_regular)) return CUFK_ERR_NULL;
  const int N = static_cast<int>(points);
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    if constexpr (sizeof(T) == 2) {
      return shadow_fwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0), cp<T>(first_direction),
                                 cp<T>(initial_normal), mp<T>(xyz), positions, chain_regular, batch, N, st);
    } else {
      return static_cast<int>(CUFK_ERR_DTYPE);
    }
  });
}

int cufk_reconstruct_bwd_shadow(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                const void* p0, const void* first_direction, const void* initial_normal,
                                const float* positions, const uint8_t* chain_regular, const void* grad_xyz,
                                void* grad_lengths, void* grad_angles, void* grad_dihedrals, int64_t batch,
                                int64_t points, void* stream) {
  if (dtype != CUFK_FLOAT16 && dtype != CUFK_BFLOAT16) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !grad_xyz || !grad_lengths ||
      !grad_angles || !grad_dihedrals)
    return CUFK_ERR_NULL;
  if (use_shadow(batch, points - 3) && (!positions || !chain_regular)) return CUFK_ERR_NULL;
  const int N = static_cast<int>(points);
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    if constexpr (sizeof(T) == 2) {
      return shadow_bwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0), cp<T>(first_direction),
                                 cp<T>(initial_normal), positions, chain_regular, cp<T>(grad_xyz), mp<T>(grad_lengths),
                                 mp<T>(grad_angles), mp<T>(grad_dihedrals), batch, N, st);
    } else {
      return static_cast<int>(CUFK_ERR_DTYPE);
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
  const int sc = check_pair_strides(raw_stride, grad_raw_stride, batch, points);
  if (sc != CUFK_OK) return sc;
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
      bool saved = false;
      if constexpr (FastPath<T>::kEnabled) {
        if (xyz != nullptr) {
          saved = true;
          r = reconstruct_bwd_saved_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0),
                                             cp<T>(first_direction), cp<T>(initial_normal), cp<T>(xyz), chain_regular,
                                             cp<T>(grad_xyz), mp<T>(grad_lengths), mp<T>(grad_angles),
                                             mp<T>(grad_dihedrals), batch, N, st, anchor_work);
        }
      }
      if (!saved) {
        r = reconstruct_bwd_recompute_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0),
                                               cp<T>(first_direction), cp<T>(initial_normal), cp<T>(grad_xyz),
                                               mp<T>(grad_lengths), mp<T>(grad_angles), mp<T>(grad_dihedrals), batch,
                                               N, st, anchor_work);
      }
      if (r != CUFK_OK) return r;
    }
    return anchor_grads_typed<T>(anchor_work, batch, cp<T>(first_direction), cp<T>(initial_normal), mp<T>(grad_p0),
                                 mp<T>(grad_first_direction), mp<T>(grad_initial_normal), st);
  });
}

int cufk_reconstruct_bwd_anchored_noalloc(int dtype, const void* lengths, const void* angles,
                                          const void* dihedrals, const void* p0, const void* first_direction,
                                          const void* initial_normal, const void* xyz, const uint8_t* chain_regular,
                                          const void* grad_xyz, void* grad_lengths, void* grad_angles,
                                          void* grad_dihedrals, void* grad_p0, void* grad_first_direction,
                                          void* grad_initial_normal, int64_t batch, int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch > kNoAllocMaxChains) return CUFK_ERR_SCRATCH;
  double* work = nullptr;
  const int sc = scratch_on_current_device(&work);
  if (sc != CUFK_OK) return sc;
  return cufk_reconstruct_bwd_anchored(dtype, lengths, angles, dihedrals, p0, first_direction, initial_normal, xyz,
                                       chain_regular, grad_xyz, grad_lengths, grad_angles, grad_dihedrals, work,
                                       grad_p0, grad_first_direction, grad_initial_normal, batch, points, stream);
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

int cufk_reconstruct_loss_bwd_anchored(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                       const void* p0, const void* first_direction, const void* initial_normal,
                                       const void* xyz, const uint8_t* chain_regular, const void* target,
                                       const void* grad_loss, void* grad_lengths, void* grad_angles,
                                       void* grad_dihedrals, double* anchor_work, void* grad_p0,
                                       void* grad_first_direction, void* grad_initial_normal, int64_t batch,
                                       int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (!p0 || !first_direction || !initial_normal || !grad_p0 || !grad_first_direction || !grad_initial_normal)
    return CUFK_ERR_NULL;
  if (batch > 0 && (!lengths || !angles || !dihedrals || !xyz || !chain_regular || !target || !grad_lengths ||
                    !grad_angles || !grad_dihedrals || !anchor_work))
    return CUFK_ERR_NULL;
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    if (batch > 0) {
      const int r = loss_bwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0),
                                      cp<T>(first_direction), cp<T>(initial_normal), cp<T>(xyz), chain_regular,
                                      cp<T>(target), cp<T>(grad_loss), mp<T>(grad_lengths), mp<T>(grad_angles),
                                      mp<T>(grad_dihedrals), batch, static_cast<int>(points), st, anchor_work);
      if (r != CUFK_OK) return r;
    }
    return anchor_grads_typed<T>(anchor_work, batch, cp<T>(first_direction), cp<T>(initial_normal), mp<T>(grad_p0),
                                 mp<T>(grad_first_direction), mp<T>(grad_initial_normal), st);
  });
}

int cufk_reconstruct_superposed_fwd(int dtype, int loss_kind, const void* lengths, const void* angles,
                                    const void* dihedrals, const void* p0, const void* first_direction,
                                    const void* initial_normal, const void* target, void* xyz, uint8_t* chain_regular,
                                    void* loss, double* superposition, int64_t batch, int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  if (loss_kind != CUFK_LOSS_MSD && loss_kind != CUFK_LOSS_RMSD) return CUFK_ERR_LOSS;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !target || !xyz ||
      !chain_regular || !loss || !superposition)
    return CUFK_ERR_NULL;
  auto st = static_cast<hipStream_t>(stream);
  const int squared = loss_kind == CUFK_LOSS_MSD;
  return dispatch(dtype, [&]<typename T>() {
    return superposed_fwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0), cp<T>(first_direction),
                                   cp<T>(initial_normal), cp<T>(target), mp<T>(xyz), chain_regular, mp<T>(loss),
                                   superposition, squared, batch, static_cast<int>(points), st);
  });
}

int cufk_reconstruct_superposed_bwd(int dtype, int loss_kind, const void* lengths, const void* angles,
                                    const void* dihedrals, const void* p0, const void* first_direction,
                                    const void* initial_normal, const void* xyz, const uint8_t* chain_regular,
                                    const void* target, const double* superposition, const void* grad_loss,
                                    void* grad_lengths, void* grad_angles, void* grad_dihedrals, int64_t batch,
                                    int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  if (loss_kind != CUFK_LOSS_MSD && loss_kind != CUFK_LOSS_RMSD) return CUFK_ERR_LOSS;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (batch == 0) return CUFK_OK;
  if (!lengths || !angles || !dihedrals || !p0 || !first_direction || !initial_normal || !xyz || !chain_regular ||
      !target || !superposition || !grad_lengths || !grad_angles || !grad_dihedrals)
    return CUFK_ERR_NULL;
  auto st = static_cast<hipStream_t>(stream);
  const int squared = loss_kind == CUFK_LOSS_MSD;
  return dispatch(dtype, [&]<typename T>() {
    return superposed_bwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0), cp<T>(first_direction),
                                   cp<T>(initial_normal), cp<T>(xyz), chain_regular, cp<T>(target), superposition,
                                   cp<T>(grad_loss), squared, mp<T>(grad_lengths), mp<T>(grad_angles),
                                   mp<T>(grad_dihedrals), batch, static_cast<int>(points), st);
  });
}

int cufk_torsion_loss_fwd(int dtype, int loss_kind, const void* raw_pairs, int64_t raw_stride,
                          const cufk_torsion_consts* consts, const void* target, void* xyz, void* loss,
                          double* superposition, int64_t batch, int64_t points, void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  if (loss_kind < CUFK_LOSS_SQUARED_DISTANCE || loss_kind > CUFK_LOSS_RMSD) return CUFK_ERR_LOSS;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  if (raw_stride < 0) return CUFK_ERR_STRIDE;
  if (!consts) return CUFK_ERR_NULL;
  if (batch == 0) return CUFK_OK;
  const bool superposed = loss_kind != CUFK_LOSS_SQUARED_DISTANCE;
  if (!raw_pairs || !target || !xyz || !loss || (superposed && !superposition)) return CUFK_ERR_NULL;
  const TorsionArgs args = torsion_args(*consts);
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    return torsion_loss_fwd_typed<T>(superposed ? kLossSuperposed : kLossSquared, cp<T>(raw_pairs), raw_stride, args,
                                     cp<T>(target), mp<T>(xyz), mp<T>(loss), superposed ? superposition : nullptr,
                                     loss_kind == CUFK_LOSS_MSD, batch, static_cast<int>(points), st);
  });
}

int cufk_torsion_loss_bwd(int dtype, int loss_kind, const void* raw_pairs, int64_t raw_stride, const void* xyz,
                          const void* target, const double* superposition, const void* grad_loss, void* grad_raw,
                          int64_t grad_raw_stride, const cufk_torsion_consts* consts, int64_t batch, int64_t points,
                          void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  if (loss_kind < CUFK_LOSS_SQUARED_DISTANCE || loss_kind > CUFK_LOSS_RMSD) return CUFK_ERR_LOSS;
  const int rc = check_chain(batch, points);
  if (rc != CUFK_OK) return rc;
  const int sc = check_pair_strides(raw_stride, grad_raw_stride, batch, points);
  if (sc != CUFK_OK) return sc;
  if (!consts) return CUFK_ERR_NULL;
  if (batch == 0) return CUFK_OK;
  const bool superposed = loss_kind != CUFK_LOSS_SQUARED_DISTANCE;
  if (!raw_pairs || !xyz || !target || !grad_raw || (superposed && !superposition)) return CUFK_ERR_NULL;
  const TorsionArgs args = torsion_args(*consts);
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    return torsion_loss_bwd_typed<T>(superposed ? kLossSuperposed : kLossSquared, cp<T>(raw_pairs), raw_stride,
                                     cp<T>(xyz), cp<T>(target), superposed ? superposition : nullptr,
                                     cp<T>(grad_loss), loss_kind == CUFK_LOSS_MSD, mp<T>(grad_raw), grad_raw_stride,
                                     args, batch, static_cast<int>(points), st);
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
  return long_state_size(batch, points, long_segments(points, segment_steps));
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

int cufk_reconstruct_long_bwd_anchored(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                       const void* p0, const void* first_direction, const void* initial_normal,
                                       const void* xyz, const double* state, const void* grad_xyz, double* work,
                                       void* grad_lengths, void* grad_angles, void* grad_dihedrals,
                                       double* anchor_work, void* grad_p0, void* grad_first_direction,
                                       void* grad_initial_normal, int64_t batch, int64_t points, int64_t segment_steps,
                                       void* stream) {
  if (!valid_dtype(dtype)) return CUFK_ERR_DTYPE;
  const int rc = check_long(batch, points, segment_steps);
  if (rc != CUFK_OK) return rc;
  if (!p0 || !first_direction || !initial_normal || !grad_p0 || !grad_first_direction || !grad_initial_normal)
    return CUFK_ERR_NULL;
  if (batch > 0 && (!lengths || !angles || !dihedrals || !xyz || !state || !grad_xyz || !work || !grad_lengths ||
                    !grad_angles || !grad_dihedrals || !anchor_work))
    return CUFK_ERR_NULL;
  auto st = static_cast<hipStream_t>(stream);
  return dispatch(dtype, [&]<typename T>() {
    if (batch > 0) {
      const int r = long_bwd_typed<T>(cp<T>(lengths), cp<T>(angles), cp<T>(dihedrals), cp<T>(p0),
                                      cp<T>(first_direction), cp<T>(initial_normal), cp<T>(xyz), state,
                                      cp<T>(grad_xyz), work, mp<T>(grad_lengths), mp<T>(grad_angles),
                                      mp<T>(grad_dihedrals), batch, static_cast<int>(points),
                                      static_cast<int>(segment_steps), st, anchor_work);
      if (r != CUFK_OK) return r;
    }
    return anchor_grads_typed<T>(anchor_work, batch, cp<T>(first_direction), cp<T>(initial_normal), mp<T>(grad_p0),
                                 mp<T>(grad_first_direction), mp<T>(grad_initial_normal), st);
  });
}

int cufk_max_steps(int dtype, int direction, int device) {
  if (!valid_dtype(dtype)) return -CUFK_ERR_DTYPE;
  if (direction != CUFK_FORWARD && direction != CUFK_BACKWARD) return -CUFK_ERR_DIRECTION;
  if (!cufk_amd::device_supported(device)) return -CUFK_ERR_DEVICE;
  return CUFK_MAX_STEPS;
}

const char* cufk_error_string(int status) {
  switch (status) {
    case CUFK_OK: return "success";
    case CUFK_ERR_DTYPE: return "unsupported dtype";
    case CUFK_ERR_POINTS: return "point_count must be >= 4";
    case CUFK_ERR_SHAPE: return "shape exceeds int32 kernel limits";
    case CUFK_ERR_STEPS: return "too many local transforms";
    case CUFK_ERR_NULL: return "null pointer argument";
    case CUFK_ERR_STRIDE: return "negative row stride, or gradient row stride shorter than the row";
    case CUFK_ERR_LAUNCH: return "kernel launch failed";
    case CUFK_ERR_DEVICE: return "device query failed";
    case CUFK_ERR_SEGMENT: return "segment length must be in [1, 2048] local transforms";
    case CUFK_ERR_SCRATCH: return "batch exceeds the 65536 chains of the allocation-free entry point's static scratch";
    case CUFK_ERR_LOSS: return "unknown or unsupported loss kind";
    case CUFK_ERR_DIRECTION: return "direction must be CUFK_FORWARD or CUFK_BACKWARD";
    default: return "unknown status";
  }
}

const char* cufk_version(void) { return "0.1.0"; }

}  // extern "C"
