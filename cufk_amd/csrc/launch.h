// Interface between the C ABI (cufk_hip.hip) and the typed kernel launchers (launchers.hip).
//
// launchers.hip is compiled once per (dtype, kernel family): the device code of the library
// then builds as independent translation units, in parallel.  This header declares the typed
// launchers those units instantiate and the limits the C ABI checks against; it instantiates
// no kernel itself.
#pragma once

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "cufk_hip.h"
#include "reconstruct_kernels.h"  // FastPath
#include "fused_loss.h"           // kLoss*
#include "superpose.h"            // kSuperposeRecord
#include "torsion_kernels.h"      // TorsionArgs

namespace cufk_amd {

constexpr int kMaxSteps = CUFK_MAX_STEPS;  // block.cu:88, torsion.cu:97 (512 threads x 4 items)

// Long chains: per-(chain, segment) state and backward scratch, in doubles.
constexpr int kLongStateDoubles = 24;
constexpr int kLongWorkDoubles = 12;
// Default segment length: the largest plan capacity (2048 steps) unless the grid would then
// hold fewer than ~4 workgroups per CU; halved down to 256 steps until it does.
constexpr int64_t kLongMinSegment = 256;
constexpr int64_t kLongTargetGroups = 1024;
// Grid extents of the long-chain launches count work-items in 32 bits.
constexpr int64_t kLongMaxGroups = int64_t{UINT32_MAX} / 256;

inline int64_t long_segments(int64_t points, int64_t seg_steps) { return (points - 3 + seg_steps - 1) / seg_steps; }
// The state buffer: the per-(chain, segment) records, one flag byte per (chain, segment)
// rounded up to 16 bytes, then the local positions, room for (batch, points, 3) doubles.
inline int64_t long_flag_offset(int64_t batch, int64_t segs) { return batch * segs * kLongStateDoubles; }
inline int64_t long_local_offset(int64_t batch, int64_t segs) {
  return long_flag_offset(batch, segs) + (batch * segs + 15) / 16 * 2;
}
inline int64_t long_state_size(int64_t batch, int64_t points, int64_t segs) {
  return long_local_offset(batch, segs) + batch * points * 3;
}

// Short chains: G lanes per chain, 8 steps per lane, several chains per workgroup (packed
// kernels).  Measured on MI355X against one chain per workgroup: packing wins from about 4096
// chains up (at 8192 chains: forward 9.5-15.5 us against 19-21 us for 9-128 steps), loses
// below (fewer waves in flight), and its backward stops winning past 64 steps (at 128 steps
// and 32768 chains: 44 us against 34 us).
constexpr int kPackedFwdMaxSteps = 128;
constexpr int kPackedBwdMaxSteps = 64;
constexpr int64_t kPackedMinBatch = 4096;
inline bool use_packed_fwd(int64_t B, int64_t steps) { return steps <= kPackedFwdMaxSteps && B >= kPackedMinBatch; }
inline bool use_packed_bwd(int64_t B, int64_t steps) { return steps <= kPackedBwdMaxSteps && B >= kPackedMinBatch; }
// Whether a float16/bfloat16 chain keeps float positions for its backward: wherever the
// forward runs one chain per workgroup, so that the output is the plain forward's, bit for bit.
inline bool use_shadow(int64_t B, int64_t steps) { return !use_packed_fwd(B, steps); }

// ---------------------------------------------------------------------------- typed launchers
// Each returns a cufk_status.  Pointers are device rows of B chains of N points; `anchor`
// (optional) receives each chain's six anchor sums (F, tau) for anchor_grads_typed.

// Forward, one chain per workgroup or packed (short chains, large batches).
template <typename T>
int reconstruct_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz,
                          uint8_t* regular, int64_t B, int N, hipStream_t st);

// Backward without a saved output: the forward scan is rerun per chain.
template <typename T>
int reconstruct_bwd_recompute_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0,
                                    const T* g, T* gL, T* gA, T* gD, int64_t B, int N, hipStream_t st,
                                    double* anchor = nullptr);

// float16/bfloat16 forward that also keeps the positions in float (pos, B*N*3 floats) and the
// chains' regularity flags, and the backward over them (position-based adjoint, exact
// recompute for irregular chains).  Where use_shadow(B, N-3) is false the forward writes
// neither pos nor regular and the backward recomputes the positions.
template <typename T>
int shadow_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz, float* pos,
                     uint8_t* regular, int64_t B, int N, hipStream_t st);
template <typename T>
int shadow_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const float* pos,
                     const uint8_t* regular, const T* g, T* gL, T* gA, T* gD, int64_t B, int N, hipStream_t st);

// Backward over the saved forward output and its regularity flags (float and double only).
template <typename T>
int reconstruct_bwd_saved_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0,
                                const T* xyz, const uint8_t* regular, const T* g, T* gL, T* gA, T* gD, int64_t B, int N,
                                hipStream_t st, double* anchor = nullptr);

// Batch reduction of the anchor sums and the map to the anchor gradients.
template <typename T>
int anchor_grads_typed(const double* anchor, int64_t B, const T* fd, const T* n0, T* grad_p0, T* grad_fd, T* grad_n0,
                       hipStream_t st);

// Short chains packed several per wave (called by the two functions above).
template <typename T>
int packed_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz,
                     uint8_t* regular, int64_t B, int N, hipStream_t st);
template <typename T, bool Saved>
int packed_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* xyz,
                     const uint8_t* regular, const T* g, T* gL, T* gA, T* gD, int64_t B, int N, hipStream_t st,
                     double* anchor = nullptr);

// Fused coordinate loss.
template <typename T>
int loss_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* target, T* xyz,
                   uint8_t* regular, T* loss, int64_t B, int N, hipStream_t st);
template <typename T>
int loss_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* xyz,
                   const uint8_t* regular, const T* target, const T* grad_loss, T* gL, T* gA, T* gD, int64_t B, int N,
                   hipStream_t st, double* anchor = nullptr);

// Fused superposed losses (mean squared deviation after optimal superposition, or its
// square root unless `squared`); record: kSuperposeRecord doubles per chain (superpose.h).
template <typename T>
int superposed_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* target,
                         T* xyz, uint8_t* regular, T* loss, double* record, int squared, int64_t B, int N,
                         hipStream_t st);
template <typename T>
int superposed_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* xyz,
                         const uint8_t* regular, const T* target, const double* record, const T* grad_loss,
                         int squared, T* gL, T* gA, T* gD, int64_t B, int N, hipStream_t st);

// Chains past the single-workgroup cap, in segments of S steps.
template <typename T>
int long_fwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, T* xyz, double* state,
                   int64_t B, int N, int S, hipStream_t st);
template <typename T>
int long_bwd_typed(const T* L, const T* A, const T* D, const T* p0, const T* fd, const T* n0, const T* xyz,
                   const double* state, const T* g, double* work, T* gL, T* gA, T* gD, int64_t B, int N, int S,
                   hipStream_t st, double* anchor = nullptr);

// Torsion path.
template <typename T>
int torsion_fwd_typed(const T* raw, int64_t rs, const TorsionArgs& c, T* xyz, int64_t B, int N, hipStream_t st);
template <typename T>
int torsion_bwd_typed(const T* raw, int64_t rs, const T* xyz, const T* g, T* graw, int64_t gs, const TorsionArgs& c,
                      int64_t B, int N, hipStream_t st);

// Torsion path with a fused loss (kind: kLossSquared or kLossSuperposed, fused_loss.h); the
// backward takes the target in place of grad_xyz.
template <typename T>
int torsion_loss_fwd_typed(int kind, const T* raw, int64_t rs, const TorsionArgs& c, const T* target, T* xyz, T* loss,
                           double* record, int squared, int64_t B, int N, hipStream_t st);
template <typename T>
int torsion_loss_bwd_typed(int kind, const T* raw, int64_t rs, const T* xyz, const T* target, const double* record,
                           const T* grad_loss, int squared, T* graw, int64_t gs, const TorsionArgs& c, int64_t B, int N,
                           hipStream_t st);

}  // namespace cufk_amd
