// PyTorch-ROCm extension cufk_amd._C: autograd wrappers and input validation over the C ABI
// of libcufk_hip.so.  Mirrors the reference's C++ layer (paths under src/cufk/csrc/):
//   ReconstructAutograd + apply      block.cu:367-445
//   TorsionAutograd + apply          torsion.cu:413-447
//   validation messages              extension_utils.cuh:57-130
// All device work goes through cufk_* entry points on the current HIP stream of the
// input's device; nothing here launches kernels itself.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <array>
#include <cstdint>
#include <string>
#include <vector>

#include "cufk_hip.h"

namespace {

using torch::Tensor;
using TensorList = std::vector<Tensor>;

bool supported_dtype(torch::ScalarType t) {
  return t == torch::kFloat32 || t == torch::kFloat64 || t == torch::kFloat16 || t == torch::kBFloat16;
}

// extension_utils.cuh:35-51 dispatch_dtype.
int dtype_code(const Tensor& x) {
  switch (x.scalar_type()) {
    case torch::kFloat32: return CUFK_FLOAT32;
    case torch::kFloat64: return CUFK_FLOAT64;
    case torch::kFloat16: return CUFK_FLOAT16;
    case torch::kBFloat16: return CUFK_BFLOAT16;
    default: break;
  }
  TORCH_CHECK(false, "unsupported dtype");
  return -1;
}

// extension_utils.cuh:57-61.  `device` false skips the device-type check so that the rest of
// the contract can be exercised with host tensors.
void check_cuda_float(const Tensor& x, const char* name, bool device) {
  TORCH_CHECK(!device || x.is_cuda(), name, " must be CUDA");
  TORCH_CHECK(supported_dtype(x.scalar_type()), name, " must be float32, float64, float16, or bfloat16");
  TORCH_CHECK(x.is_contiguous(), name, " must be contiguous");
}

// extension_utils.cuh:63-68.
void check_cuda_float_row_contiguous(const Tensor& x, const char* name, bool device) {
  TORCH_CHECK(!device || x.is_cuda(), name, " must be CUDA");
  TORCH_CHECK(supported_dtype(x.scalar_type()), name, " must be float32, float64, float16, or bfloat16");
  TORCH_CHECK(x.dim() == 2, name, " must have shape (B, K)");
  TORCH_CHECK(x.stride(1) == 1, name, " must have stride(1) == 1");
}

// extension_utils.cuh:70-74.
void check_like(const Tensor& x, const Tensor& ref, const char* name, bool device) {
  check_cuda_float(x, name, device);
  TORCH_CHECK(x.scalar_type() == ref.scalar_type(), name, " must have the same dtype as reference");
  TORCH_CHECK(x.device() == ref.device(), name, " must be on the same device as reference");
}

// extension_utils.cuh:76-82.
void check_anchor(const Tensor& x, const Tensor& ref, const char* name, bool device) {
  TORCH_CHECK(!device || x.is_cuda(), name, " must be CUDA");
  TORCH_CHECK(x.scalar_type() == ref.scalar_type(), name, " must have the same dtype as reference");
  TORCH_CHECK(x.device() == ref.device(), name, " must be on the same device as reference");
  TORCH_CHECK(x.sizes() == torch::IntArrayRef({3}), name, " must have shape (3,)");
  TORCH_CHECK(!x.requires_grad(), name, " gradients are not supported");
}

struct Shape {
  int64_t batch;
  int64_t points;
};

// extension_utils.cuh:119-126.
Shape chain_shape_from_steps(const Tensor& ref, int64_t steps) {
  TORCH_CHECK(ref.size(0) <= INT32_MAX && steps + 3 <= INT32_MAX, "shape exceeds int32 kernel limits");
  TORCH_CHECK(steps >= 1, "point_count must be >= 4");
  return {ref.size(0), steps + 3};
}

// extension_utils.cuh:128-130.
void check_max_local_transforms(int64_t steps, int64_t max_steps, const char* op_name) {
  TORCH_CHECK(steps <= max_steps, op_name, " supports at most ", max_steps, " local transforms");
}

// block.cu:367-378.
Shape check_geom(const Tensor& lengths, const Tensor& angles, const Tensor& dihedrals, bool device) {
  check_cuda_float(lengths, "lengths", device);
  check_like(angles, lengths, "angles", device);
  check_like(dihedrals, lengths, "dihedrals", device);
  TORCH_CHECK(lengths.dim() == 2, "lengths must have shape (B, N-1)");
  TORCH_CHECK(angles.dim() == 2, "angles must have shape (B, N-2)");
  TORCH_CHECK(dihedrals.dim() == 2, "dihedrals must have shape (B, N-3)");
  const Shape shape = chain_shape_from_steps(lengths, lengths.size(1) - 2);
  TORCH_CHECK(angles.sizes() == torch::IntArrayRef({shape.batch, shape.points - 2}), "bad angles shape");
  TORCH_CHECK(dihedrals.sizes() == torch::IntArrayRef({shape.batch, shape.points - 3}), "bad dihedrals shape");
  return shape;
}

struct Anchors {
  Tensor p0, first_direction, initial_normal;
};

// extension_utils.cuh:90-103.  With allow_grad the anchors may require grad (the anchored
// autograd below, which has no reference counterpart).
Anchors checked_anchors(const Tensor& p0, const Tensor& fd, const Tensor& n0, const Tensor& ref, bool device,
                        bool allow_grad = false) {
  if (allow_grad) {
    const Tensor d0 = p0.detach(), d1 = fd.detach(), d2 = n0.detach();
    check_anchor(d0, ref, "p0", device);
    check_anchor(d1, ref, "first_direction", device);
    check_anchor(d2, ref, "initial_normal", device);
    return {d0.contiguous(), d1.contiguous(), d2.contiguous()};
  }
  check_anchor(p0, ref, "p0", device);
  check_anchor(fd, ref, "first_direction", device);
  check_anchor(n0, ref, "initial_normal", device);
  return {p0.contiguous(), fd.contiguous(), n0.contiguous()};
}

// The shape of a batch saved by a forward that validated it (check_geom).  Backwards take their
// saved tensors as they are: they cannot change shape, dtype or device after the forward (the
// reference checks them again, block.cu:422-428; only the incoming gradient is new here).
Shape saved_shape(const Tensor& lengths) { return {lengths.size(0), lengths.size(1) + 1}; }

// torsion.cu:413-417.
Shape check_pairs(const Tensor& raw_pairs, bool device) {
  check_cuda_float_row_contiguous(raw_pairs, "raw_pairs", device);
  TORCH_CHECK(raw_pairs.size(1) % 2 == 0, "raw_pairs second dimension must be even");
  return chain_shape_from_steps(raw_pairs, raw_pairs.size(1) / 2);
}

int max_steps(const Tensor& ref, int direction) {
  const int m = cufk_max_steps(dtype_code(ref), direction, ref.get_device());
  TORCH_CHECK(m >= 0, "cufk_max_steps: ", cufk_error_string(-m));
  return m;
}

void* current_stream(const Tensor& ref) { return c10::hip::getCurrentHIPStream(ref.get_device()).stream(); }

// The version counter of an output kept for the backward.  An output made under
// torch.inference_mode() has none (reading it raises), but no backward is ever recorded for
// it either, so any value does.
int64_t saved_version(const Tensor& t) { return t.is_inference() ? 0 : static_cast<int64_t>(t._version()); }

void check_status(int status, const char* what) {
  TORCH_CHECK(status == CUFK_OK, what, " failed: ", cufk_error_string(status));
}

// ------------------------------------------------------------------ reconstruct

class ReconstructAutograd : public torch::autograd::Function<ReconstructAutograd> {
 public:
  static Tensor forward(torch::autograd::AutogradContext* ctx, Tensor lengths, Tensor angles, Tensor dihedrals,
                        Tensor p0, Tensor first_direction, Tensor initial_normal, bool grad) {
    const Shape shape = check_geom(lengths, angles, dihedrals, true);
    const Anchors a = checked_anchors(p0, first_direction, initial_normal, lengths, true);
    const c10::DeviceGuard guard(lengths.device());
    check_max_local_transforms(shape.points - 3, max_steps(lengths, CUFK_FORWARD), "reconstruct");
    Tensor xyz = torch::empty({shape.batch, shape.points, 3}, lengths.options());
    ctx->save_for_backward({lengths, angles, dihedrals, a.p0, a.first_direction, a.initial_normal});
    // grad: the call records a backward (grad mode on and a parameter row requiring grad).
    const bool half = lengths.scalar_type() == torch::kFloat16 || lengths.scalar_type() == torch::kBFloat16;
    const int64_t shadow_floats = half && grad ? cufk_reconstruct_shadow_floats(shape.batch, shape.points) : 0;
    if (shadow_floats > 0) {
      // float16/bfloat16 outputs are too coarse for the position-based adjoint: the forward
      // keeps a float copy of the positions (12 bytes per point until the backward) and the
      // backward runs over it instead of recomputing the chain.
      Tensor positions = torch::empty({shape.batch, shape.points, 3}, lengths.options().dtype(torch::kFloat32));
      Tensor regular = torch::empty({shape.batch}, lengths.options().dtype(torch::kUInt8));
      check_status(cufk_reconstruct_fwd_shadow(dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(),
                                               dihedrals.data_ptr(), a.p0.data_ptr(), a.first_direction.data_ptr(),
                                               a.initial_normal.data_ptr(), xyz.data_ptr(),
                                               static_cast<float*>(positions.data_ptr()),
                                               static_cast<uint8_t*>(regular.data_ptr()), shape.batch, shape.points,
                                               current_stream(lengths)),
                   "cufk_reconstruct_fwd_shadow");
      ctx->saved_data["positions"] = positions;
      ctx->saved_data["regular"] = regular;
      return xyz;
    }
    Tensor regular = torch::empty({shape.batch}, lengths.options().dtype(torch::kUInt8));
    check_status(cufk_reconstruct_fwd_flagged(dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(),
                                              dihedrals.data_ptr(), a.p0.data_ptr(), a.first_direction.data_ptr(),
                                              a.initial_normal.data_ptr(), xyz.data_ptr(),
                                              static_cast<uint8_t*>(regular.data_ptr()), shape.batch, shape.points,
                                              current_stream(lengths)),
                 "cufk_reconstruct_fwd_flagged");
    // The reference saves only the inputs (block.cu:408).  The output is kept as a detached
    // alias (no grad_fn, so no reference cycle; it shares the output's version counter): when
    // it is untouched at backward time, regular chains use the position-based adjoint;
    // if the caller modified it in place, every chain takes the exact recompute.
    ctx->saved_data["xyz"] = xyz.detach();
    ctx->saved_data["xyz_version"] = saved_version(xyz);
    ctx->saved_data["regular"] = regular;
    return xyz;
  }

  static torch::autograd::tensor_list backward(torch::autograd::AutogradContext* ctx,
                                               torch::autograd::tensor_list grad_outputs) {
    const auto saved = ctx->get_saved_variables();
    const Tensor& lengths = saved[0];
    const Tensor& angles = saved[1];
    const Tensor& dihedrals = saved[2];
    Tensor grad_points = grad_outputs[0].is_contiguous() ? grad_outputs[0] : grad_outputs[0].contiguous();
    check_like(grad_points, lengths, "grad_points", true);
    const Shape shape = saved_shape(lengths);
    const Anchors a{saved[3], saved[4], saved[5]};
    const c10::DeviceGuard guard(lengths.device());
    const int64_t steps = shape.points - 3;
    const int64_t limit = max_steps(lengths, CUFK_BACKWARD);
    // block.cu:335-345 (this build has no shared-memory cap below the plan cap).
    TORCH_CHECK(steps <= limit, "backward supports at most ", limit, " local transforms for this dtype/device, got ", steps,
                " (plan cap ", limit, ", shared-memory cap ", limit, ")");
    Tensor grad_lengths = torch::empty_like(lengths);
    Tensor grad_angles = torch::empty_like(angles);
    Tensor grad_dihedrals = torch::empty_like(dihedrals);
    const Tensor regular = ctx->saved_data["regular"].toTensor();
    if (ctx->saved_data.count("positions") != 0) {
      const Tensor positions = ctx->saved_data["positions"].toTensor();
      check_status(cufk_reconstruct_bwd_shadow(
                       dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(), dihedrals.data_ptr(), a.p0.data_ptr(),
                       a.first_direction.data_ptr(), a.initial_normal.data_ptr(),
                       static_cast<const float*>(positions.data_ptr()), static_cast<const uint8_t*>(regular.data_ptr()),
                       grad_points.data_ptr(), grad_lengths.data_ptr(), grad_angles.data_ptr(),
                       grad_dihedrals.data_ptr(), shape.batch, shape.points, current_stream(lengths)),
                   "cufk_reconstruct_bwd_shadow");
      return {grad_lengths, grad_angles, grad_dihedrals, Tensor(), Tensor(), Tensor(), Tensor()};
    }
    const Tensor xyz = ctx->saved_data["xyz"].toTensor();
    if (xyz._version() == ctx->saved_data["xyz_version"].toInt()) {
      check_status(cufk_reconstruct_bwd_saved(
                       dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(), dihedrals.data_ptr(), a.p0.data_ptr(),
                       a.first_direction.data_ptr(), a.initial_normal.data_ptr(), xyz.data_ptr(),
                       static_cast<const uint8_t*>(regular.data_ptr()), grad_points.data_ptr(), grad_lengths.data_ptr(),
                       grad_angles.data_ptr(), grad_dihedrals.data_ptr(), shape.batch, shape.points,
                       current_stream(lengths)),
                   "cufk_reconstruct_bwd_saved");
    } else {
      check_status(cufk_reconstruct_bwd(dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(), dihedrals.data_ptr(),
                                        a.p0.data_ptr(), a.first_direction.data_ptr(), a.initial_normal.data_ptr(),
                                        grad_points.data_ptr(), grad_lengths.data_ptr(), grad_angles.data_ptr(),
                                        grad_dihedrals.data_ptr(), shape.batch, shape.points, current_stream(lengths)),
                   "cufk_reconstruct_bwd");
    }
    return {grad_lengths, grad_angles, grad_dihedrals, Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

Tensor apply_reconstruct(const Tensor& lengths, const Tensor& angles, const Tensor& dihedrals, const Tensor& p0,
                         const Tensor& first_direction, const Tensor& initial_normal) {
  const bool grad = torch::GradMode::is_enabled() &&
                    (lengths.requires_grad() || angles.requires_grad() || dihedrals.requires_grad());
  return ReconstructAutograd::apply(lengths, angles, dihedrals, p0, first_direction, initial_normal, grad);
}

// ------------------------------------------------------------------ anchor gradients

// ReconstructAutograd with gradients for the anchors as well (no reference counterpart).
class AnchoredAutograd : public torch::autograd::Function<AnchoredAutograd> {
 public:
  static Tensor forward(torch::autograd::AutogradContext* ctx, Tensor lengths, Tensor angles, Tensor dihedrals,
                        Tensor p0, Tensor first_direction, Tensor initial_normal) {
    const Shape shape = check_geom(lengths, angles, dihedrals, true);
    const Anchors a = checked_anchors(p0, first_direction, initial_normal, lengths, true, true);
    const c10::DeviceGuard guard(lengths.device());
    check_max_local_transforms(shape.points - 3, max_steps(lengths, CUFK_FORWARD), "reconstruct");
    Tensor xyz = torch::empty({shape.batch, shape.points, 3}, lengths.options());
    Tensor regular = torch::empty({shape.batch}, lengths.options().dtype(torch::kUInt8));
    check_status(cufk_reconstruct_fwd_flagged(dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(),
                                              dihedrals.data_ptr(), a.p0.data_ptr(), a.first_direction.data_ptr(),
                                              a.initial_normal.data_ptr(), xyz.data_ptr(),
                                              static_cast<uint8_t*>(regular.data_ptr()), shape.batch, shape.points,
                                              current_stream(lengths)),
                 "cufk_reconstruct_fwd_flagged");
    ctx->save_for_backward({lengths, angles, dihedrals, a.p0, a.first_direction, a.initial_normal});
    ctx->saved_data["xyz"] = xyz.detach();
    ctx->saved_data["xyz_version"] = saved_version(xyz);
    ctx->saved_data["regular"] = regular;
    return xyz;
  }

  static torch::autograd::tensor_list backward(torch::autograd::AutogradContext* ctx,
                                               torch::autograd::tensor_list grad_outputs) {
    const auto saved = ctx->get_saved_variables();
    const Tensor& lengths = saved[0];
    const Tensor& angles = saved[1];
    const Tensor& dihedrals = saved[2];
    Tensor grad_points = grad_outputs[0].is_contiguous() ? grad_outputs[0] : grad_outputs[0].contiguous();
    check_like(grad_points, lengths, "grad_points", true);
    const Shape shape = saved_shape(lengths);
    const Anchors a{saved[3], saved[4], saved[5]};
    const c10::DeviceGuard guard(lengths.device());
    Tensor grad_lengths = torch::empty_like(lengths);
    Tensor grad_angles = torch::empty_like(angles);
    Tensor grad_dihedrals = torch::empty_like(dihedrals);
    Tensor grad_p0 = torch::empty({3}, lengths.options());
    Tensor grad_fd = torch::empty({3}, lengths.options());
    Tensor grad_n0 = torch::empty({3}, lengths.options());
    Tensor work = torch::empty({std::max<int64_t>(shape.batch, 1) * 6}, lengths.options().dtype(torch::kFloat64));
    const Tensor xyz = ctx->saved_data["xyz"].toTensor();
    const Tensor regular = ctx->saved_data["regular"].toTensor();
    const bool unmodified = xyz._version() == ctx->saved_data["xyz_version"].toInt();
    check_status(cufk_reconstruct_bwd_anchored(
                     dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(), dihedrals.data_ptr(), a.p0.data_ptr(),
                     a.first_direction.data_ptr(), a.initial_normal.data_ptr(), unmodified ? xyz.data_ptr() : nullptr,
                     unmodified ? static_cast<const uint8_t*>(regular.data_ptr()) : nullptr, grad_points.data_ptr(),
                     grad_lengths.data_ptr(), grad_angles.data_ptr(), grad_dihedrals.data_ptr(),
                     static_cast<double*>(work.data_ptr()), grad_p0.data_ptr(), grad_fd.data_ptr(), grad_n0.data_ptr(),
                     shape.batch, shape.points, current_stream(lengths)),
                 "cufk_reconstruct_bwd_anchored");
    return {grad_lengths, grad_angles, grad_dihedrals, grad_p0, grad_fd, grad_n0};
  }
};

Tensor apply_anchored(const Tensor& lengths, const Tensor& angles, const Tensor& dihedrals, const Tensor& p0,
                      const Tensor& first_direction, const Tensor& initial_normal) {
  return AnchoredAutograd::apply(lengths, angles, dihedrals, p0, first_direction, initial_normal);
}

// ------------------------------------------------------------------ fused coordinate loss

// loss[b] = sum_i |x_bi - target_bi|^2 with the reconstruction fused in (no reference
// counterpart).  Gradients flow to lengths, angles and dihedrals; not to the target or anchors.
class LossAutograd : public torch::autograd::Function<LossAutograd> {
 public:
  static Tensor forward(torch::autograd::AutogradContext* ctx, Tensor lengths, Tensor angles, Tensor dihedrals,
                        Tensor target, Tensor p0, Tensor first_direction, Tensor initial_normal, bool anchored) {
    const Shape shape = check_geom(lengths, angles, dihedrals, true);
    const Anchors a = checked_anchors(p0, first_direction, initial_normal, lengths, true, anchored);
    check_like(target, lengths, "target", true);
    TORCH_CHECK(target.sizes() == torch::IntArrayRef({shape.batch, shape.points, 3}), "target must have shape (B, N, 3)");
    TORCH_CHECK(!target.requires_grad(), "target gradients are not supported");
    const c10::DeviceGuard guard(lengths.device());
    check_max_local_transforms(shape.points - 3, max_steps(lengths, CUFK_FORWARD), "reconstruct");
    ctx->saved_data["anchored"] = anchored;
    Tensor loss = torch::empty({shape.batch}, lengths.options());
    Tensor xyz = torch::empty({shape.batch, shape.points, 3}, lengths.options());
    Tensor regular = torch::empty({shape.batch}, lengths.options().dtype(torch::kUInt8));
    check_status(cufk_reconstruct_loss_fwd(dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(),
                                           dihedrals.data_ptr(), a.p0.data_ptr(), a.first_direction.data_ptr(),
                                           a.initial_normal.data_ptr(), target.data_ptr(), xyz.data_ptr(),
                                           static_cast<uint8_t*>(regular.data_ptr()), loss.data_ptr(), shape.batch,
                                           shape.points, current_stream(lengths)),
                 "cufk_reconstruct_loss_fwd");
    // The positions stay internal (never returned), so nothing can modify them before backward.
    ctx->save_for_backward({lengths, angles, dihedrals, target, a.p0, a.first_direction, a.initial_normal});
    ctx->saved_data["xyz"] = xyz;
    ctx->saved_data["regular"] = regular;
    return loss;
  }

  static torch::autograd::tensor_list backward(torch::autograd::AutogradContext* ctx,
                                               torch::autograd::tensor_list grad_outputs) {
    const auto saved = ctx->get_saved_variables();
    const Tensor& lengths = saved[0];
    const Tensor& angles = saved[1];
    const Tensor& dihedrals = saved[2];
    const Tensor& target = saved[3];
    const Shape shape = saved_shape(lengths);
    const bool anchored = ctx->saved_data["anchored"].toBool();
    const Anchors a{saved[4], saved[5], saved[6]};
    Tensor grad_loss = grad_outputs[0].is_contiguous() ? grad_outputs[0] : grad_outputs[0].contiguous();
    check_like(grad_loss, lengths, "grad_loss", true);
    const c10::DeviceGuard guard(lengths.device());
    Tensor grad_lengths = torch::empty_like(lengths);
    Tensor grad_angles = torch::empty_like(angles);
    Tensor grad_dihedrals = torch::empty_like(dihedrals);
    const Tensor xyz = ctx->saved_data["xyz"].toTensor();
    const Tensor regular = ctx->saved_data["regular"].toTensor();
    if (anchored) {
      Tensor grad_p0 = torch::empty({3}, lengths.options());
      Tensor grad_fd = torch::empty({3}, lengths.options());
      Tensor grad_n0 = torch::empty({3}, lengths.options());
      Tensor work = torch::empty({std::max<int64_t>(shape.batch, 1) * 6}, lengths.options().dtype(torch::kFloat64));
      check_status(cufk_reconstruct_loss_bwd_anchored(
                       dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(), dihedrals.data_ptr(),
                       a.p0.data_ptr(), a.first_direction.data_ptr(), a.initial_normal.data_ptr(), xyz.data_ptr(),
                       static_cast<const uint8_t*>(regular.data_ptr()), target.data_ptr(), grad_loss.data_ptr(),
                       grad_lengths.data_ptr(), grad_angles.data_ptr(), grad_dihedrals.data_ptr(),
                       static_cast<double*>(work.data_ptr()), grad_p0.data_ptr(), grad_fd.data_ptr(),
                       grad_n0.data_ptr(), shape.batch, shape.points, current_stream(lengths)),
                   "cufk_reconstruct_loss_bwd_anchored");
      return {grad_lengths, grad_angles, grad_dihedrals, Tensor(), grad_p0, grad_fd, grad_n0, Tensor()};
    }
    check_status(cufk_reconstruct_loss_bwd(dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(),
                                           dihedrals.data_ptr(), a.p0.data_ptr(), a.first_direction.data_ptr(),
                                           a.initial_normal.data_ptr(), xyz.data_ptr(),
                                           static_cast<const uint8_t*>(regular.data_ptr()), target.data_ptr(),
                                           grad_loss.data_ptr(),
                                           grad_lengths.data_ptr(), grad_angles.data_ptr(), grad_dihedrals.data_ptr(),
                                           shape.batch, shape.points, current_stream(lengths)),
                 "cufk_reconstruct_loss_bwd");
    return {grad_lengths, grad_angles, grad_dihedrals, Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

Tensor apply_loss(const Tensor& lengths, const Tensor& angles, const Tensor& dihedrals, const Tensor& target,
                  const Tensor& p0, const Tensor& first_direction, const Tensor& initial_normal, bool anchor_grads) {
  return LossAutograd::apply(lengths, angles, dihedrals, target, p0, first_direction, initial_normal, anchor_grads);
}

// ------------------------------------------------------------------ fused superposed loss

// loss[b] = mean squared deviation of the reconstruction from target[b] after optimal
// superposition (kind CUFK_LOSS_MSD), or its square root (CUFK_LOSS_RMSD); no reference
// counterpart.  Gradients flow to lengths, angles and dihedrals.
class SuperposedAutograd : public torch::autograd::Function<SuperposedAutograd> {
 public:
  static Tensor forward(torch::autograd::AutogradContext* ctx, Tensor lengths, Tensor angles, Tensor dihedrals,
                        Tensor target, Tensor p0, Tensor first_direction, Tensor initial_normal, int64_t kind) {
    const Shape shape = check_geom(lengths, angles, dihedrals, true);
    const Anchors a = checked_anchors(p0, first_direction, initial_normal, lengths, true);
    check_like(target, lengths, "target", true);
    TORCH_CHECK(target.sizes() == torch::IntArrayRef({shape.batch, shape.points, 3}), "target must have shape (B, N, 3)");
    TORCH_CHECK(!target.requires_grad(), "target gradients are not supported");
    const c10::DeviceGuard guard(lengths.device());
    check_max_local_transforms(shape.points - 3, max_steps(lengths, CUFK_FORWARD), "reconstruct");
    Tensor loss = torch::empty({shape.batch}, lengths.options());
    Tensor xyz = torch::empty({shape.batch, shape.points, 3}, lengths.options());
    Tensor regular = torch::empty({shape.batch}, lengths.options().dtype(torch::kUInt8));
    Tensor record = torch::empty({shape.batch, CUFK_SUPERPOSITION_DOUBLES}, lengths.options().dtype(torch::kFloat64));
    check_status(cufk_reconstruct_superposed_fwd(dtype_code(lengths), static_cast<int>(kind), lengths.data_ptr(),
                                                 angles.data_ptr(), dihedrals.data_ptr(), a.p0.data_ptr(),
                                                 a.first_direction.data_ptr(), a.initial_normal.data_ptr(),
                                                 target.data_ptr(), xyz.data_ptr(),
                                                 static_cast<uint8_t*>(regular.data_ptr()), loss.data_ptr(),
                                                 static_cast<double*>(record.data_ptr()), shape.batch, shape.points,
                                                 current_stream(lengths)),
                 "cufk_reconstruct_superposed_fwd");
    ctx->save_for_backward({lengths, angles, dihedrals, target, a.p0, a.first_direction, a.initial_normal});
    ctx->saved_data["xyz"] = xyz;
    ctx->saved_data["regular"] = regular;
    ctx->saved_data["record"] = record;
    ctx->saved_data["kind"] = kind;
    return loss;
  }

  static torch::autograd::tensor_list backward(torch::autograd::AutogradContext* ctx,
                                               torch::autograd::tensor_list grad_outputs) {
    const auto saved = ctx->get_saved_variables();
    const Tensor& lengths = saved[0];
    const Tensor& angles = saved[1];
    const Tensor& dihedrals = saved[2];
    const Tensor& target = saved[3];
    const Shape shape = saved_shape(lengths);
    const Anchors a{saved[4], saved[5], saved[6]};
    Tensor grad_loss = grad_outputs[0].is_contiguous() ? grad_outputs[0] : grad_outputs[0].contiguous();
    check_like(grad_loss, lengths, "grad_loss", true);
    const c10::DeviceGuard guard(lengths.device());
    Tensor grad_lengths = torch::empty_like(lengths);
    Tensor grad_angles = torch::empty_like(angles);
    Tensor grad_dihedrals = torch::empty_like(dihedrals);
    const Tensor xyz = ctx->saved_data["xyz"].toTensor();
    const Tensor regular = ctx->saved_data["regular"].toTensor();
    const Tensor record = ctx->saved_data["record"].toTensor();
    check_status(cufk_reconstruct_superposed_bwd(
                     dtype_code(lengths), static_cast<int>(ctx->saved_data["kind"].toInt()), lengths.data_ptr(),
                     angles.data_ptr(), dihedrals.data_ptr(), a.p0.data_ptr(), a.first_direction.data_ptr(),
                     a.initial_normal.data_ptr(), xyz.data_ptr(), static_cast<const uint8_t*>(regular.data_ptr()),
                     target.data_ptr(), static_cast<const double*>(record.data_ptr()), grad_loss.data_ptr(),
                     grad_lengths.data_ptr(), grad_angles.data_ptr(), grad_dihedrals.data_ptr(), shape.batch,
                     shape.points, current_stream(lengths)),
                 "cufk_reconstruct_superposed_bwd");
    return {grad_lengths, grad_angles, grad_dihedrals, Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

Tensor apply_superposed(const Tensor& lengths, const Tensor& angles, const Tensor& dihedrals, const Tensor& target,
                        const Tensor& p0, const Tensor& first_direction, const Tensor& initial_normal, int64_t kind) {
  TORCH_CHECK(kind == CUFK_LOSS_MSD || kind == CUFK_LOSS_RMSD, "unknown superposed loss kind ", kind);
  return SuperposedAutograd::apply(lengths, angles, dihedrals, target, p0, first_direction, initial_normal, kind);
}

// ------------------------------------------------------------------ long chains

// Segmented reconstruction without the 2048-step cap (no reference counterpart: its README:58
// leaves long chains to a separate repository).  Same inputs, validation and gradients as
// ReconstructAutograd; segment_steps 0 picks the library default.
int64_t long_segment_steps(const Shape& shape, int64_t requested) {
  const int64_t s = requested > 0 ? requested : cufk_long_segment_steps(shape.batch, shape.points);
  TORCH_CHECK(s >= 1 && s <= 2048, "segment_steps must be in [1, 2048], got ", s);
  return s;
}

Tensor long_buffer(int64_t doubles, const Tensor& ref) {
  TORCH_CHECK(doubles >= 0, "shape exceeds int32 kernel limits");
  return torch::empty({doubles}, ref.options().dtype(torch::kFloat64));
}

void long_forward(const Tensor& lengths, const Tensor& angles, const Tensor& dihedrals, const Anchors& a,
                  const Shape& shape, int64_t seg, const Tensor& xyz, const Tensor& state) {
  check_status(cufk_reconstruct_long_fwd(dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(),
                                         dihedrals.data_ptr(), a.p0.data_ptr(), a.first_direction.data_ptr(),
                                         a.initial_normal.data_ptr(), xyz.data_ptr(),
                                         static_cast<double*>(state.data_ptr()), shape.batch, shape.points, seg,
                                         current_stream(lengths)),
               "cufk_reconstruct_long_fwd");
}

class LongReconstructAutograd : public torch::autograd::Function<LongReconstructAutograd> {
 public:
  static Tensor forward(torch::autograd::AutogradContext* ctx, Tensor lengths, Tensor angles, Tensor dihedrals,
                        Tensor p0, Tensor first_direction, Tensor initial_normal, int64_t segment_steps,
                        bool anchored) {
    const Shape shape = check_geom(lengths, angles, dihedrals, true);
    const Anchors a = checked_anchors(p0, first_direction, initial_normal, lengths, true, anchored);
    ctx->saved_data["anchored"] = anchored;
    const c10::DeviceGuard guard(lengths.device());
    const int64_t seg = long_segment_steps(shape, segment_steps);
    Tensor xyz = torch::empty({shape.batch, shape.points, 3}, lengths.options());
    Tensor state = long_buffer(cufk_long_state_doubles(shape.batch, shape.points, seg), lengths);
    long_forward(lengths, angles, dihedrals, a, shape, seg, xyz, state);
    // As in ReconstructAutograd: the output is kept as a detached alias with its version; if
    // the caller modified it in place, the backward recomputes it.
    ctx->save_for_backward({lengths, angles, dihedrals, a.p0, a.first_direction, a.initial_normal});
    ctx->saved_data["xyz"] = xyz.detach();
    ctx->saved_data["xyz_version"] = saved_version(xyz);
    ctx->saved_data["state"] = state;
    ctx->saved_data["segment_steps"] = seg;
    return xyz;
  }

  static torch::autograd::tensor_list backward(torch::autograd::AutogradContext* ctx,
                                               torch::autograd::tensor_list grad_outputs) {
    const auto saved = ctx->get_saved_variables();
    const Tensor& lengths = saved[0];
    const Tensor& angles = saved[1];
    const Tensor& dihedrals = saved[2];
    Tensor grad_points = grad_outputs[0].is_contiguous() ? grad_outputs[0] : grad_outputs[0].contiguous();
    check_like(grad_points, lengths, "grad_points", true);
    const Shape shape = saved_shape(lengths);
    const bool anchored = ctx->saved_data["anchored"].toBool();
    const Anchors a{saved[3], saved[4], saved[5]};
    const c10::DeviceGuard guard(lengths.device());
    const int64_t seg = ctx->saved_data["segment_steps"].toInt();
    Tensor xyz = ctx->saved_data["xyz"].toTensor();
    Tensor state = ctx->saved_data["state"].toTensor();
    if (xyz._version() != ctx->saved_data["xyz_version"].toInt()) {
      xyz = torch::empty_like(xyz);
      state = torch::empty_like(state);
      long_forward(lengths, angles, dihedrals, a, shape, seg, xyz, state);
    }
    Tensor work = long_buffer(cufk_long_work_doubles(shape.batch, shape.points, seg), lengths);
    Tensor grad_lengths = torch::empty_like(lengths);
    Tensor grad_angles = torch::empty_like(angles);
    Tensor grad_dihedrals = torch::empty_like(dihedrals);
    if (anchored) {
      Tensor grad_p0 = torch::empty({3}, lengths.options());
      Tensor grad_fd = torch::empty({3}, lengths.options());
      Tensor grad_n0 = torch::empty({3}, lengths.options());
      Tensor anchor_work =
          torch::empty({std::max<int64_t>(shape.batch, 1) * 6}, lengths.options().dtype(torch::kFloat64));
      check_status(cufk_reconstruct_long_bwd_anchored(
                       dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(), dihedrals.data_ptr(),
                       a.p0.data_ptr(), a.first_direction.data_ptr(), a.initial_normal.data_ptr(), xyz.data_ptr(),
                       static_cast<const double*>(state.data_ptr()), grad_points.data_ptr(),
                       static_cast<double*>(work.data_ptr()), grad_lengths.data_ptr(), grad_angles.data_ptr(),
                       grad_dihedrals.data_ptr(), static_cast<double*>(anchor_work.data_ptr()), grad_p0.data_ptr(),
                       grad_fd.data_ptr(), grad_n0.data_ptr(), shape.batch, shape.points, seg,
                       current_stream(lengths)),
                   "cufk_reconstruct_long_bwd_anchored");
      return {grad_lengths, grad_angles, grad_dihedrals, grad_p0, grad_fd, grad_n0, Tensor(), Tensor()};
    }
    check_status(cufk_reconstruct_long_bwd(dtype_code(lengths), lengths.data_ptr(), angles.data_ptr(),
                                           dihedrals.data_ptr(), a.p0.data_ptr(), a.first_direction.data_ptr(),
                                           a.initial_normal.data_ptr(), xyz.data_ptr(),
                                           static_cast<const double*>(state.data_ptr()), grad_points.data_ptr(),
                                           static_cast<double*>(work.data_ptr()), grad_lengths.data_ptr(),
                                           grad_angles.data_ptr(), grad_dihedrals.data_ptr(), shape.batch,
                                           shape.points, seg, current_stream(lengths)),
                 "cufk_reconstruct_long_bwd");
    return {grad_lengths, grad_angles, grad_dihedrals, Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

Tensor apply_reconstruct_long(const Tensor& lengths, const Tensor& angles, const Tensor& dihedrals, const Tensor& p0,
                              const Tensor& first_direction, const Tensor& initial_normal, int64_t segment_steps,
                              bool anchor_grads) {
  return LongReconstructAutograd::apply(lengths, angles, dihedrals, p0, first_direction, initial_normal,
                                        segment_steps, anchor_grads);
}

// ------------------------------------------------------------------ torsion

// The raw-pair gradient keeps the input's strides (torsion.cu:401, empty_strided_like), unless
// the input's rows overlap (a row stride shorter than the row, as an unfold or as_strided view
// can give): gradient rows laid out that way would overlap too, so it is dense instead.
Tensor pair_gradient_like(const Tensor& raw_pairs) {
  if (raw_pairs.size(0) > 1 && raw_pairs.stride(0) < raw_pairs.size(1))
    return torch::empty(raw_pairs.sizes(), raw_pairs.options());
  return torch::empty_strided(raw_pairs.sizes(), raw_pairs.strides(), raw_pairs.options());
}

cufk_torsion_consts consts_from(const std::vector<double>& packed) {
  cufk_torsion_consts c;
  for (int i = 0; i < 3; ++i) {
    c.length[i] = static_cast<float>(packed[i]);
    c.sin[i] = packed[3 + i];
    c.cos[i] = packed[6 + i];
  }
  return c;
}

class TorsionAutograd : public torch::autograd::Function<TorsionAutograd> {
 public:
  static Tensor forward(torch::autograd::AutogradContext* ctx, Tensor raw_pairs, std::vector<double> packed) {
    const Shape shape = check_pairs(raw_pairs, true);
    const c10::DeviceGuard guard(raw_pairs.device());
    check_max_local_transforms(shape.points - 3, max_steps(raw_pairs, CUFK_FORWARD), "torsion_pairs");
    const cufk_torsion_consts c = consts_from(packed);
    Tensor xyz = torch::empty({shape.batch, shape.points, 3}, raw_pairs.options());
    check_status(cufk_torsion_fwd(dtype_code(raw_pairs), raw_pairs.data_ptr(), raw_pairs.stride(0), &c, xyz.data_ptr(),
                                  shape.batch, shape.points, current_stream(raw_pairs)),
                 "cufk_torsion_fwd");
    ctx->save_for_backward({raw_pairs, xyz});
    ctx->saved_data["consts"] = c10::List<double>(packed);
    return xyz;
  }

  static torch::autograd::tensor_list backward(torch::autograd::AutogradContext* ctx,
                                               torch::autograd::tensor_list grad_outputs) {
    const auto saved = ctx->get_saved_variables();
    const Tensor& raw_pairs = saved[0];
    const Tensor& xyz = saved[1];
    Tensor grad_points = grad_outputs[0].is_contiguous() ? grad_outputs[0] : grad_outputs[0].contiguous();
    check_like(grad_points, raw_pairs, "grad_points", true);
    const Shape shape = Shape{raw_pairs.size(0), raw_pairs.size(1) / 2 + 3};
    const c10::DeviceGuard guard(raw_pairs.device());
    check_max_local_transforms(shape.points - 3, max_steps(raw_pairs, CUFK_FORWARD), "torsion_pairs");
    const auto list = ctx->saved_data["consts"].toDoubleList();
    const cufk_torsion_consts c = consts_from(std::vector<double>(list.begin(), list.end()));
    // extension_utils.cuh:162-164: the gradient keeps the raw tensor's strides.
    Tensor grad = pair_gradient_like(raw_pairs);
    check_status(cufk_torsion_bwd(dtype_code(raw_pairs), raw_pairs.data_ptr(), raw_pairs.stride(0), xyz.data_ptr(),
                                  grad_points.data_ptr(), grad.data_ptr(), grad.stride(0), &c, shape.batch, shape.points,
                                  current_stream(raw_pairs)),
                 "cufk_torsion_bwd");
    return {grad, Tensor()};
  }
};

// The torsion path with a fused loss against target (any cufk_loss kind; no reference
// counterpart): the reference's backward (torsion.cu:297-381) consumes a materialised
// grad_xyz, which here is formed inside the kernel from the saved positions and the target.
class TorsionLossAutograd : public torch::autograd::Function<TorsionLossAutograd> {
 public:
  static Tensor forward(torch::autograd::AutogradContext* ctx, Tensor raw_pairs, Tensor target,
                        std::vector<double> packed, int64_t kind) {
    const Shape shape = check_pairs(raw_pairs, true);
    check_like(target, raw_pairs, "target", true);
    TORCH_CHECK(target.sizes() == torch::IntArrayRef({shape.batch, shape.points, 3}), "target must have shape (B, N, 3)");
    TORCH_CHECK(!target.requires_grad(), "target gradients are not supported");
    const c10::DeviceGuard guard(raw_pairs.device());
    check_max_local_transforms(shape.points - 3, max_steps(raw_pairs, CUFK_FORWARD), "torsion_pairs");
    const cufk_torsion_consts c = consts_from(packed);
    Tensor xyz = torch::empty({shape.batch, shape.points, 3}, raw_pairs.options());
    Tensor loss = torch::empty({shape.batch}, raw_pairs.options());
    Tensor record = kind == CUFK_LOSS_SQUARED_DISTANCE
                        ? Tensor()
                        : torch::empty({shape.batch, CUFK_SUPERPOSITION_DOUBLES}, raw_pairs.options().dtype(torch::kFloat64));
    double* rec = record.defined() ? static_cast<double*>(record.data_ptr()) : nullptr;
    check_status(cufk_torsion_loss_fwd(dtype_code(raw_pairs), static_cast<int>(kind), raw_pairs.data_ptr(),
                                       raw_pairs.stride(0), &c, target.data_ptr(), xyz.data_ptr(), loss.data_ptr(), rec,
                                       shape.batch, shape.points, current_stream(raw_pairs)),
                 "cufk_torsion_loss_fwd");
    ctx->save_for_backward({raw_pairs, target});
    ctx->saved_data["xyz"] = xyz;
    if (record.defined()) ctx->saved_data["record"] = record;
    ctx->saved_data["consts"] = c10::List<double>(packed);
    ctx->saved_data["kind"] = kind;
    return loss;
  }

  static torch::autograd::tensor_list backward(torch::autograd::AutogradContext* ctx,
                                               torch::autograd::tensor_list grad_outputs) {
    const auto saved = ctx->get_saved_variables();
    const Tensor& raw_pairs = saved[0];
    const Tensor& target = saved[1];
    Tensor grad_loss = grad_outputs[0].is_contiguous() ? grad_outputs[0] : grad_outputs[0].contiguous();
    check_like(grad_loss, raw_pairs, "grad_loss", true);
    const Shape shape = Shape{raw_pairs.size(0), raw_pairs.size(1) / 2 + 3};
    const c10::DeviceGuard guard(raw_pairs.device());
    const auto list = ctx->saved_data["consts"].toDoubleList();
    const cufk_torsion_consts c = consts_from(std::vector<double>(list.begin(), list.end()));
    const int kind = static_cast<int>(ctx->saved_data["kind"].toInt());
    const Tensor xyz = ctx->saved_data["xyz"].toTensor();
    const double* rec = nullptr;
    if (kind != CUFK_LOSS_SQUARED_DISTANCE) rec = static_cast<const double*>(ctx->saved_data["record"].toTensor().data_ptr());
    // extension_utils.cuh:162-164: the gradient keeps the raw tensor's strides.
    Tensor grad = pair_gradient_like(raw_pairs);
    check_status(cufk_torsion_loss_bwd(dtype_code(raw_pairs), kind, raw_pairs.data_ptr(), raw_pairs.stride(0),
                                       xyz.data_ptr(), target.data_ptr(), rec, grad_loss.data_ptr(), grad.data_ptr(),
                                       grad.stride(0), &c, shape.batch, shape.points, current_stream(raw_pairs)),
                 "cufk_torsion_loss_bwd");
    return {grad, Tensor(), Tensor(), Tensor()};
  }
};

// A compiled torsion reconstructor: the three bond lengths and bond-angle sin/cos fixed at
// construction (torsion.py:89-135 compiles them into a JIT module instead).
class TorsionModule {
 public:
  TorsionModule(const std::vector<double>& lengths, const std::vector<double>& sins, const std::vector<double>& coss) {
    TORCH_CHECK(lengths.size() == 3 && sins.size() == 3 && coss.size() == 3, "torsion constants must have 3 elements");
    packed_.reserve(9);
    for (double v : lengths) packed_.push_back(static_cast<double>(static_cast<float>(v)));
    for (double v : sins) packed_.push_back(v);
    for (double v : coss) packed_.push_back(v);
  }
  Tensor apply(const Tensor& raw_pairs) const { return TorsionAutograd::apply(raw_pairs, packed_); }
  Tensor loss(const Tensor& raw_pairs, const Tensor& target, int64_t kind) const {
    TORCH_CHECK(kind >= CUFK_LOSS_SQUARED_DISTANCE && kind <= CUFK_LOSS_RMSD, "unknown loss kind ", kind);
    return TorsionLossAutograd::apply(raw_pairs, target, packed_, kind);
  }
  std::vector<double> lengths() const { return {packed_[0], packed_[1], packed_[2]}; }
  std::vector<double> sins() const { return {packed_[3], packed_[4], packed_[5]}; }
  std::vector<double> coss() const { return {packed_[6], packed_[7], packed_[8]}; }

 private:
  std::vector<double> packed_;
};

// ------------------------------------------------------------------ host-side contract hooks

std::vector<int64_t> validate_reconstruct(const Tensor& lengths, const Tensor& angles, const Tensor& dihedrals,
                                          const Tensor& p0, const Tensor& first_direction, const Tensor& initial_normal,
                                          bool device) {
  const Shape shape = check_geom(lengths, angles, dihedrals, device);
  checked_anchors(p0, first_direction, initial_normal, lengths, device);
  const int64_t cap = device ? max_steps(lengths, CUFK_FORWARD) : CUFK_MAX_STEPS;
  check_max_local_transforms(shape.points - 3, cap, "reconstruct");
  return {shape.batch, shape.points};
}

void validate_grad_points(const Tensor& grad_points, const Tensor& lengths, bool device) {
  check_like(grad_points, lengths, "grad_points", device);
}

std::vector<int64_t> validate_torsion(const Tensor& raw_pairs, bool device) {
  const Shape shape = check_pairs(raw_pairs, device);
  const int64_t cap = device ? max_steps(raw_pairs, CUFK_FORWARD) : CUFK_MAX_STEPS;
  check_max_local_transforms(shape.points - 3, cap, "torsion_pairs");
  return {shape.batch, shape.points};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("apply", &apply_reconstruct, "reconstruct autograd apply (block.cu:443-445)", py::arg("lengths"),
        py::arg("angles"), py::arg("dihedrals"), py::arg("p0"), py::arg("first_direction"), py::arg("initial_normal"));
  m.def("apply_anchored", &apply_anchored, "reconstruct with anchor gradients", py::arg("lengths"), py::arg("angles"),
        py::arg("dihedrals"), py::arg("p0"), py::arg("first_direction"), py::arg("initial_normal"));
  m.def("apply_loss", &apply_loss, "fused reconstruct + per-chain coordinate loss", py::arg("lengths"),
        py::arg("angles"), py::arg("dihedrals"), py::arg("target"), py::arg("p0"), py::arg("first_direction"),
        py::arg("initial_normal"), py::arg("anchor_grads") = false);
  m.def("apply_superposed", &apply_superposed, "fused reconstruct + per-chain superposed loss (1 msd, 2 rmsd)",
        py::arg("lengths"), py::arg("angles"), py::arg("dihedrals"), py::arg("target"), py::arg("p0"),
        py::arg("first_direction"), py::arg("initial_normal"), py::arg("kind"));
  m.def("apply_long", &apply_reconstruct_long, "segmented reconstruct for chains of any length", py::arg("lengths"),
        py::arg("angles"), py::arg("dihedrals"), py::arg("p0"), py::arg("first_direction"), py::arg("initial_normal"),
        py::arg("segment_steps") = 0, py::arg("anchor_grads") = false);
  m.def("long_segment_steps", [](int64_t batch, int64_t points) { return cufk_long_segment_steps(batch, points); });
  py::class_<TorsionModule>(m, "TorsionModule")
      .def(py::init<const std::vector<double>&, const std::vector<double>&, const std::vector<double>&>(),
           py::arg("lengths"), py::arg("sin"), py::arg("cos"))
      .def("apply", &TorsionModule::apply, "torsion-only autograd apply (torsion.cu:445-447)", py::arg("raw_pairs"))
      .def("__call__", &TorsionModule::apply, py::arg("raw_pairs"))
      .def("loss", &TorsionModule::loss, "torsion path with a fused loss (0 squared distance, 1 msd, 2 rmsd)",
           py::arg("raw_pairs"), py::arg("target"), py::arg("kind"))
      .def_property_readonly("lengths", &TorsionModule::lengths)
      .def_property_readonly("sin", &TorsionModule::sins)
      .def_property_readonly("cos", &TorsionModule::coss);
  m.def("validate_reconstruct", &validate_reconstruct, py::arg("lengths"), py::arg("angles"), py::arg("dihedrals"),
        py::arg("p0"), py::arg("first_direction"), py::arg("initial_normal"), py::arg("device") = true);
  m.def("validate_grad_points", &validate_grad_points, py::arg("grad_points"), py::arg("lengths"),
        py::arg("device") = true);
  m.def("validate_torsion", &validate_torsion, py::arg("raw_pairs"), py::arg("device") = true);
  m.def("max_steps", [](int dtype, int direction, int device) { return cufk_max_steps(dtype, direction, device); });
  m.def("library_version", []() { return std::string(cufk_version()); });
}
