/*
 * cufk_hip.h -- C ABI of the MI355X (gfx950) NeRF chain-reconstruction library.
 *
 * Plain device pointers and sizes; no torch types.  Every entry point enqueues work on
 * `stream` (a hipStream_t passed as void*; NULL = the default stream) and returns a status
 * code without synchronising.  Tensors are dense row-major: chain b of an (B, K) array
 * starts at element b*K, except torsion raw pairs whose row stride is explicit.
 *
 * Reference entry points replaced (paths under the reference tree src/cufk/):
 *   cufk._C.apply forward        csrc/block.cu:319-329 (forward_cuda_impl), 393-410
 *   cufk._C.apply backward       csrc/block.cu:331-365 (backward_cuda_impl), 412-428
 *   torsion module apply fwd     csrc/torsion.cu:387-397 (forward_default_impl), 421-426
 *   torsion module apply bwd     csrc/torsion.cu:399-411 (backward_xyz_impl), 428-436
 *   step caps                    csrc/block.cu:88, 334-345; csrc/extension_utils.cuh:128-130,190-199
 */
#ifndef CUFK_HIP_H
#define CUFK_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (csrc/extension_utils.cuh:35-51 dispatch_dtype). */
enum cufk_dtype {
  CUFK_FLOAT32 = 0,
  CUFK_FLOAT64 = 1,
  CUFK_FLOAT16 = 2,
  CUFK_BFLOAT16 = 3
};

/* Status codes. */
enum cufk_status {
  CUFK_OK = 0,
  CUFK_ERR_DTYPE = 1,       /* "unsupported dtype" (extension_utils.cuh:49) */
  CUFK_ERR_POINTS = 2,      /* "point_count must be >= 4" (extension_utils.cuh:121) */
  CUFK_ERR_SHAPE = 3,       /* "shape exceeds int32 kernel limits" (extension_utils.cuh:120) */
  CUFK_ERR_STEPS = 4,       /* more local transforms than the step cap (extension_utils.cuh:128-130) */
  CUFK_ERR_NULL = 5,        /* a required pointer is NULL while B > 0 */
  CUFK_ERR_STRIDE = 6,      /* negative raw-pair row stride, or (B > 1) a raw-pair gradient row stride shorter
                             * than the row, which would make gradient rows overlap */
  CUFK_ERR_LAUNCH = 7,      /* kernel launch failed (C10_CUDA_KERNEL_LAUNCH_CHECK, block.cu:327) */
  CUFK_ERR_DEVICE = 8,      /* device query failed */
  CUFK_ERR_SEGMENT = 9,     /* long-chain segment length outside [1, 2048] */
  CUFK_ERR_SCRATCH = 10,    /* batch larger than the static scratch of an allocation-free entry point */
  CUFK_ERR_LOSS = 11,       /* unknown or unsupported loss kind */
  CUFK_ERR_DIRECTION = 12   /* cufk_max_steps: direction is neither CUFK_FORWARD nor CUFK_BACKWARD */
};

/* Fused loss kinds (cufk_torsion_loss_*, cufk_reconstruct_superposed_*). */
enum cufk_loss {
  CUFK_LOSS_SQUARED_DISTANCE = 0, /* sum_i |x_i - t_i|^2 */
  CUFK_LOSS_MSD = 1,              /* mean squared deviation after optimal superposition */
  CUFK_LOSS_RMSD = 2              /* its square root: the RMSD */
};
/* Doubles per chain of a superposition record: the optimal rotation's transpose (row-major),
 * xbar - R^T tbar, and the mean squared deviation (the rest is working space); written by the
 * forward, read by the backward. */
#define CUFK_SUPERPOSITION_DOUBLES 24

/* Chains per call of cufk_reconstruct_bwd_anchored_noalloc (its static scratch: 6 doubles each). */
#define CUFK_NOALLOC_MAX_CHAINS 65536

/* The step cap (N-3) of every dtype and direction on the architecture the library is built
 * for: what cufk_max_steps returns for a supported device (block.cu:88, torsion.cu:97). */
#define CUFK_MAX_STEPS 2048

/* Direction argument of cufk_max_steps. */
enum cufk_direction { CUFK_FORWARD = 0, CUFK_BACKWARD = 1 };

/*
 * Compiled torsion constants (csrc/torsion.cu:43-53; torsion.py:81-86): bond lengths are
 * float even for float64 chains, bond-angle sin/cos are float64 values.  Step k uses
 * length[(k+2)%3] and angle (k+1)%3 (torsion.cu:67-73).
 */
typedef struct cufk_torsion_consts {
  float length[3];
  double sin[3];
  double cos[3];
} cufk_torsion_consts;

/*
 * Forward reconstruction.  Replaces block.cu:319-329 (forward_cuda_impl) and its launch of
 * block_forward_kernel (block.cu:157-204).
 *   lengths (B, N-1), angles (B, N-2), dihedrals (B, N-3); anchors p0, first_direction,
 *   initial_normal (3,) each; xyz (B, N, 3) output.  4 <= N <= 2051.
 */
int cufk_reconstruct_fwd(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                         const void* p0, const void* first_direction, const void* initial_normal,
                         void* xyz, int64_t batch, int64_t points, void* stream);

/*
 * Forward reconstruction that also classifies each chain for the position-based backward:
 * chain_regular[b] = 1 when every bond length is positive, every bond angle has sin >= 0.5
 * (float32; 1e-2 for float64), every coordinate lies within 256 (float32; 8192 for float64)
 * shortest bonds of the origin and within 2^29 (float32; 2^250 for float64) of it, and (float32)
 * the shortest bond is at least 2^-20; 0 otherwise
 * and always 0 for float16/bfloat16.  Same inputs and
 * output as cufk_reconstruct_fwd; chain_regular is a (B,) byte array.  No reference counterpart:
 * the reference's forward (block.cu:319-329) saves only the inputs.
 */
int cufk_reconstruct_fwd_flagged(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                 const void* p0, const void* first_direction, const void* initial_normal, void* xyz,
                                 uint8_t* chain_regular, int64_t batch, int64_t points, void* stream);

/*
 * Backward reconstruction: dL/d(lengths, angles, dihedrals) from grad_xyz (B, N, 3).
 * Replaces block.cu:331-365 (backward_cuda_impl) and block_backward_kernel
 * (block.cu:230-313).  The anchors receive no gradient (block.cu:427).  Needs no saved output:
 * each chain's positions are recomputed in the compute precision (float for float16/bfloat16)
 * and the force/moment adjoint runs over them; chains failing the regularity test of
 * cufk_reconstruct_fwd_flagged (applied to those positions) take the exact recompute.
 */
int cufk_reconstruct_bwd(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                         const void* p0, const void* first_direction, const void* initial_normal,
                         const void* grad_xyz, void* grad_lengths, void* grad_angles, void* grad_dihedrals,
                         int64_t batch, int64_t points, void* stream);

/*
 * Backward reconstruction given the forward's own output: chains with chain_regular[b] != 0
 * take the position-based adjoint over xyz (the force/moment form the reference's torsion
 * backward uses, torsion.cu:204-217), the others the exact recompute.  For float16/bfloat16
 * (never flagged) it behaves as cufk_reconstruct_bwd.  xyz and chain_regular must be exactly
 * what cufk_reconstruct_fwd_flagged wrote for these inputs.  Replaces block.cu:331-365 for
 * callers that keep the forward output.
 */
int cufk_reconstruct_bwd_saved(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                               const void* p0, const void* first_direction, const void* initial_normal,
                               const void* xyz, const uint8_t* chain_regular, const void* grad_xyz, void* grad_lengths,
                               void* grad_angles, void* grad_dihedrals, int64_t batch, int64_t points, void* stream);

/*
 * float16/bfloat16 forward and backward over a float copy of the positions.  No reference
 * counterpart: the reference's backward (block.cu:331-365) recomputes from the saved inputs.
 * Half-precision outputs are too coarse for the position-based adjoint that float32 and
 * float64 run over their saved output (cufk_reconstruct_bwd_saved), so cufk_reconstruct_bwd
 * reruns the forward scan for them; these two replace that rerun by a float copy kept by the
 * forward, at 12 bytes per point of extra memory between the two calls.
 *
 * cufk_reconstruct_shadow_floats(batch, points): the number of floats `positions` must hold,
 * batch*points*3, or 0 where the forward packs short chains several per workgroup (batch >=
 * 4096 and points <= 131): there the forward writes neither positions nor chain_regular, the
 * backward recomputes the positions, and both may be NULL.  -1 for invalid shapes.
 *
 * cufk_reconstruct_fwd_shadow: xyz exactly as cufk_reconstruct_fwd writes it, plus the
 * unrounded float positions (B, N, 3) and chain_regular (B,) under the float32 test of
 * cufk_reconstruct_fwd_flagged.  cufk_reconstruct_bwd_shadow: what cufk_reconstruct_bwd
 * computes, from positions and chain_regular as the forward wrote them for the same inputs.
 * Other dtypes: CUFK_ERR_DTYPE.
 */
int64_t cufk_reconstruct_shadow_floats(int64_t batch, int64_t points);
int cufk_reconstruct_fwd_shadow(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                const void* p0, const void* first_direction, const void* initial_normal, void* xyz,
                                float* positions, uint8_t* chain_regular, int64_t batch, int64_t points, void* stream);
int cufk_reconstruct_bwd_shadow(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                const void* p0, const void* first_direction, const void* initial_normal,
                                const float* positions, const uint8_t* chain_regular, const void* grad_xyz,
                                void* grad_lengths, void* grad_angles, void* grad_dihedrals, int64_t batch,
                                int64_t points, void* stream);

/*
 * Torsion-only forward from raw interleaved (sin, cos) pairs, raw row b at
 * raw + b*raw_stride (elements), 2*(N-3) values per row.  xyz (B, N, 3) dense.
 * Replaces torsion.cu:387-397 and forward_kernel (torsion.cu:254-295).
 */
int cufk_torsion_fwd(int dtype, const void* raw_pairs, int64_t raw_stride, const cufk_torsion_consts* consts,
                     void* xyz, int64_t batch, int64_t points, void* stream);

/*
 * Torsion-only backward: grad_raw (row stride grad_raw_stride) from the saved forward xyz
 * and grad_xyz.  Replaces torsion.cu:399-411 and backward_kernel (torsion.cu:297-381).
 */
int cufk_torsion_bwd(int dtype, const void* raw_pairs, int64_t raw_stride, const void* xyz, const void* grad_xyz,
                     void* grad_raw, int64_t grad_raw_stride, const cufk_torsion_consts* consts, int64_t batch,
                     int64_t points, void* stream);

/*
 * Backward with anchor gradients.  No reference counterpart: the reference rejects anchors
 * that require grad (extension_utils.cuh:81, "gradients are not supported").  Computes what
 * cufk_reconstruct_bwd_saved (xyz and chain_regular given) or cufk_reconstruct_bwd (xyz NULL)
 * computes, plus dL/dp0, dL/dfirst_direction, dL/dinitial_normal (3 values each, summed over
 * the batch since the anchors are shared).  anchor_work: 6*B doubles of scratch (per-chain
 * force and torque about p0), no initialisation needed.  The gradients assume
 * |first_direction| >= 1e-6; with initial_normal parallel to first_direction the normal comes
 * from the fixed helper axis and dL/dinitial_normal is 0.
 */
int cufk_reconstruct_bwd_anchored(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                  const void* p0, const void* first_direction, const void* initial_normal,
                                  const void* xyz, const uint8_t* chain_regular, const void* grad_xyz,
                                  void* grad_lengths, void* grad_angles, void* grad_dihedrals, double* anchor_work,
                                  void* grad_p0, void* grad_first_direction, void* grad_initial_normal, int64_t batch,
                                  int64_t points, void* stream);

/*
 * cufk_reconstruct_bwd_anchored without the anchor_work argument: it allocates nothing and
 * takes no workspace, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  No counterpart in the
 * reference.  The per-chain sums live in a static device array of the library, one per GPU,
 * of CUFK_NOALLOC_MAX_CHAINS * 6 doubles (3 MiB, held until the process ends); batch >
 * CUFK_NOALLOC_MAX_CHAINS returns CUFK_ERR_SCRATCH.  Call it with the stream's device current.
 * Every call on one GPU shares that array: calls that overlap in time on one GPU (other
 * streams, other host threads) race and must be serialised by the caller.  Results equal
 * those of cufk_reconstruct_bwd_anchored.
 */
int cufk_reconstruct_bwd_anchored_noalloc(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                          const void* p0, const void* first_direction, const void* initial_normal,
                                          const void* xyz, const uint8_t* chain_regular, const void* grad_xyz,
                                          void* grad_lengths, void* grad_angles, void* grad_dihedrals, void* grad_p0,
                                          void* grad_first_direction, void* grad_initial_normal, int64_t batch,
                                          int64_t points, void* stream);

/*
 * Fused coordinate loss: loss[b] = sum_i |x_bi - target_bi|^2 over the points of chain b, with
 * x the reconstruction of (lengths, angles, dihedrals, anchors); target is (B, N, 3) in the
 * same dtype, loss (B,).  No reference counterpart: the reference reconstructs
 * (block.cu:319-329) and leaves the loss to PyTorch, whose kernels read xyz and the target,
 * write and read back the loss terms and grad_xyz, and hand grad_xyz to its backward
 * (block.cu:331-365).  Here the forward writes xyz and chain_regular as
 * cufk_reconstruct_fwd_flagged does (bit for bit, except for batches of at least 4096 chains of
 * at most 131 points, which that entry point packs several to a wave and this one does not:
 * there they agree within float rounding), plus the loss reduced from the positions in registers;
 * the backward reads xyz and the target and forms grad_xyz = 2 grad_loss[b] (x - target) in
 * LDS, so grad_xyz never exists in memory.  The loss uses the positions as stored (rounded to
 * the dtype).  grad_loss (B,) may be NULL (all ones).  4 <= N <= 2051.
 */
int cufk_reconstruct_loss_fwd(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                              const void* p0, const void* first_direction, const void* initial_normal,
                              const void* target, void* xyz, uint8_t* chain_regular, void* loss, int64_t batch,
                              int64_t points, void* stream);
int cufk_reconstruct_loss_bwd(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                              const void* p0, const void* first_direction, const void* initial_normal, const void* xyz,
                              const uint8_t* chain_regular, const void* target, const void* grad_loss,
                              void* grad_lengths, void* grad_angles, void* grad_dihedrals, int64_t batch,
                              int64_t points, void* stream);

/*
 * cufk_reconstruct_loss_bwd plus the anchors' gradients (summed over the batch), as
 * cufk_reconstruct_bwd_anchored adds them to the backward of reconstruct; anchor_work: 6*B
 * doubles of scratch.  No reference counterpart (extension_utils.cuh:81 rejects anchor grads).
 */
int cufk_reconstruct_loss_bwd_anchored(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                       const void* p0, const void* first_direction, const void* initial_normal,
                                       const void* xyz, const uint8_t* chain_regular, const void* target,
                                       const void* grad_loss, void* grad_lengths, void* grad_angles,
                                       void* grad_dihedrals, double* anchor_work, void* grad_p0,
                                       void* grad_first_direction, void* grad_initial_normal, int64_t batch,
                                       int64_t points, void* stream);

/*
 * Fused superposed losses: loss[b] = min over rotations R of (1/N) sum_i |R (x_i - xbar) -
 * (t_i - tbar)|^2 (CUFK_LOSS_MSD), or its square root (CUFK_LOSS_RMSD), x the reconstruction of
 * (lengths, angles, dihedrals, anchors) as stored (rounded to the dtype) and t = target (B, N, 3).
 * The optimal rotation comes from Horn's quaternion method, solved per chain in double inside the
 * forward; no reference counterpart (the reference leaves losses to PyTorch).  The forward
 * writes xyz and chain_regular as cufk_reconstruct_loss_fwd does, loss (B,) and
 * superposition (B x CUFK_SUPERPOSITION_DOUBLES doubles).  The backward takes them (same
 * loss_kind) with grad_loss (B,) or NULL (ones) and forms grad_xyz = c (x_i - R^T (t_i - tbar) -
 * xbar) per point inside the kernel, c = (2/N) grad_loss[b] (divided by 2 rmsd for the RMSD; 0
 * where rmsd = 0).  4 <= N <= 2051.
 */
int cufk_reconstruct_superposed_fwd(int dtype, int loss_kind, const void* lengths, const void* angles,
                                    const void* dihedrals, const void* p0, const void* first_direction,
                                    const void* initial_normal, const void* target, void* xyz, uint8_t* chain_regular,
                                    void* loss, double* superposition, int64_t batch, int64_t points, void* stream);
int cufk_reconstruct_superposed_bwd(int dtype, int loss_kind, const void* lengths, const void* angles,
                                    const void* dihedrals, const void* p0, const void* first_direction,
                                    const void* initial_normal, const void* xyz, const uint8_t* chain_regular,
                                    const void* target, const double* superposition, const void* grad_loss,
                                    void* grad_lengths, void* grad_angles, void* grad_dihedrals, int64_t batch,
                                    int64_t points, void* stream);

/*
 * Torsion path with a fused loss of any cufk_loss kind against target (B, N, 3).  The forward
 * is cufk_torsion_fwd plus loss (B,) and, for the superposed kinds, superposition (B x
 * CUFK_SUPERPOSITION_DOUBLES; NULL allowed for CUFK_LOSS_SQUARED_DISTANCE).  The backward is
 * cufk_torsion_bwd with grad_xyz formed inside the kernel from the saved xyz and the target
 * (torsion.cu:297-381 consumes a materialised grad_xyz), grad_loss (B,) or NULL (ones).  No
 * reference counterpart.
 */
int cufk_torsion_loss_fwd(int dtype, int loss_kind, const void* raw_pairs, int64_t raw_stride,
                          const cufk_torsion_consts* consts, const void* target, void* xyz, void* loss,
                          double* superposition, int64_t batch, int64_t points, void* stream);
int cufk_torsion_loss_bwd(int dtype, int loss_kind, const void* raw_pairs, int64_t raw_stride, const void* xyz,
                          const void* target, const double* superposition, const void* grad_loss, void* grad_raw,
                          int64_t grad_raw_stride, const cufk_torsion_consts* consts, int64_t batch, int64_t points,
                          void* stream);

/*
 * Long chains (any N >= 4; no step cap).  The reference stops at 2048 local transforms
 * (extension_utils.cuh:128-130) and its README:58 points long chains to a separate repository
 * (coord_scan_repro, not part of it), so these have no reference counterpart; they extend
 * cufk_reconstruct_fwd / _bwd with the same inputs, outputs and conventions.
 *
 * The chain is cut into segments of segment_steps local transforms (1..2048), each scanned by
 * one workgroup, joined by short per-chain passes in double.  The caller provides two float64
 * buffers: `state` (cufk_long_state_doubles elements), written by the forward and read by the
 * backward of the same inputs and segment_steps; and `work` (cufk_long_work_doubles
 * elements), scratch for the backward.  Neither needs initialising.  Besides the per-segment
 * records, `state` holds the local positions of every segment after the first and a flag per
 * segment (the forward's regularity test on its own positions), so it is sized for
 * (batch, points, 3) doubles more.  The backward takes the forward's xyz and state: the
 * position-based adjoint over the local positions in flagged segments (whose predecessor is
 * flagged too), the exact adjoint in the others.
 */
/* Default segment length for (batch, points): 2048, halved (down to 256) while the grid would
 * hold fewer than 1024 segments.  0 for invalid shapes. */
int64_t cufk_long_segment_steps(int64_t batch, int64_t points);
/* Sizes of the state and work buffers in doubles, or -1 for invalid arguments. */
int64_t cufk_long_state_doubles(int64_t batch, int64_t points, int64_t segment_steps);
int64_t cufk_long_work_doubles(int64_t batch, int64_t points, int64_t segment_steps);
int cufk_reconstruct_long_fwd(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                              const void* p0, const void* first_direction, const void* initial_normal, void* xyz,
                              double* state, int64_t batch, int64_t points, int64_t segment_steps, void* stream);
int cufk_reconstruct_long_bwd(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                              const void* p0, const void* first_direction, const void* initial_normal, const void* xyz,
                              const double* state, const void* grad_xyz, double* work, void* grad_lengths,
                              void* grad_angles, void* grad_dihedrals, int64_t batch, int64_t points,
                              int64_t segment_steps, void* stream);

/*
 * cufk_reconstruct_long_bwd plus the anchors' gradients (summed over the batch); anchor_work:
 * 6*B doubles of scratch.  The head segment's adjoint holds each chain's whole force and moment
 * sums and writes them.  No reference counterpart.
 */
int cufk_reconstruct_long_bwd_anchored(int dtype, const void* lengths, const void* angles, const void* dihedrals,
                                       const void* p0, const void* first_direction, const void* initial_normal,
                                       const void* xyz, const double* state, const void* grad_xyz, double* work,
                                       void* grad_lengths, void* grad_angles, void* grad_dihedrals,
                                       double* anchor_work, void* grad_p0, void* grad_first_direction,
                                       void* grad_initial_normal, int64_t batch, int64_t points, int64_t segment_steps,
                                       void* stream);

/*
 * Largest step count (N-3) accepted for (dtype, direction) on `device`, or a negative
 * status: -CUFK_ERR_DTYPE, -CUFK_ERR_DIRECTION, or -CUFK_ERR_DEVICE when `device` is not a
 * present HIP device of the architecture the library is built for (gfx950).  Every kernel's
 * LDS fits that architecture, so the cap is 2048 for each dtype and direction.  Replaces
 * kMaxSteps (block.cu:88, torsion.cu:97) and dynamic_shared_plan_limit
 * (extension_utils.cuh:190-199).
 */
int cufk_max_steps(int dtype, int direction, int device);

/* Static text for a status code. */
const char* cufk_error_string(int status);

/* Library version, "major.minor.patch". */
const char* cufk_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CUFK_HIP_H */
