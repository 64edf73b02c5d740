// Optimal superposition of a chain onto a target (the RMSD losses).
//
// No reference counterpart: the reference leaves losses to PyTorch.  The fused RMSD losses
// need, per chain, the rotation R and the centroids that minimise
//   msd = (1/N) sum_i |R (x_i - xbar) - (t_i - tbar)|^2
// over proper rotations.  It is solved with Horn's quaternion method (B. K. P. Horn, "Closed-
// form solution of absolute orientation using unit quaternions", JOSA A 4(4), 1987): with the
// centred cross-covariance S_ab = sum_i x'_ia t'_ib, the largest eigenvalue lambda of the
// symmetric 4x4 key matrix N(S) equals max_R sum_i t'_i . R x'_i, and its eigenvector is the
// unit quaternion of that R.  So msd = (sum |x'|^2 + sum |t'|^2 - 2 lambda) / N, and since R
// is optimal the gradient is d msd / d x_i = (2/N) ((x_i - xbar) - R^T (t_i - tbar)).
//
// lambda comes from Newton's method on the characteristic polynomial of N, started above the
// largest root (D. L. Theobald, Acta Cryst. A61, 2005: the QCP method), and the quaternion from
// the largest column of the adjugate of N - lambda I, which for a simple eigenvalue is
// proportional to its eigenvector (P. Liu, D. K. Agrafiotis, D. L. Theobald, J. Comput. Chem. 31,
// 2010).  Where that column is small against the matrix's scale (a nearly repeated top
// eigenvalue: the rotation is then nearly undetermined) the eigenpair comes from cyclic Jacobi
// rotations instead.  Everything here is plain C++ usable on the host and the device (CUFK_HD),
// so the host tests can check it directly.
#pragma once

#include <cmath>

#if defined(__HIPCC__)
#define CUFK_HD __host__ __device__
#else
#define CUFK_HD
#endif

namespace cufk_amd {

// Per-chain sums, relative to shift points cx (chain) and ct (target): x' = x - cx, t' = t - ct.
//   [0..2] sum x',  [3..5] sum t',  [6..14] sum x'_a t'_b (row a, column b),
//   [15] sum |x'|^2,  [16] sum |t'|^2.
constexpr int kSuperposeSums = 17;

CUFK_HD inline void superpose_add(double (&s)[kSuperposeSums], const double (&x)[3], const double (&t)[3]) {
  for (int a = 0; a < 3; ++a) {
    s[a] += x[a];
    s[3 + a] += t[a];
    for (int b = 0; b < 3; ++b) s[6 + 3 * a + b] += x[a] * t[b];
  }
  s[15] += x[0] * x[0] + x[1] * x[1] + x[2] * x[2];
  s[16] += t[0] * t[0] + t[1] * t[1] + t[2] * t[2];
}

// A part of the chain summed about its own shift points (xl, tl), moved to the chain's (cx, ct).
// s1 = [sum a, sum b] and s2 = [sum a b^T (row-major), sum |a|^2, sum |b|^2] over its m points,
// a = x - xl, b = t - tl; e = xl - cx, f = tl - ct.  With x - cx = a + e and t - ct = b + f:
//   sum (a + e) = sum a + m e,
//   sum (a + e)(b + f)^T = sum a b^T + (sum a) f^T + e (sum b + m f)^T,
//   sum |a + e|^2 = sum |a|^2 + 2 e . sum a + m |e|^2   (and the same for b, f).
CUFK_HD inline void superpose_move(const double (&s1)[6], const double (&s2)[11], double m, const double (&e)[3],
                                   const double (&f)[3], double (&out)[kSuperposeSums]) {
  double ea = 0.0, fb = 0.0, ee = 0.0, ff = 0.0;
  for (int i = 0; i < 3; ++i) {
    out[i] = s1[i] + m * e[i];
    out[3 + i] = s1[3 + i] + m * f[i];
    ea += e[i] * s1[i];
    fb += f[i] * s1[3 + i];
    ee += e[i] * e[i];
    ff += f[i] * f[i];
  }
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) out[6 + 3 * i + j] = s2[3 * i + j] + s1[i] * f[j] + e[i] * out[3 + j];
  out[15] = s2[9] + 2.0 * ea + m * ee;
  out[16] = s2[10] + 2.0 * fb + m * ff;
}

// A chain's record, 24 doubles.  The fused forward writes the sums (kSuperposeSums) and the
// shift points cx (at 17) and ct (at 20); superpose_solve_record then replaces them with what
// the backward needs:
//   [0..8]  M = R^T (row-major),  [9..11] a = xbar - R^T tbar (world coordinates),
//   [12]    msd,                  [13..23] unused (zero).
// The residual whose gradient the adjoint takes is then (2/N) (x_i - M t_i - a).
constexpr int kSuperposeRecord = 24;

// Largest eigenpair of the symmetric 4x4 matrix A (destroyed) by cyclic Jacobi rotations:
// returns lambda and writes its unit eigenvector to q.
CUFK_HD inline double jacobi4_max(double (&A)[4][4], double (&q)[4]) {
  double V[4][4] = {{1, 0, 0, 0}, {0, 1, 0, 0}, {0, 0, 1, 0}, {0, 0, 0, 1}};
  double scale = 0.0;
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) scale += A[i][j] * A[i][j];
  for (int sweep = 0; sweep < 24; ++sweep) {
    double off = 0.0;
    for (int p = 0; p < 3; ++p)
      for (int r = p + 1; r < 4; ++r) off += A[p][r] * A[p][r];
    if (!(off > 1.0e-30 * scale)) break;  // also ends on NaN
#pragma unroll
    for (int p = 0; p < 3; ++p) {
#pragma unroll
      for (int r = p + 1; r < 4; ++r) {
        const double apr = A[p][r];
        if (apr == 0.0) continue;
        // Rotation J in the (p, r) plane with J^T A J zeroing A[p][r].
        const double theta = (A[r][r] - A[p][p]) / (2.0 * apr);
        const double t = (theta >= 0.0 ? 1.0 : -1.0) / (std::fabs(theta) + std::sqrt(theta * theta + 1.0));
        const double c = 1.0 / std::sqrt(t * t + 1.0);
        const double s = t * c;
        for (int k = 0; k < 4; ++k) {  // columns p, r
          const double akp = A[k][p], akr = A[k][r];
          A[k][p] = c * akp - s * akr;
          A[k][r] = s * akp + c * akr;
        }
        for (int k = 0; k < 4; ++k) {  // rows p, r
          const double apk = A[p][k], ark = A[r][k];
          A[p][k] = c * apk - s * ark;
          A[r][k] = s * apk + c * ark;
        }
        for (int k = 0; k < 4; ++k) {
          const double vkp = V[k][p], vkr = V[k][r];
          V[k][p] = c * vkp - s * vkr;
          V[k][r] = s * vkp + c * vkr;
        }
      }
    }
  }
  double top = A[0][0];
#pragma unroll
  for (int i = 0; i < 4; ++i) q[i] = V[i][0];
#pragma unroll
  for (int j = 1; j < 4; ++j) {
    const bool better = A[j][j] > top;
    top = better ? A[j][j] : top;
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = better ? V[i][j] : q[i];
  }
  return top;
}

// 3x3 minor of the 4x4 matrix A without row r and column c.
// Rows and columns are picked arithmetically (k, or k + 1 past the removed one), so that with
// r and c known at compile time every index folds to a constant and A stays in registers.
CUFK_HD inline double minor3(const double (&A)[4][4], int r, int c) {
  const int r0 = r > 0 ? 0 : 1, r1 = r > 1 ? 1 : 2, r2 = r > 2 ? 2 : 3;
  const int c0 = c > 0 ? 0 : 1, c1 = c > 1 ? 1 : 2, c2 = c > 2 ? 2 : 3;
  return A[r0][c0] * (A[r1][c1] * A[r2][c2] - A[r1][c2] * A[r2][c1]) -
         A[r0][c1] * (A[r1][c0] * A[r2][c2] - A[r1][c2] * A[r2][c0]) +
         A[r0][c2] * (A[r1][c0] * A[r2][c1] - A[r1][c1] * A[r2][c0]);
}

// Largest eigenpair of the symmetric, traceless 4x4 key matrix N (QCP; see the file comment),
// with the Jacobi fallback.  `bound` is an upper bound of the largest eigenvalue.
CUFK_HD inline double key_matrix_max(const double (&N)[4][4], double bound, double (&q)[4]) {
  // Characteristic polynomial det(N - l I) = l^4 + c2 l^2 + c1 l + c0 (trace N = 0):
  // c2 = -tr(N^2) / 2, c1 = -tr(N^3) / 3, c0 = det N.
  double N2[4][4];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) N2[i][j] = N[i][0] * N[0][j] + N[i][1] * N[1][j] + N[i][2] * N[2][j] + N[i][3] * N[3][j];
  double p2 = 0.0, p3 = 0.0;
  for (int i = 0; i < 4; ++i) {
    p2 += N2[i][i];
    for (int k = 0; k < 4; ++k) p3 += N2[i][k] * N[k][i];
  }
  if (!(p2 > 0.0)) {  // N = 0: every rotation is optimal; take the identity
    q[0] = 1.0;
    q[1] = q[2] = q[3] = 0.0;
    return 0.0;
  }
  const double c2 = -0.5 * p2, c1 = -p3 / 3.0;
  const double c0 = N[0][0] * minor3(N, 0, 0) - N[0][1] * minor3(N, 0, 1) + N[0][2] * minor3(N, 0, 2) -
                    N[0][3] * minor3(N, 0, 3);
  // The eigenvalues sum to 0 and their squares to p2, so none exceeds sqrt(3 p2 / 4).
  const double cap = std::sqrt(0.75 * p2);
  double l = bound < cap ? bound : cap;
  for (int it = 0; it < 60; ++it) {
    const double l2 = l * l;
    const double f = (l2 + c2) * l2 + c1 * l + c0;
    const double df = 4.0 * l2 * l + 2.0 * c2 * l + c1;
    if (!(df != 0.0)) break;
    const double next = l - f / df;
    const bool done = std::fabs(next - l) <= 1.0e-13 * std::fabs(next);
    l = next;
    if (done) break;
  }
  // The adjugate of A = N - l I: its largest column.
  double A[4][4];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) A[i][j] = N[i][j] - (i == j ? l : 0.0);
  double best = -1.0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    double v[4], n2 = 0.0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[r] = (((r + c) & 1) ? -1.0 : 1.0) * minor3(A, c, r);  // adj(A)[r][c] = cofactor (c, r)
      n2 += v[r] * v[r];
    }
    const bool better = n2 > best;
    best = better ? n2 : best;
#pragma unroll
    for (int r = 0; r < 4; ++r) q[r] = better ? v[r] : q[r];
  }
  const double scale = std::sqrt(p2);
  if (best > 1.0e-8 * scale * scale * scale * scale * scale * scale) {
    const double inv = 1.0 / std::sqrt(best);
    for (int r = 0; r < 4; ++r) q[r] *= inv;
    return l;
  }
  double W[4][4];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) W[i][j] = N[i][j];
  return jacobi4_max(W, q);
}

// The superposition record of a chain of n points from its sums (shift points cx, ct).
CUFK_HD inline void superpose_solve(const double (&s)[kSuperposeSums], int n, const double (&cx)[3],
                                    const double (&ct)[3], double (&out)[kSuperposeRecord]) {
  const double inv = 1.0 / n;
  const double xb[3] = {s[0] * inv, s[1] * inv, s[2] * inv};  // centroids, shifted frames
  const double tb[3] = {s[3] * inv, s[4] * inv, s[5] * inv};
  double S[3][3];
  for (int a = 0; a < 3; ++a)
    for (int b = 0; b < 3; ++b) S[a][b] = s[6 + 3 * a + b] - n * xb[a] * tb[b];
  const double gx = s[15] - n * (xb[0] * xb[0] + xb[1] * xb[1] + xb[2] * xb[2]);
  const double gt = s[16] - n * (tb[0] * tb[0] + tb[1] * tb[1] + tb[2] * tb[2]);
  // Horn's key matrix.
  double N[4][4] = {
      {S[0][0] + S[1][1] + S[2][2], S[1][2] - S[2][1], S[2][0] - S[0][2], S[0][1] - S[1][0]},
      {S[1][2] - S[2][1], S[0][0] - S[1][1] - S[2][2], S[0][1] + S[1][0], S[2][0] + S[0][2]},
      {S[2][0] - S[0][2], S[0][1] + S[1][0], -S[0][0] + S[1][1] - S[2][2], S[1][2] + S[2][1]},
      {S[0][1] - S[1][0], S[2][0] + S[0][2], S[1][2] + S[2][1], -S[0][0] - S[1][1] + S[2][2]},
  };
  double q[4];
  // lambda_max <= (sum |x'|^2 + sum |t'|^2) / 2 (Cauchy-Schwarz), the start of the Newton walk.
  const double lambda = key_matrix_max(N, 0.5 * (gx + gt), q);
  const double w = q[0], x = q[1], y = q[2], z = q[3];
  // R (model onto target) from the unit quaternion; M = R^T.
  const double R[3][3] = {
      {w * w + x * x - y * y - z * z, 2 * (x * y - w * z), 2 * (x * z + w * y)},
      {2 * (y * x + w * z), w * w - x * x + y * y - z * z, 2 * (y * z - w * x)},
      {2 * (z * x - w * y), 2 * (z * y + w * x), w * w - x * x - y * y + z * z},
  };
  for (int a = 0; a < 3; ++a)
    for (int b = 0; b < 3; ++b) out[3 * a + b] = R[b][a];
  // a = xbar - R^T tbar in world coordinates (xbar = cx + xb, tbar = ct + tb).
  for (int a = 0; a < 3; ++a) {
    double rt = 0.0;
    for (int b = 0; b < 3; ++b) rt += R[b][a] * (ct[b] + tb[b]);
    out[9 + a] = cx[a] + xb[a] - rt;
  }
  const double msd = (gx + gt - 2.0 * lambda) * inv;
  out[12] = msd > 0.0 ? msd : 0.0;
  for (int k = 13; k < kSuperposeRecord; ++k) out[k] = 0.0;
}

// In place: a record holding the sums and shift points becomes the solved record.
CUFK_HD inline void superpose_solve_record(double (&rec)[kSuperposeRecord], int n) {
  double s[kSuperposeSums];
  for (int k = 0; k < kSuperposeSums; ++k) s[k] = rec[k];
  const double cx[3] = {rec[17], rec[18], rec[19]};
  const double ct[3] = {rec[20], rec[21], rec[22]};
  superpose_solve(s, n, cx, ct, rec);
}

}  // namespace cufk_amd
