// Block layout of the lmax 2..4 edge arrays (mmax = 2), shared by the lmax edge kernels and
// the radial GEMM that writes the gather's outputs:
//   SH coefficient (l, m) of a node row sits at row l^2 + l + m; the edge frame keeps the
//   orders |m| <= min(l, 2).  Per edge, with side so = 0 (sender) / 1 (receiver):
//     X_m0 (2(L+1) blocks): (l, 0) at block 2l + so
//     X_m1 (4L blocks):     (l, +1) at 2(l-1) + so, (l, -1) at 2(L + l - 1) + so
//     X_m2 (4(L-1) blocks): (l, +2) at 2(l-2) + so, (l, -2) at 2(L - 1 + l - 2) + so
//     rad (6L blocks):      |m| = 0: 2l + so; 1: 2(L+1) + 2(l-1) + so; 2: 4L + 2 + 2(l-2) + so
//   Wigner rows: the reference's 34 scalars give D^1 and D^2; the ext array gives rows
//   m = -2..2 of D^3 (5 x 7) and D^4 (5 x 9).
#pragma once

#include <hip/hip_runtime.h>

namespace fu {
namespace lm {

__host__ __device__ constexpr int mmx(int l) { return l < 2 ? l : 2; }
__host__ __device__ constexpr int ncoef(int L) { return (L + 1) * (L + 1); }
__host__ __device__ constexpr int extw(int L) { return L >= 4 ? 80 : L == 3 ? 35 : 0; }
__host__ __device__ constexpr int wx0(int L) { return 2 * (L + 1); }
__host__ __device__ constexpr int wx1(int L) { return 4 * L; }
__host__ __device__ constexpr int wx2(int L) { return 4 * (L - 1); }
__host__ __device__ constexpr int wrad(int L) { return 6 * L; }
__host__ __device__ constexpr int xblk(int L, int l, int m, int so) {
  return m == 0 ? 2 * l + so
         : (m == 1 || m == -1) ? 2 * ((m > 0 ? 0 : L) + l - 1) + so
                               : 2 * ((m > 0 ? 0 : L - 1) + l - 2) + so;
}
__host__ __device__ constexpr int radblk(int L, int l, int am, int so) {
  return am == 0 ? 2 * l + so : am == 1 ? 2 * (L + 1) + 2 * (l - 1) + so : 4 * L + 2 + 2 * (l - 2) + so;
}
// block of (l, m) in Z_m0 / Z_m1 / Z_m2 (no sides)
__host__ __device__ constexpr int zblk(int L, int l, int m) {
  return m == 0 ? l : (m == 1 || m == -1) ? (m > 0 ? 0 : L) + l - 1 : (m > 0 ? 0 : L - 1) + l - 2;
}
// index of D^l[m][mp] in the reference's 34 scalars (l <= 2) or in the ext array (l >= 3)
__host__ __device__ constexpr int widx(int l, int m, int mp) {
  return l == 1 ? 3 * (1 + m) + 1 + mp : l == 2 ? 9 + 5 * (2 + m) + 2 + mp
         : l == 3 ? 7 * (2 + m) + 3 + mp : 35 + 9 * (2 + m) + 4 + mp;
}

}  // namespace lm
}  // namespace fu
