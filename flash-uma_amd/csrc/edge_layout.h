// Column blocks of the lmax = 2 edge arrays (gather outputs X_m0 / X_m1 / X_m2 and the radial
// rows), shared by the gather kernels and the radial GEMM that writes the gather's outputs.
//
// Slot q of side so (0 = sender, 1 = receiver).  Layout 0 is the reference order, sides
// interleaved (2q + so, ops/gather.py:132-154).  Layout 1:
//   X_m0, rad: each side's slots contiguous (so * per_side + q);
//   X_m1: real slots (q = 0, 1) then imaginary slots (q = 2, 3), each half side-major, so
//         that x_r and x_i are the two contiguous halves the complex layer reads;
//   X_m2: reference order (already [x_r | x_i]).
// Radial slot q: (l, |m|) = (0, 0), (1, 0), (2, 0), (1, 1), (2, 1), (2, 2).
#pragma once

#include <hip/hip_runtime.h>

namespace fu {

template <int L>
__host__ __device__ constexpr int slot_m0(int so, int q) { return L ? so * 3 + q : 2 * q + so; }
template <int L>
__host__ __device__ constexpr int slot_m1(int so, int q) {
  return L ? (q >> 1) * 4 + so * 2 + (q & 1) : 2 * q + so;
}
template <int L>
__host__ __device__ constexpr int slot_m2(int so, int q) { return 2 * q + so; }
template <int L>
__host__ __device__ constexpr int slot_rad(int so, int q) { return L ? so * 6 + q : 2 * q + so; }

}  // namespace fu
