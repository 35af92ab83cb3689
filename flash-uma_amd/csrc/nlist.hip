// Capped periodic radius graph on the GPU (the FAIRChem a2g graph the reference takes as
// input, readme.md:34), with the exact definition of the host builder in systems.py:
//
//   for receiver j, candidates (i, o), o an integer cell offset (0 on non-periodic axes),
//   (i, o) != (j, 0);  d = (pos_i - pos_j) + ((o0 c0 + o1 c1) + o2 c2) in float64 from the
//   float32 inputs;  |d|^2 = (dx dx + dy dy) + dz dz < cutoff^2;  ordered by
//   (|d|^2, i, o0, o1, o2);  the first max_neighbors kept;  edges grouped by receiver.
//
// Every float64 operation is written out in that order with contraction disabled, so the
// graph is bit-identical to the host one (same edges, same order, same offsets).
//
// Pipeline: (1) fu_nlist_bin: fractional coordinates -> wrapped cell-list bin + wrap count
// per atom; atoms are then sorted by bin (fu_sort_pairs_i64) and bin ranges found
// (fu_csr_row_ptr).  Bins are at least cutoff + 1e-3 wide, so with `reach` bins searched
// per side every neighbour is visited exactly once per periodic image.  (2) fu_nlist_search:
// one wave per receiver walks the neighbouring bins, tests 64 candidates at a time, appends
// hits to an LDS list (ballot + prefix count), then ranks the list by the ordering key
// (each entry's rank = number of smaller keys; keys are unique) and writes the first
// max_neighbors.  (3) fu_nlist_scan: exclusive scan of the per-receiver counts.
// (4) fu_nlist_emit: edge_index (2, E) int64 and cell_offsets (E, 3) float32.
#include "fu_common.h"

namespace fu {

constexpr int NL_CAP = 512;  // hits held per receiver (the host checks the counts against it)

struct NLGeom {
  double cell[9];   // lattice vectors as rows, float64 copies of the float32 cell
  double inv[9];    // inverse of cell (fractional coordinates s = pos inv)
  int nb[3];        // bins per axis
  int reach[3];     // bins searched on each side (0 on non-periodic axes)
  int pbc[3];
  double cut2;      // cutoff * cutoff
};

__device__ __forceinline__ int floor_div(int a, int n) { return a >= 0 ? a / n : -((-a + n - 1) / n); }

__global__ __launch_bounds__(256) void nlist_bin_kernel(const float* __restrict__ pos, NLGeom g, int64_t N,
                                                        int64_t* __restrict__ bin_key, int32_t* __restrict__ wrap) {
  for (int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; a < N; a += (int64_t)gridDim.x * blockDim.x) {
    const double p[3] = {(double)pos[3 * a], (double)pos[3 * a + 1], (double)pos[3 * a + 2]};
    int b[3];
#pragma unroll
    for (int ax = 0; ax < 3; ++ax) {
      double s = p[0] * g.inv[ax] + p[1] * g.inv[3 + ax] + p[2] * g.inv[6 + ax];
      int w = 0;
      if (g.pbc[ax]) {
        const double f = floor(s);
        w = (int)f;
        s -= f;
        int bb = (int)floor(s * g.nb[ax]);
        b[ax] = bb < 0 ? 0 : (bb >= g.nb[ax] ? g.nb[ax] - 1 : bb);
      } else {
        b[ax] = 0;
      }
      wrap[3 * a + ax] = w;
    }
    bin_key[a] = ((int64_t)b[0] * g.nb[1] + b[1]) * g.nb[2] + b[2];
  }
}

// d and |d|^2 in the host's operation order, each operation rounded separately.
__device__ __forceinline__ double pair_d2(const double* pi, const double* pj, const int* o, const double* cell) {
#pragma clang fp contract(off)
  double d[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const double sh = ((double)o[0] * cell[a] + (double)o[1] * cell[3 + a]) + (double)o[2] * cell[6 + a];
    d[a] = (pi[a] - pj[a]) + sh;
  }
  return (d[0] * d[0] + d[1] * d[1]) + d[2] * d[2];
}

__global__ __launch_bounds__(256) void nlist_search_kernel(
    const float* __restrict__ pos, const int64_t* __restrict__ sorted_atoms, const int32_t* __restrict__ bin_ptr,
    const int32_t* __restrict__ wrap, const int64_t* __restrict__ bin_key, NLGeom g, int64_t N, int32_t K,
    int32_t* __restrict__ out_sender, int32_t* __restrict__ out_off, int32_t* __restrict__ count,
    int32_t* __restrict__ nout) {
  __shared__ double s_d2[4][NL_CAP];
  __shared__ uint64_t s_key[4][NL_CAP];  // (i << 24) | (o0 + 128) << 16 | (o1 + 128) << 8 | (o2 + 128)
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t j = (int64_t)blockIdx.x * 4 + w;
  const bool active = j < N;
  int cnt = 0;  // wave-uniform
  if (active) {
    const double pj[3] = {(double)pos[3 * j], (double)pos[3 * j + 1], (double)pos[3 * j + 2]};
    const int wj[3] = {wrap[3 * j], wrap[3 * j + 1], wrap[3 * j + 2]};
    const int64_t kj = bin_key[j];
    const int bj[3] = {(int)(kj / ((int64_t)g.nb[1] * g.nb[2])), (int)((kj / g.nb[2]) % g.nb[1]), (int)(kj % g.nb[2])};
    for (int dx = -g.reach[0]; dx <= g.reach[0]; ++dx)
      for (int dy = -g.reach[1]; dy <= g.reach[1]; ++dy)
        for (int dz = -g.reach[2]; dz <= g.reach[2]; ++dz) {
          const int u[3] = {bj[0] + dx, bj[1] + dy, bj[2] + dz};
          int nbn[3], kk[3];
#pragma unroll
          for (int a = 0; a < 3; ++a) {
            kk[a] = floor_div(u[a], g.nb[a]);
            nbn[a] = u[a] - kk[a] * g.nb[a];
          }
          const int64_t bin = ((int64_t)nbn[0] * g.nb[1] + nbn[1]) * g.nb[2] + nbn[2];
          const int32_t lo = bin_ptr[bin], hi = bin_ptr[bin + 1];
          for (int32_t t = lo; t < hi; t += 64) {
            const int32_t idx = t + lane;
            bool hit = false;
            double d2 = 0.0;
            uint64_t key = 0;
            if (idx < hi) {
              const int64_t i = sorted_atoms[idx];
              int o[3];
#pragma unroll
              for (int a = 0; a < 3; ++a) o[a] = g.pbc[a] ? kk[a] - wrap[3 * i + a] + wj[a] : 0;
              const bool self = (i == j) && o[0] == 0 && o[1] == 0 && o[2] == 0;
              const double pi[3] = {(double)pos[3 * i], (double)pos[3 * i + 1], (double)pos[3 * i + 2]};
              d2 = pair_d2(pi, pj, o, g.cell);
              hit = !self && d2 < g.cut2;
              key = ((uint64_t)i << 24) | ((uint64_t)(o[0] + 128) << 16) | ((uint64_t)(o[1] + 128) << 8) |
                    (uint64_t)(o[2] + 128);
            }
            const uint64_t mask = __ballot(hit);
            const int slot = cnt + __popcll(mask & ((1ull << lane) - 1ull));
            if (hit && slot < NL_CAP) {
              s_d2[w][slot] = d2;
              s_key[w][slot] = key;
            }
            cnt += __popcll(mask);
          }
        }
  }
  __syncthreads();
  if (!active) return;
  const int n = cnt < NL_CAP ? cnt : NL_CAP;
  for (int e = lane; e < n; e += 64) {
    const double de = s_d2[w][e];
    const uint64_t ke = s_key[w][e];
    int rank = 0;
    for (int f = 0; f < n; ++f) {
      const double df = s_d2[w][f];
      rank += (df < de || (df == de && s_key[w][f] < ke)) ? 1 : 0;
    }
    if (rank < K) {
      const int64_t slot = j * K + rank;
      out_sender[slot] = (int32_t)(ke >> 24);
      out_off[3 * slot + 0] = (int)((ke >> 16) & 0xff) - 128;
      out_off[3 * slot + 1] = (int)((ke >> 8) & 0xff) - 128;
      out_off[3 * slot + 2] = (int)(ke & 0xff) - 128;
    }
  }
  if (lane == 0) {
    count[j] = cnt;
    nout[j] = n < K ? n : K;
  }
}

// Exclusive scan of nout into row_ptr (N + 1 entries, row_ptr[N] = E) by one workgroup.
__global__ __launch_bounds__(1024) void nlist_scan_kernel(const int32_t* __restrict__ nout, int64_t* __restrict__ row_ptr,
                                                          int64_t N) {
  __shared__ int64_t s[1024];
  const int t = threadIdx.x;
  const int64_t chunk = (N + 1023) / 1024;
  const int64_t b = t * chunk, e = b + chunk < N ? b + chunk : N;
  int64_t sum = 0;
  for (int64_t k = b; k < e; ++k) sum += nout[k];
  s[t] = sum;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int64_t v = t >= off ? s[t - off] : 0;
    __syncthreads();
    s[t] += v;
    __syncthreads();
  }
  int64_t run = t ? s[t - 1] : 0;
  for (int64_t k = b; k < e; ++k) {
    row_ptr[k] = run;
    run += nout[k];
  }
  if (t == 1023) row_ptr[N] = s[1023];
}

__global__ __launch_bounds__(256) void nlist_emit_kernel(const int32_t* __restrict__ sender,
                                                         const int32_t* __restrict__ off,
                                                         const int32_t* __restrict__ nout,
                                                         const int64_t* __restrict__ row_ptr, int64_t N, int32_t K,
                                                         int64_t* __restrict__ edge_index,
                                                         float* __restrict__ cell_offsets, int64_t E) {
  const int64_t total = N * K;
  for (int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s < total; s += (int64_t)gridDim.x * blockDim.x) {
    const int64_t j = s / K;
    const int r = (int)(s - j * K);
    if (r >= nout[j]) continue;
    const int64_t e = row_ptr[j] + r;
    edge_index[e] = sender[s];
    edge_index[E + e] = j;
#pragma unroll
    for (int a = 0; a < 3; ++a) cell_offsets[3 * e + a] = (float)off[3 * s + a];
  }
}

static NLGeom nl_geom(const double* cell, const double* inv, const int32_t* nbins, const int32_t* reach,
                      const int32_t* pbc, double cutoff) {
  NLGeom g;
  for (int k = 0; k < 9; ++k) {
    g.cell[k] = cell[k];
    g.inv[k] = inv[k];
  }
  for (int a = 0; a < 3; ++a) {
    g.nb[a] = nbins[a];
    g.reach[a] = reach[a];
    g.pbc[a] = pbc[a] ? 1 : 0;
  }
  g.cut2 = cutoff * cutoff;
  return g;
}

static int nl_check_geom(const double* cell, const double* inv, const int32_t* nbins, const int32_t* reach,
                         const int32_t* pbc, const char* who) {
  if (!cell || !inv || !nbins || !reach || !pbc) return set_error(FU_ERR_NULL, "%s: NULL geometry", who);
  int64_t total = 1;
  for (int a = 0; a < 3; ++a) {
    if (nbins[a] < 1 || reach[a] < 0 || reach[a] > 64 || (!pbc[a] && (nbins[a] != 1 || reach[a] != 0)))
      return set_error(FU_ERR_SHAPE, "%s: bad bins/reach on axis %d", who, a);
    total *= nbins[a];
  }
  if (total > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "%s: too many bins", who);
  return FU_OK;
}

}  // namespace fu

using namespace fu;

extern "C" int fu_nlist_bin(const float* pos, int64_t N, const double* cell, const double* inv_cell,
                            const int32_t* nbins, const int32_t* reach, const int32_t* pbc, int64_t* bin_key,
                            int32_t* wrap, void* stream) {
  if (N < 0) return set_error(FU_ERR_SHAPE, "fu_nlist_bin: bad shape");
  int st = nl_check_geom(cell, inv_cell, nbins, reach, pbc, "fu_nlist_bin");
  if (st != FU_OK) return st;
  if (N == 0) return FU_OK;
  if (!pos || !bin_key || !wrap) return set_error(FU_ERR_NULL, "fu_nlist_bin: NULL argument");
  const NLGeom g = nl_geom(cell, inv_cell, nbins, reach, pbc, 0.0);
  hipLaunchKernelGGL(nlist_bin_kernel, dim3((unsigned)std::min<int64_t>(cdiv(N, 256), 65536)), dim3(256), 0,
                     as_stream(stream), pos, g, N, bin_key, wrap);
  return check_launch("fu_nlist_bin");
}

extern "C" int fu_nlist_search(const float* pos, const int64_t* sorted_atoms, const int32_t* bin_ptr,
                               const int32_t* wrap, const int64_t* bin_key, int64_t N, const double* cell,
                               const double* inv_cell, const int32_t* nbins, const int32_t* reach,
                               const int32_t* pbc, double cutoff, int32_t max_neighbors, int32_t* out_sender,
                               int32_t* out_off, int32_t* count, int32_t* nout, void* stream) {
  if (N < 0 || max_neighbors < 1 || !(cutoff > 0.0)) return set_error(FU_ERR_SHAPE, "fu_nlist_search: bad arguments");
  if (N > 0x7fffffffLL) return set_error(FU_ERR_SHAPE, "fu_nlist_search: N too large");
  int st = nl_check_geom(cell, inv_cell, nbins, reach, pbc, "fu_nlist_search");
  if (st != FU_OK) return st;
  if (N == 0) return FU_OK;
  if (!pos || !sorted_atoms || !bin_ptr || !wrap || !bin_key || !out_sender || !out_off || !count || !nout)
    return set_error(FU_ERR_NULL, "fu_nlist_search: NULL argument");
  const NLGeom g = nl_geom(cell, inv_cell, nbins, reach, pbc, cutoff);
  hipLaunchKernelGGL(nlist_search_kernel, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, as_stream(stream), pos,
                     sorted_atoms, bin_ptr, wrap, bin_key, g, N, max_neighbors, out_sender, out_off, count, nout);
  return check_launch("fu_nlist_search");
}

extern "C" int fu_nlist_scan(const int32_t* nout, int64_t* row_ptr, int64_t N, void* stream) {
  if (N < 0) return set_error(FU_ERR_SHAPE, "fu_nlist_scan: bad shape");
  if (!row_ptr || (N > 0 && !nout)) return set_error(FU_ERR_NULL, "fu_nlist_scan: NULL argument");
  hipLaunchKernelGGL(nlist_scan_kernel, dim3(1), dim3(1024), 0, as_stream(stream), nout, row_ptr, N);
  return check_launch("fu_nlist_scan");
}

extern "C" int fu_nlist_emit(const int32_t* sender, const int32_t* off, const int32_t* nout, const int64_t* row_ptr,
                             int64_t N, int32_t max_neighbors, int64_t* edge_index, float* cell_offsets, int64_t E,
                             void* stream) {
  if (N < 0 || E < 0 || max_neighbors < 1) return set_error(FU_ERR_SHAPE, "fu_nlist_emit: bad shape");
  if (N == 0 || E == 0) return FU_OK;
  if (!sender || !off || !nout || !row_ptr || !edge_index || !cell_offsets)
    return set_error(FU_ERR_NULL, "fu_nlist_emit: NULL argument");
  hipLaunchKernelGGL(nlist_emit_kernel, dim3((unsigned)std::min<int64_t>(cdiv(N * max_neighbors, 256), 65536)),
                     dim3(256), 0, as_stream(stream), sender, off, nout, row_ptr, N, max_neighbors, edge_index,
                     cell_offsets, E);
  return check_launch("fu_nlist_emit");
}
