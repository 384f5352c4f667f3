// fp64 path of the ChebyKAN layer.  The reference layer computes in fp64
// when its parameter is fp64 (kan/layers/chebykan.py:48-51 after .double();
// kan/basis/chebyshev.py:78-101 then runs in fp64).  On MI355X the vector
// ALU's fp64 FMA rate is of the same order as fp64 MFMA, so these kernels are
// register-tiled VALU kernels with LDS staging: no packing, no workspace, the
// basis recurrence in fp64 registers.
//   forward  y[b, o]     = sum_{i, d} T_d(t[b, i]) C[i, o, d],  t = tanh(x)
//   dx       dx[b, i]    = (1 - t^2) sum_d G[b, i, d] d U_{d-1}(t),
//                          G[b, i, d] = sum_o dy[b, o] C[i, o, d]
//   dC       dC[i, o, d] = sum_b T_d(t[b, i]) dy[b, o]
#include "ckan_kernels.hpp"

#include <math.h>

namespace ckan {

__global__ void __launch_bounds__(256)
k_tanh_f64(const double* __restrict__ x, double* __restrict__ t, int64_t n) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x)
    t[q] = tanh(x[q]);
}

// Forward: block tile 64 rows x 64 outputs, 256 threads, thread (tr, to)
// owns rows tr + 16 r and outputs to + 16 c (r, c < 4).  Inputs are taken
// F64_KI at a time: t [64][KI] and C as [KI][D][64 outputs] in LDS.
constexpr int F64_KI = 4;
template <int DM>
__global__ void __launch_bounds__(256)
k_fwd_f64(const double* __restrict__ t, const double* __restrict__ C, double* __restrict__ y,
          int64_t B, int I, int O, int D) {
  __shared__ double ts[64][F64_KI + 1];
  __shared__ double cs[F64_KI][DM][64];
  const int tid = threadIdx.x, tr = tid >> 4, to = tid & 15;
  const int64_t b0 = (int64_t)blockIdx.x * 64;
  const int o0 = blockIdx.y * 64;
  double acc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r][c] = 0.0;
  for (int i0 = 0; i0 < I; i0 += F64_KI) {
    __syncthreads();
    for (int k = tid; k < 64 * F64_KI; k += 256) {
      const int r = k / F64_KI, ii = k % F64_KI;
      const int64_t b = b0 + r;
      ts[r][ii] = (b < B && i0 + ii < I) ? t[b * I + i0 + ii] : 0.0;
    }
    // C rows [i][o0 .. o0+64)[0 .. D) are contiguous runs of 64 * D values
    for (int k = tid; k < F64_KI * 64 * D; k += 256) {
      const int ii = k / (64 * D), rem = k % (64 * D), ol = rem / D, d = rem % D;
      const int i = i0 + ii, o = o0 + ol;
      cs[ii][d][ol] = (i < I && o < O) ? C[((size_t)i * O + o) * D + d] : 0.0;
    }
    __syncthreads();
#pragma unroll
    for (int ii = 0; ii < F64_KI; ++ii) {
      double tp[4], tc[4], tw[4];  // T_{d-1}, T_d, 2 t
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        tw[r] = 2.0 * ts[tr + 16 * r][ii];
        tp[r] = 0.0;
        tc[r] = 1.0;
      }
      for (int d = 0; d < D; ++d) {
        double cv[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) cv[c] = cs[ii][d][to + 16 * c];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[r][c] = fma(tc[r], cv[c], acc[r][c]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // T_{d+1} = 2t T_d - T_{d-1} (T_1 = t)
          const double nx = d == 0 ? 0.5 * tw[r] : fma(tw[r], tc[r], -tp[r]);
          tp[r] = tc[r];
          tc[r] = nx;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t b = b0 + tr + 16 * r;
    if (b >= B) continue;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int o = o0 + to + 16 * c;
      if (o < O) y[b * O + o] = acc[r][c];
    }
  }
}

// dx: block tile 128 rows x 8 inputs; thread (rr, ii) = (tid / 8, tid % 8)
// owns G[b, i, 0..D) of rows rr + 32 h (h < 4) in registers.  Outputs are
// taken 16 at a time: dy [128][16] and C as [8 inputs][16 outputs][D] in LDS,
// the per-input stride padded to an odd number of doubles so the 8 inputs of
// a wave read distinct banks.
template <int DM>
__global__ void __launch_bounds__(256)
k_dx_f64(const double* __restrict__ t, const double* __restrict__ C, const double* __restrict__ dy,
         double* __restrict__ dx, int64_t B, int I, int O, int D) {
  constexpr int OC = 16, CST = OC * (DM + 1) + 1;
  __shared__ double ys[128][OC + 1];
  __shared__ double cs[8 * CST];
  const int tid = threadIdx.x, rr = tid >> 3, ii = tid & 7;
  const int64_t b0 = (int64_t)blockIdx.x * 128;
  const int i0 = blockIdx.y * 8;
  double g[4][DM];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int d = 0; d < DM; ++d) g[h][d] = 0.0;
  for (int oc = 0; oc < O; oc += OC) {
    __syncthreads();
    for (int k = tid; k < 128 * OC; k += 256) {
      const int r = k / OC, ol = k % OC;
      const int64_t b = b0 + r;
      ys[r][ol] = (b < B && oc + ol < O) ? dy[b * O + oc + ol] : 0.0;
    }
    for (int k = tid; k < 8 * OC * D; k += 256) {
      const int il = k / (OC * D), rem = k % (OC * D), ol = rem / D, d = rem % D;
      const int i = i0 + il, o = oc + ol;
      cs[il * CST + ol * (DM + 1) + d] = (i < I && o < O) ? C[((size_t)i * O + o) * D + d] : 0.0;
    }
    __syncthreads();
    for (int ol = 0; ol < OC; ++ol) {
      double a[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) a[h] = ys[rr + 32 * h][ol];
      const double* cr = cs + ii * CST + ol * (DM + 1);
#pragma unroll
      for (int d = 0; d < DM; ++d) {
        if (d < D) {
          const double cv = cr[d];
#pragma unroll
          for (int h = 0; h < 4; ++h) g[h][d] = fma(a[h], cv, g[h][d]);
        }
      }
    }
  }
  const int i = i0 + ii;
  if (i >= I) return;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int64_t b = b0 + rr + 32 * h;
    if (b >= B) continue;
    const double tv = t[b * I + i];
    const double t2 = 2.0 * tv;
    double up = 0.0, u = 1.0, s = 0.0;  // U_{-1}, U_0
#pragma unroll
    for (int d = 1; d < DM; ++d) {
      if (d < D) {
        s = fma(g[h][d] * (double)d, u, s);
        const double un = fma(t2, u, -up);
        up = u;
        u = un;
      }
    }
    dx[b * I + i] = s * (1.0 - tv * tv);
  }
}

// dC: block tile 8 inputs x 128 outputs; thread (il, ol) = (tid / 32, tid % 32)
// owns outputs ol + 32 c (c < 4) of input il, all D degrees, so each basis
// recurrence serves four outputs.  Rows are taken 32 at a time: t [32][8] and
// dy [32][128] in LDS.
template <int DM>
__global__ void __launch_bounds__(256)
k_dc_f64(const double* __restrict__ t, const double* __restrict__ dy, double* __restrict__ dC,
         int64_t B, int I, int O, int D, int accumulate) {
  __shared__ double ts[32][9];
  __shared__ double ys[32][129];
  const int tid = threadIdx.x, il = tid >> 5, ol = tid & 31;
  const int i0 = blockIdx.x * 8, o0 = blockIdx.y * 128;
  double acc[4][DM];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int d = 0; d < DM; ++d) acc[c][d] = 0.0;
  for (int64_t bc = 0; bc < B; bc += 32) {
    __syncthreads();
    {
      const int r = tid >> 3, k = tid & 7;
      const int64_t b = bc + r;
      ts[r][k] = (b < B && i0 + k < I) ? t[b * I + i0 + k] : 0.0;
    }
    for (int k = tid; k < 32 * 128; k += 256) {
      const int r = k >> 7, o = k & 127;
      const int64_t b = bc + r;
      ys[r][o] = (b < B && o0 + o < O) ? dy[b * O + o0 + o] : 0.0;
    }
    __syncthreads();
    for (int r = 0; r < 32; ++r) {
      const double tv = ts[r][il], t2 = 2.0 * tv;
      double yv[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) yv[c] = ys[r][ol + 32 * c];
      double tp = 0.0, tc = 1.0;
#pragma unroll
      for (int d = 0; d < DM; ++d) {
        if (d < D) {
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[c][d] = fma(tc, yv[c], acc[c][d]);
          const double nx = d == 0 ? tv : fma(t2, tc, -tp);
          tp = tc;
          tc = nx;
        }
      }
    }
  }
  const int i = i0 + il;
  if (i >= I) return;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int o = o0 + ol + 32 * c;
    if (o >= O) continue;
    double* dst = dC + ((size_t)i * O + o) * D;
#pragma unroll
    for (int d = 0; d < DM; ++d)
      if (d < D) dst[d] = accumulate ? dst[d] + acc[c][d] : acc[c][d];
  }
}

static unsigned grid1(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (unsigned)(g < 1 ? 1 : g);
}

void launch_forward_f64(const double* x, const double* C, double* y, double* t, int64_t B, int I,
                        int O, int deg, hipStream_t s) {
  hipLaunchKernelGGL(k_tanh_f64, dim3(grid1(B * I)), dim3(256), 0, s, x, t, B * I);
  const int D = deg + 1;
  const dim3 g((unsigned)((B + 63) / 64), (unsigned)((O + 63) / 64));
  if (D <= 3) hipLaunchKernelGGL((k_fwd_f64<3>), g, dim3(256), 0, s, t, C, y, B, I, O, D);
  else if (D <= 5) hipLaunchKernelGGL((k_fwd_f64<5>), g, dim3(256), 0, s, t, C, y, B, I, O, D);
  else if (D <= 9) hipLaunchKernelGGL((k_fwd_f64<9>), g, dim3(256), 0, s, t, C, y, B, I, O, D);
  else hipLaunchKernelGGL((k_fwd_f64<17>), g, dim3(256), 0, s, t, C, y, B, I, O, D);
}

void launch_backward_f64(const double* t, const double* C, const double* dy, double* dx,
                         double* dC, bool accumulate, int64_t B, int I, int O, int deg,
                         hipStream_t s) {
  const int D = deg + 1;
  if (dx) {
    const dim3 g((unsigned)((B + 127) / 128), (unsigned)((I + 7) / 8));
    if (D <= 3) hipLaunchKernelGGL((k_dx_f64<3>), g, dim3(256), 0, s, t, C, dy, dx, B, I, O, D);
    else if (D <= 5) hipLaunchKernelGGL((k_dx_f64<5>), g, dim3(256), 0, s, t, C, dy, dx, B, I, O, D);
    else if (D <= 9) hipLaunchKernelGGL((k_dx_f64<9>), g, dim3(256), 0, s, t, C, dy, dx, B, I, O, D);
    else hipLaunchKernelGGL((k_dx_f64<17>), g, dim3(256), 0, s, t, C, dy, dx, B, I, O, D);
  }
  if (dC) {
    const dim3 g((unsigned)((I + 7) / 8), (unsigned)((O + 127) / 128));
    const int acc = accumulate ? 1 : 0;
    if (D <= 3) hipLaunchKernelGGL((k_dc_f64<3>), g, dim3(256), 0, s, t, dy, dC, B, I, O, D, acc);
    else if (D <= 5) hipLaunchKernelGGL((k_dc_f64<5>), g, dim3(256), 0, s, t, dy, dC, B, I, O, D, acc);
    else if (D <= 9) hipLaunchKernelGGL((k_dc_f64<9>), g, dim3(256), 0, s, t, dy, dC, B, I, O, D, acc);
    else hipLaunchKernelGGL((k_dc_f64<17>), g, dim3(256), 0, s, t, dy, dC, B, I, O, D, acc);
  }
}

}  // namespace ckan
