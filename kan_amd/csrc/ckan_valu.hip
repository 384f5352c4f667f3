// The ChebyKAN layer on the vector ALU, for any degree, in fp32 or fp64:
//   forward  y[b, o]     = sum_{i, d} T_d(t[b, i]) C[i, o, d],  t = tanh(x)
//   dx       dx[b, i]    = (1 - t^2) sum_d G[b, i, d] d U_{d-1}(t),
//                          G[b, i, d] = sum_o dy[b, o] C[i, o, d]
//   dC       dC[i, o, d] = sum_b T_d(t[b, i]) dy[b, o]
// It serves the fp64 layer (the reference computes in fp64 when its
// parameter is fp64: kan/layers/chebykan.py:48-51 after .double()) and fp32
// layers above the MFMA kernels' degree 16 (the reference layer takes any
// degree, kan/layers/chebykan.py:21-51).  Register-tiled kernels with LDS
// staging read C in its own [I, O, D] layout.  The degree axis is taken in
// chunks of at most DM degrees (one launch each; DM = 3, 5, 9 or 17, the
// smallest that holds D, and 17 above): a chunk starting at d0
// first advances the recurrence to T_{d0-1}, T_{d0} (or U_{d0-2}, U_{d0-1}),
// so register arrays stay bounded for any degree.  t = tanh(x) is [B, I].
#include "ckan_kernels.hpp"

#include <math.h>

namespace ckan {

constexpr int kValuDM = 17;  // degrees per chunk above degree 16

template <typename T> __device__ __forceinline__ T vtanh(T x);
template <> __device__ __forceinline__ float vtanh<float>(float x) { return tanhf(x); }
template <> __device__ __forceinline__ double vtanh<double>(double x) { return tanh(x); }

template <typename T>
__global__ void __launch_bounds__(256)
k_tanh_v(const T* __restrict__ x, T* __restrict__ t, int64_t n) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x)
    t[q] = vtanh<T>(x[q]);
}

// T_{d0-1} and T_{d0} of t.  T_{-1} = t extends the recurrence
// T_{d+1} = 2t T_d - T_{d-1} down to d = 0 (its first step gives
// 2t - t = t = T_1 exactly), so every step below is the same FMA.
template <typename T>
__device__ __forceinline__ void cheb_seek(T t, int d0, T& tp, T& tc) {
  tp = t;     // T_{-1}
  tc = T(1);  // T_0
  const T t2 = t + t;
  for (int d = 0; d < d0; ++d) {
    const T nx = fma(t2, tc, -tp);
    tp = tc;
    tc = nx;
  }
}

// SEEK = false instantiations serve the first chunk (d0 = 0, stored, not
// accumulated) with no seek loops in the code, as register-lean as a
// single-chunk kernel.

// Forward, degrees [d0, d0 + dn): block tile 64 rows x 64 outputs, 256
// threads, thread (tr, to) owns rows tr + 16 r and outputs to + 16 c
// (r, c < 4).  Inputs are taken KI at a time: t [64][KI] and the chunk of C
// as [KI][DM][64 outputs] in LDS.  accumulate: add to y (later chunks).
constexpr int kValuKI = 4;
template <typename T, int DM, bool SEEK>
__global__ void __launch_bounds__(256)
k_fwd_v(const T* __restrict__ t, const T* __restrict__ C, T* __restrict__ y, int64_t B, int I,
        int O, int D, int d0_arg, int dn, int accumulate) {
  constexpr int KI = kValuKI;
  const int d0 = SEEK ? d0_arg : 0;
  __shared__ T ts[64][KI + 1];
  __shared__ T cs[KI][DM][64];
  const int tid = threadIdx.x, tr = tid >> 4, to = tid & 15;
  const int64_t b0 = (int64_t)blockIdx.x * 64;
  const int o0 = blockIdx.y * 64;
  T acc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r][c] = T(0);
  for (int i0 = 0; i0 < I; i0 += KI) {
    __syncthreads();
    for (int k = tid; k < 64 * KI; k += 256) {
      const int r = k / KI, ii = k % KI;
      const int64_t b = b0 + r;
      ts[r][ii] = (b < B && i0 + ii < I) ? t[b * I + i0 + ii] : T(0);
    }
    for (int k = tid; k < KI * 64 * dn; k += 256) {
      const int ii = k / (64 * dn), rem = k % (64 * dn), ol = rem / dn, d = rem % dn;
      const int i = i0 + ii, o = o0 + ol;
      cs[ii][d][ol] = (i < I && o < O) ? C[((size_t)i * O + o) * D + d0 + d] : T(0);
    }
    __syncthreads();
#pragma unroll
    for (int ii = 0; ii < KI; ++ii) {
      T tp[4], tc[4], tw[4];  // T_{d-1}, T_d, 2 t
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const T tv = ts[tr + 16 * r][ii];
        tw[r] = tv + tv;
        cheb_seek<T>(tv, d0, tp[r], tc[r]);
      }
      for (int d = 0; d < dn; ++d) {  // rolled: measured faster than unrolled here
        {
          T cv[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) cv[c] = cs[ii][d][to + 16 * c];
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[r][c] = fma(tc[r], cv[c], acc[r][c]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {  // T_{d+1} = 2t T_d - T_{d-1}
            const T nx = fma(tw[r], tc[r], -tp[r]);
            tp[r] = tc[r];
            tc[r] = nx;
          }
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
      if (o < O) y[b * O + o] = SEEK && accumulate ? y[b * O + o] + acc[r][c] : acc[r][c];
    }
  }
}

// dx, degrees [d0, d0 + dn): block tile 128 rows x 8 inputs; thread
// (rr, ii) = (tid / 8, tid % 8) owns G[b, i, d0 .. d0+dn) of rows rr + 32 h
// (h < 4) in registers.  Outputs are taken 16 at a time: dy [128][16] and the
// chunk of C as [8 inputs][16 outputs][DM] in LDS, the per-input stride padded
// to an odd number of elements so the 8 inputs of a wave read distinct banks.
// accumulate: add to dx (later chunks).
template <typename T, int DM, bool SEEK>
__global__ void __launch_bounds__(256)
k_dx_v(const T* __restrict__ t, const T* __restrict__ C, const T* __restrict__ dy,
       T* __restrict__ dx, int64_t B, int I, int O, int D, int d0_arg, int dn,
       int accumulate) {
  constexpr int OC = 16, CST = OC * (DM + 1) + 1;
  const int d0 = SEEK ? d0_arg : 0;
  __shared__ T ys[128][OC + 1];
  __shared__ T cs[8 * CST];
  const int tid = threadIdx.x, rr = tid >> 3, ii = tid & 7;
  const int64_t b0 = (int64_t)blockIdx.x * 128;
  const int i0 = blockIdx.y * 8;
  T g[4][DM];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int d = 0; d < DM; ++d) g[h][d] = T(0);
  for (int oc = 0; oc < O; oc += OC) {
    __syncthreads();
    for (int k = tid; k < 128 * OC; k += 256) {
      const int r = k / OC, ol = k % OC;
      const int64_t b = b0 + r;
      ys[r][ol] = (b < B && oc + ol < O) ? dy[b * O + oc + ol] : T(0);
    }
    for (int k = tid; k < 8 * OC * dn; k += 256) {
      const int il = k / (OC * dn), rem = k % (OC * dn), ol = rem / dn, d = rem % dn;
      const int i = i0 + il, o = oc + ol;
      cs[il * CST + ol * (DM + 1) + d] = (i < I && o < O) ? C[((size_t)i * O + o) * D + d0 + d] : T(0);
    }
    __syncthreads();
    for (int ol = 0; ol < OC; ++ol) {
      T a[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) a[h] = ys[rr + 32 * h][ol];
      const T* cr = cs + ii * CST + ol * (DM + 1);
#pragma unroll
      for (int d = 0; d < DM; ++d) {
        if (d < dn) {
          const T cv = cr[d];
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
    const T tv = t[b * I + i];
    const T t2 = tv + tv;
    // (up, u) = (U_{deg-2}, U_{deg-1}) at degree deg.  The first chunk starts
    // at degree 1 (T_0 has no derivative, so G[., ., 0] is never formed) from
    // (U_{-1}, U_0) = (0, 1); a later chunk advances the recurrence
    // U_{n+1} = 2t U_n - U_{n-1} from (U_{-1}, U_0) to degree d0.
    constexpr int dfirst = SEEK ? 0 : 1;
    T up = T(0), u = T(1), s = T(0);
    for (int d = 1; d < d0; ++d) {
      const T un = fma(t2, u, -up);
      up = u;
      u = un;
    }
    T deg = (T)(d0 + dfirst);  // counted in T (exact)
#pragma unroll
    for (int d = dfirst; d < DM; ++d) {
      if (d < dn) {  // dT_deg/dt = deg U_{deg-1}
        s = fma(g[h][d] * deg, u, s);
        const T un = fma(t2, u, -up);
        up = u;
        u = un;
        deg += T(1);
      }
    }
    const T v = s * (T(1) - tv * tv);
    dx[b * I + i] = SEEK && accumulate ? dx[b * I + i] + v : v;
  }
}

// dC, degrees [d0, d0 + dn): block tile 8 inputs x 128 outputs; thread
// (il, ol) = (tid / 32, tid % 32) owns outputs ol + 32 c (c < 4) of input il,
// all degrees of the chunk, so each basis recurrence serves four outputs.
// Rows are taken 32 at a time: t [32][8] and dy [32][128] in LDS.
template <typename T> struct DcWrite;
template <> struct DcWrite<float> {  // the dC write modes of the MFMA kernels
  static __device__ __forceinline__ void put(float* d, float v, const DcOut& om) { dc_write(d, v, om); }
};
template <> struct DcWrite<double> {  // store or accumulate
  static __device__ __forceinline__ void put(double* d, double v, const DcOut& om) {
    *d = om.mode == kDcAccumulate ? *d + v : v;
  }
};

template <typename T, int DM, bool SEEK>
__global__ void __launch_bounds__(256)
k_dc_v(const T* __restrict__ t, const T* __restrict__ dy, T* __restrict__ dC, int64_t B, int I,
       int O, int D, int d0_arg, int dn, DcOut om) {
  const int d0 = SEEK ? d0_arg : 0;
  __shared__ T ts[32][9];
  __shared__ T ys[32][129];
  const int tid = threadIdx.x, il = tid >> 5, ol = tid & 31;
  const int i0 = blockIdx.x * 8, o0 = blockIdx.y * 128;
  T acc[4][DM];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int d = 0; d < DM; ++d) acc[c][d] = T(0);
  for (int64_t bc = 0; bc < B; bc += 32) {
    __syncthreads();
    {
      const int r = tid >> 3, k = tid & 7;
      const int64_t b = bc + r;
      ts[r][k] = (b < B && i0 + k < I) ? t[b * I + i0 + k] : T(0);
    }
    for (int k = tid; k < 32 * 128; k += 256) {
      const int r = k >> 7, o = k & 127;
      const int64_t b = bc + r;
      ys[r][o] = (b < B && o0 + o < O) ? dy[b * O + o0 + o] : T(0);
    }
    __syncthreads();
    for (int r = 0; r < 32; ++r) {
      const T tv = ts[r][il], t2 = tv + tv;
      T yv[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) yv[c] = ys[r][ol + 32 * c];
      T tp, tc;
      cheb_seek<T>(tv, d0, tp, tc);
#pragma unroll
      for (int d = 0; d < DM; ++d) {
        if (d < dn) {
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[c][d] = fma(tc, yv[c], acc[c][d]);
          const T nx = fma(t2, tc, -tp);
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
    T* dst = dC + ((size_t)i * O + o) * D + d0;
#pragma unroll
    for (int d = 0; d < DM; ++d)
      if (d < dn) DcWrite<T>::put(dst + d, acc[c][d], om);
  }
}

// dst = float(src), src fp32 or bf16 (the coefficient copy of this path).
__global__ void __launch_bounds__(256)
k_to_f32(const void* __restrict__ src, int src_bf16, float* __restrict__ dst, int64_t n) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x)
    dst[q] = src_bf16 ? __uint_as_float((uint32_t)static_cast<const uint16_t*>(src)[q] << 16)
                      : static_cast<const float*>(src)[q];
}

static unsigned vgrid(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (unsigned)(g < 1 ? 1 : g);
}

void launch_to_f32(const void* src, bool src_bf16, float* dst, int64_t n, hipStream_t s) {
  if (n > 0)
    hipLaunchKernelGGL(k_to_f32, dim3(vgrid(n)), dim3(256), 0, s, src, src_bf16 ? 1 : 0, dst, n);
}

// Chunk size: the smallest instantiated DM that holds D, 17 above.
static int valu_dm(int D) { return D <= 3 ? 3 : D <= 5 ? 5 : D <= 9 ? 9 : kValuDM; }

template <typename T, int DM>
static void fwd_chunks(const T* t, const T* C, T* y, int64_t B, int I, int O, int D,
                       hipStream_t s) {
  const dim3 g((unsigned)((B + 63) / 64), (unsigned)((O + 63) / 64));
  for (int d0 = 0; d0 < D; d0 += DM) {
    const int dn = D - d0 < DM ? D - d0 : DM;
    if (d0 == 0)
      hipLaunchKernelGGL((k_fwd_v<T, DM, false>), g, dim3(256), 0, s, t, C, y, B, I, O, D,
                         d0, dn, 0);
    else
      hipLaunchKernelGGL((k_fwd_v<T, DM, true>), g, dim3(256), 0, s, t, C, y, B, I, O, D,
                         d0, dn, 1);
  }
}

template <typename T, int DM>
static void bwd_chunks(const T* t, const T* C, const T* dy, T* dx, T* dC, DcOut om, int64_t B,
                       int I, int O, int D, hipStream_t s) {
  for (int d0 = 0; d0 < D; d0 += DM) {
    const int dn = D - d0 < DM ? D - d0 : DM;
    if (dx && B > 0) {
      const dim3 g((unsigned)((B + 127) / 128), (unsigned)((I + 7) / 8));
      if (d0 == 0)
        hipLaunchKernelGGL((k_dx_v<T, DM, false>), g, dim3(256), 0, s, t, C, dy, dx, B, I,
                           O, D, d0, dn, 0);
      else
        hipLaunchKernelGGL((k_dx_v<T, DM, true>), g, dim3(256), 0, s, t, C, dy, dx, B, I,
                           O, D, d0, dn, 1);
    }
    if (dC) {
      const dim3 g((unsigned)((I + 7) / 8), (unsigned)((O + 127) / 128));
      if (d0 == 0)
        hipLaunchKernelGGL((k_dc_v<T, DM, false>), g, dim3(256), 0, s, t, dy, dC, B, I, O,
                           D, d0, dn, om);
      else
        hipLaunchKernelGGL((k_dc_v<T, DM, true>), g, dim3(256), 0, s, t, dy, dC, B, I, O,
                           D, d0, dn, om);
    }
  }
}

template <typename T>
void launch_forward_valu(const T* x, const T* C, T* y, T* t, int64_t B, int I, int O,
                         int deg, hipStream_t s) {
  if (B == 0) return;
  hipLaunchKernelGGL(k_tanh_v<T>, dim3(vgrid(B * I)), dim3(256), 0, s, x, t, B * I);
  const int D = deg + 1;
  switch (valu_dm(D)) {
    case 3: fwd_chunks<T, 3>(t, C, y, B, I, O, D, s); break;
    case 5: fwd_chunks<T, 5>(t, C, y, B, I, O, D, s); break;
    case 9: fwd_chunks<T, 9>(t, C, y, B, I, O, D, s); break;
    default: fwd_chunks<T, kValuDM>(t, C, y, B, I, O, D, s); break;
  }
}

template <typename T>
void launch_backward_valu(const T* t, const T* C, const T* dy, T* dx, T* dC, DcOut om, int64_t B,
                          int I, int O, int deg, hipStream_t s) {
  const int D = deg + 1;
  switch (valu_dm(D)) {
    case 3: bwd_chunks<T, 3>(t, C, dy, dx, dC, om, B, I, O, D, s); break;
    case 5: bwd_chunks<T, 5>(t, C, dy, dx, dC, om, B, I, O, D, s); break;
    case 9: bwd_chunks<T, 9>(t, C, dy, dx, dC, om, B, I, O, D, s); break;
    default: bwd_chunks<T, kValuDM>(t, C, dy, dx, dC, om, B, I, O, D, s); break;
  }
}

template void launch_forward_valu<float>(const float*, const float*, float*, float*, int64_t, int,
                                         int, int, hipStream_t);
template void launch_forward_valu<double>(const double*, const double*, double*, double*, int64_t,
                                          int, int, int, hipStream_t);
template void launch_backward_valu<float>(const float*, const float*, const float*, float*, float*,
                                          DcOut, int64_t, int, int, int, hipStream_t);
template void launch_backward_valu<double>(const double*, const double*, const double*, double*,
                                           double*, DcOut, int64_t, int, int, int, hipStream_t);

}  // namespace ckan
