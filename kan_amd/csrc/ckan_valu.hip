// The ChebyKAN layer on the vector ALU, for any degree, in fp32 or fp64:
//   forward  y[b, o]     = sum_{i, d} P_d(t[b, i]) C[i, o, d],  t = tanh(x)
//   dx       dx[b, i]    = t'(x) sum_d G[b, i, d] P_d'(t),
//                          G[b, i, d] = sum_o dy[b, o] C[i, o, d]
//   dC       dC[i, o, d] = sum_b P_d(t[b, i]) dy[b, o]
// with P_d = T_d (the Chebyshev kernels, fp32 and fp64) or, in fp32, any
// basis of a three-term recurrence P_d = (a_d u + b_d) P_{d-1} - c_d P_{d-2}
// at u = s t (the Jacobi and Hermite layers, kan/basis/jacobi.py:131-188,
// kan/basis/hermite.py:158-233), whose coefficients come from the packed
// buffer's recurrence block.  t = tanh(x), or the affine map a x + b of a
// finite-domain Hermite layer (kan/basis/hermite.py:102-112).
// It serves the fp64 layer (the reference computes in fp64 when its
// parameter is fp64: kan/layers/chebykan.py:48-51 after .double()) and fp32
// layers above the MFMA kernels' degree 16 (the reference layers take any
// degree, kan/layers/chebykan.py:21-51).  Register-tiled kernels with LDS
// staging read C in its own [I, O, D] layout.  The degree axis is taken in
// chunks of at most DM degrees (DM = 3, 5, 9 or 17, the smallest that holds
// D, and 17 above), so register arrays stay bounded for any degree: the
// forward walks the chunks inside one launch with its recurrences in
// registers; dC runs the chunks side by side in one launch (grid z), each
// block advancing its recurrences to the chunk's first degree once; dx runs
// one launch per chunk, accumulating.  t is [B, I].
#include "ckan_kernels.hpp"

#include <math.h>

namespace ckan {

constexpr int kValuDM = 17;  // degrees per chunk above degree 16

template <typename T> __device__ __forceinline__ T vtanh(T x);
template <> __device__ __forceinline__ float vtanh<float>(float x) { return tanhf(x); }
template <> __device__ __forceinline__ double vtanh<double>(double x) { return tanh(x); }

// t = tanh(x), or ima x + imb with the affine map.
template <typename T>
__global__ void __launch_bounds__(256)
k_tanh_v(const T* __restrict__ x, T* __restrict__ t, int64_t n, int imap, float ima, float imb) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x)
    t[q] = imap ? fma((T)ima, x[q], (T)imb) : vtanh<T>(x[q]);
}

// Basis recurrences.  Chebyshev (GEN = false): T_{d+1} = 2t T_d - T_{d-1},
// w = 2t, started from T_{-1} = t so that the first step gives 2t - t = t =
// T_1 exactly and every step is the same FMA.  GEN: P_{d+1} = (a_{d+1} w +
// b_{d+1}) P_d - c_{d+1} P_{d-1}, w = u = s t, started from P_{-1} = 0 (c_1 =
// 0); rs holds a[D], b[D], c[D], s, kind (0: the Chebyshev recurrence, whose
// specialised code the kernels then take).
template <typename T, bool GEN>
__device__ __forceinline__ void rec_init(T t, const T* rs, int D, T& w, T& pm, T& pc) {
  if constexpr (GEN) {
    w = (T)rs[3 * D] * t;
    pm = T(0);
  } else {
    w = t + t;
    pm = t;
  }
  pc = T(1);
}
template <typename T, bool GEN>
__device__ __forceinline__ void rec_step(T w, const T* rs, int D, int n, T& pm, T& pc) {
  T nx;
  if constexpr (GEN) {
    // read the step's coefficients here: hoisted out of the unrolled degree
    // loops they would hold 3 registers per degree for the whole kernel
    asm volatile("" ::: "memory");
    nx = fma(fma((T)rs[n], w, (T)rs[D + n]), pc, -(T)rs[2 * D + n] * pm);
  } else {
    nx = fma(w, pc, -pm);
  }
  pm = pc;
  pc = nx;
}

// The recurrence block: an fp32 block is copied into the kernel's dynamic
// LDS (rec_lds_bytes, sized by the layer's degree) before the block's first
// barrier; an fp64 block (the fp64 family layers) is read where it is,
// by wave-uniform loads, which keeps the fp64 kernels' LDS (and occupancy) as
// it is.  rec_src gives the copy to read; after the barrier, rec_generic
// tells whether the block asks for the generic recurrence (a uniform branch
// around the kernel's body, which is instantiated once per recurrence kind).
template <typename T>
__device__ __forceinline__ void stage_rec(float* rs, const T* __restrict__ rec, int D) {
  if constexpr (sizeof(T) == 4) {
    if (rec)
      for (int k = threadIdx.x; k < 3 * D + 2; k += blockDim.x) rs[k] = rec[k];
  }
}
// Dynamic LDS of a vector-ALU kernel: the fp32 recurrence block a, b, c
// (D each), scale, kind, when there is one.
template <typename T> static size_t rec_lds_bytes(const T* rec, int D) {
  return sizeof(T) == 4 && rec ? (size_t)recur_floats(D - 1) * sizeof(float) : 0;
}
template <typename T>
__device__ __forceinline__ const T* rec_src(const float* lds, const T* rec) {
  if constexpr (sizeof(T) == 4) return lds;
  else return rec;
}
template <typename T>
__device__ __forceinline__ bool rec_generic(const T* rs, const T* rec, int D) {
  return rec != nullptr && rs[3 * D + 1] != T(0);
}

// dx and dC: SEEK = false instantiations serve the first (or only) chunk (d0
// = 0, stored, not accumulated) with no seek loops in the code, as
// register-lean as a single-chunk kernel.

// Register tile widths: rows per thread of the forward (WF), of dx (WX) and
// outputs per thread of dC (WC).  The fp64 forward on chunks of up to 9
// degrees takes 8 rows: half the C values read from LDS per FMA and the basis
// recurrence spread over twice the FMAs (config-3 shape in fp64: forward 5.9
// -> 5.1 ms).  8 rows in dx measured slower (occupancy 3 -> 2) and 8 outputs
// in dC no faster, so those keep 4.
template <typename T, int DM> struct VTile {
  static constexpr int WF = (sizeof(T) == 8 && DM <= 9) ? 8 : 4;
  static constexpr int WX = 4;
  static constexpr int WC = 4;
};

// Forward: block tile 16 RT rows x 64 outputs (RT = WF), 256 threads, thread
// (tr, to) owns rows tr + 16 r (r < RT) and outputs to + 16 c (c < 4).
// Inputs are taken KI at a time (t [16 RT][KI] in LDS) and, for each input
// tile, the degree axis DM degrees at a time ([KI][DM][64 outputs] of C in
// LDS).  Above one chunk (MULTI) the recurrences of the thread's (row, input)
// pairs stay in registers from chunk to chunk, so one launch covers any
// degree without re-advancing a recurrence.
constexpr int kValuKI = 4;

// Degrees [d0, d0 + dn) of one input tile: acc += P(t) C.  The recurrence of
// (row r, input ii) is (w, pm, pc)[r][ii] at degree d0 on entry; INIT: started
// here from t, input by input (so that only one input's recurrences are live).
template <typename T, int DM, bool GEN, int RT, bool INIT>
__device__ __forceinline__ void fwd_tile(T (&acc)[RT][4], T (&w)[RT][kValuKI],
                                         T (&pm)[RT][kValuKI], T (&pc)[RT][kValuKI],
                                         const T (&ts)[16 * RT][kValuKI + 1],
                                         const T (&cs)[kValuKI][DM][64], const T* rs, int D,
                                         int d0, int dn, int tr, int to) {
#pragma unroll
  for (int ii = 0; ii < kValuKI; ++ii) {
    if constexpr (INIT) {
#pragma unroll
      for (int r = 0; r < RT; ++r) rec_init<T, GEN>(ts[tr + 16 * r][ii], rs, D, w[r][ii], pm[r][ii], pc[r][ii]);
    }
    for (int d = 0; d < dn; ++d) {  // rolled: measured faster than unrolled here
      T cv[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) cv[c] = cs[ii][d][to + 16 * c];
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = fma(pc[r][ii], cv[c], acc[r][c]);
#pragma unroll
      for (int r = 0; r < RT; ++r) rec_step<T, GEN>(w[r][ii], rs, D, d0 + d + 1, pm[r][ii], pc[r][ii]);
    }
  }
}

// The forward kernel's body for one recurrence kind (uniform over the launch).
template <typename T, int DM, bool GEN, bool MULTI>
__device__ __forceinline__ void fwd_body(const T* __restrict__ t, const T* __restrict__ C,
                                         T* __restrict__ y, int64_t B, int I, int O, int D,
                                         const T* rs,
                                         T (&ts)[16 * VTile<T, DM>::WF][kValuKI + 1],
                                         T (&cs)[kValuKI][DM][64]) {
  constexpr int KI = kValuKI, RT = VTile<T, DM>::WF, BR = 16 * RT;
  const int tid = threadIdx.x, tr = tid >> 4, to = tid & 15;
  const int64_t b0 = (int64_t)blockIdx.x * BR;
  const int o0 = blockIdx.y * 64;
  auto stage_c = [&](int i0, int d0, int dn) {
    for (int k = tid; k < KI * 64 * dn; k += 256) {
      const int ii = k / (64 * dn), rem = k % (64 * dn), ol = rem / dn, d = rem % dn;
      const int i = i0 + ii, o = o0 + ol;
      cs[ii][d][ol] = (i < I && o < O) ? C[((size_t)i * O + o) * D + d0 + d] : T(0);
    }
  };
  T acc[RT][4];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r][c] = T(0);
  for (int i0 = 0; i0 < I; i0 += KI) {
    __syncthreads();
    for (int k = tid; k < BR * KI; k += 256) {
      const int r = k / KI, ii = k % KI;
      const int64_t b = b0 + r;
      ts[r][ii] = (b < B && i0 + ii < I) ? t[b * I + i0 + ii] : T(0);
    }
    if (!MULTI) stage_c(i0, 0, D);
    __syncthreads();
    T w[RT][KI], pm[RT][KI], pc[RT][KI];
    if constexpr (!MULTI) {
      fwd_tile<T, DM, GEN, RT, true>(acc, w, pm, pc, ts, cs, rs, D, 0, D, tr, to);
    } else {
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int ii = 0; ii < KI; ++ii)
          rec_init<T, GEN>(ts[tr + 16 * r][ii], rs, D, w[r][ii], pm[r][ii], pc[r][ii]);
      for (int d0 = 0; d0 < D; d0 += DM) {
        const int dn = D - d0 < DM ? D - d0 : DM;
        __syncthreads();  // the previous chunk's reads of cs are done
        stage_c(i0, d0, dn);
        __syncthreads();
        fwd_tile<T, DM, GEN, RT, false>(acc, w, pm, pc, ts, cs, rs, D, d0, dn, tr, to);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int64_t b = b0 + tr + 16 * r;
    if (b >= B) continue;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int o = o0 + to + 16 * c;
      if (o < O) y[b * O + o] = acc[r][c];
    }
  }
}

// MULTI: more degrees than one chunk of DM.
template <typename T, int DM, bool MULTI>
__global__ void __launch_bounds__(256)
k_fwd_v(const T* __restrict__ t, const T* __restrict__ C, T* __restrict__ y, int64_t B, int I,
        int O, int D, const T* __restrict__ rec) {
  __shared__ T ts[16 * VTile<T, DM>::WF][kValuKI + 1];
  __shared__ T cs[kValuKI][DM][64];
  extern __shared__ float rs_l[];  // the fp32 recurrence block (rec_lds_bytes)
  stage_rec<T>(rs_l, rec, D);
  const T* rs = rec_src<T>(rs_l, rec);
  __syncthreads();
  if (rec_generic<T>(rs, rec, D))
    fwd_body<T, DM, true, MULTI>(t, C, y, B, I, O, D, rs, ts, cs);
  else
    fwd_body<T, DM, false, MULTI>(t, C, y, B, I, O, D, rs, ts, cs);
}

// dx, degrees [d0, d0 + dn): block tile 32 HT rows x 8 inputs (HT = WX);
// thread (rr, ii) = (tid / 8, tid % 8) owns G[b, i, d0 .. d0+dn) of rows
// rr + 32 h (h < HT) in registers.  Outputs are taken 16 at a time: dy
// [32 HT][16] and the chunk of C as [8 inputs][16 outputs][DM] in LDS, the
// per-input stride padded to an odd number of elements so the 8 inputs of a
// wave read distinct banks.  accumulate: add to dx (later chunks).  The
// epilogue sums G_d P_d'(t) (Chebyshev: d U_{d-1}(t); GEN: the differentiated
// recurrence, times s) and applies t'(x): 1 - t^2, or ima with the affine map.

// The dx epilogue for one recurrence kind: dx[b, i] = t'(x) sum_d G_d P_d'(t)
// for the thread's rows rr + 32 h.
template <typename T, int DM, bool SEEK, bool GEN, int HT>
__device__ __forceinline__ void dx_epilogue(const T* __restrict__ t, T* __restrict__ dx,
                                            const T (&g)[HT][DM], int64_t B, int I, int D, int d0,
                                            int dn, int accumulate, const T* rs, int imap,
                                            float ima) {
  const int tid = threadIdx.x, rr = tid >> 3, ii = tid & 7;
  const int64_t b0 = (int64_t)blockIdx.x * (32 * HT);
  const int i = blockIdx.y * 8 + ii;
  if (i >= I) return;
#pragma unroll
  for (int h = 0; h < HT; ++h) {
    const int64_t b = b0 + rr + 32 * h;
    if (b >= B) continue;
    const T tv = t[b * I + i];
    T s = T(0);
    if constexpr (GEN) {
      // (pm, pc) = (P_{n-1}, P_n), (qm, qc) their derivatives in u, from n = 0:
      // P_n' = a_n P_{n-1} + (a_n u + b_n) P_{n-1}' - c_n P_{n-2}'
      const T u = (T)rs[3 * D] * tv;
      T pm = T(0), pc = T(1), qm = T(0), qc = T(0);
      auto step = [&](int n) {
        asm volatile("" ::: "memory");  // coefficients read per step, not hoisted
        const T an = (T)rs[n], fn = fma(an, u, (T)rs[D + n]), cn = (T)rs[2 * D + n];
        const T pn = fma(fn, pc, -cn * pm);
        const T qn = fma(an, pc, fma(fn, qc, -cn * qm));
        pm = pc;
        pc = pn;
        qm = qc;
        qc = qn;
      };
      for (int n = 1; n <= d0; ++n) step(n);
#pragma unroll
      for (int d = 0; d < DM; ++d) {
        if (d < dn) {
          s = fma(g[h][d], qc, s);
          step(d0 + d + 1);
        }
      }
      s *= (T)rs[3 * D];  // du/dt
    } else {
      const T t2 = tv + tv;
      // (up, u) = (U_{deg-2}, U_{deg-1}) at degree deg.  The first chunk
      // starts at degree 1 (T_0 has no derivative, so G[., ., 0] is never
      // formed) from (U_{-1}, U_0) = (0, 1); a later chunk advances the
      // recurrence U_{n+1} = 2t U_n - U_{n-1} from (U_{-1}, U_0) to degree d0.
      constexpr int dfirst = SEEK ? 0 : 1;
      T up = T(0), u = T(1);
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
    }
    const T v = s * (imap ? (T)ima : T(1) - tv * tv);
    dx[b * I + i] = SEEK && accumulate ? dx[b * I + i] + v : v;
  }
}

// The dx kernel's body; FULL: the chunk holds DM degrees (dn == DM).
template <typename T, int DM, bool SEEK, bool FULL, int CST, int BR>
__device__ __forceinline__ void dx_body(const T* __restrict__ t, const T* __restrict__ C,
                                        const T* __restrict__ dy, T* __restrict__ dx, int64_t B,
                                        int I, int O, int D, int d0, int dn_arg, int accumulate,
                                        const T* __restrict__ rec, int imap, float ima,
                                        T (&ys)[BR][17], T (&cs)[8 * CST], const T* rs) {
  constexpr int OC = 16, HT = BR / 32;
  const int dn = FULL ? DM : dn_arg;
  const int tid = threadIdx.x, rr = tid >> 3, ii = tid & 7;
  const int64_t b0 = (int64_t)blockIdx.x * BR;
  const int i0 = blockIdx.y * 8;
  T g[HT][DM];
#pragma unroll
  for (int h = 0; h < HT; ++h)
#pragma unroll
    for (int d = 0; d < DM; ++d) g[h][d] = T(0);
  for (int oc = 0; oc < O; oc += OC) {
    __syncthreads();
    for (int k = tid; k < BR * OC; k += 256) {
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
      T a[HT];
#pragma unroll
      for (int h = 0; h < HT; ++h) a[h] = ys[rr + 32 * h][ol];
      const T* cr = cs + ii * CST + ol * (DM + 1);
#pragma unroll
      for (int d = 0; d < DM; ++d) {
        if (d < dn) {
          const T cv = cr[d];
#pragma unroll
          for (int h = 0; h < HT; ++h) g[h][d] = fma(a[h], cv, g[h][d]);
        }
      }
    }
  }
  if (O == 0) __syncthreads();  // the recurrence block is staged before its first use
  if (rec_generic<T>(rs, rec, D))
    dx_epilogue<T, DM, SEEK, true, HT>(t, dx, g, B, I, D, d0, dn, accumulate, rs, imap, ima);
  else
    dx_epilogue<T, DM, SEEK, false, HT>(t, dx, g, B, I, D, d0, dn, accumulate, rs, imap, ima);
}

template <typename T, int DM, bool SEEK>
__global__ void __launch_bounds__(256)
k_dx_v(const T* __restrict__ t, const T* __restrict__ C, const T* __restrict__ dy,
       T* __restrict__ dx, int64_t B, int I, int O, int D, int d0_arg, int dn, int accumulate,
       const T* __restrict__ rec, int imap, float ima) {
  constexpr int OC = 16, CST = OC * (DM + 1) + 1, BR = 32 * VTile<T, DM>::WX;
  const int d0 = SEEK ? d0_arg : 0;
  __shared__ T ys[BR][OC + 1];
  __shared__ T cs[8 * CST];
  extern __shared__ float rs_l[];  // the fp32 recurrence block (rec_lds_bytes)
  stage_rec<T>(rs_l, rec, D);
  const T* rs = rec_src<T>(rs_l, rec);
  if (dn == DM)
    dx_body<T, DM, SEEK, true, CST, BR>(t, C, dy, dx, B, I, O, D, d0, dn, accumulate, rec, imap,
                                        ima, ys, cs, rs);
  else
    dx_body<T, DM, SEEK, false, CST, BR>(t, C, dy, dx, B, I, O, D, d0, dn, accumulate, rec, imap,
                                         ima, ys, cs, rs);
}

// dC, degrees [d0, d0 + dn): block tile 8 inputs x 32 CT outputs (CT = WC);
// thread (il, ol) = (tid / 32, tid % 32) owns outputs ol + 32 c (c < CT) of
// input il, all degrees of the chunk, so each basis recurrence serves CT
// outputs.  Rows are taken 32 at a time: t [32][8] and dy [32][32 CT] in LDS.
template <typename T> struct DcWrite;
template <> struct DcWrite<float> {  // the dC write modes of the MFMA kernels
  static __device__ __forceinline__ void put(float* d, float v, const DcOut& om) { dc_write(d, v, om); }
};
template <> struct DcWrite<double> {  // store or accumulate
  static __device__ __forceinline__ void put(double* d, double v, const DcOut& om) {
    *d = om.mode == kDcAccumulate ? *d + v : v;
  }
};

// One LDS tile of dC (32 rows): acc += P(t) dy.  SEEK: the recurrences start
// at degree d0 from sst, [3][32][9] (w, P_{d0-1}, P_{d0} of each (row,
// input), advanced once per block instead of once per output thread).
template <typename T, int DM, bool GEN, int CT, bool SEEK>
__device__ __forceinline__ void dc_tile(T (&acc)[CT][DM], const T (&ts)[32][9], const T* sst,
                                        const T (&ys)[32][32 * CT + 1], const T* rs, int D,
                                        int d0, int dn, int il, int ol) {
  for (int r = 0; r < 32; ++r) {
    T yv[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) yv[c] = ys[r][ol + 32 * c];
    T w, pm, pc;
    if constexpr (SEEK) {
      w = sst[r * 9 + il];
      pm = sst[288 + r * 9 + il];
      pc = sst[576 + r * 9 + il];
    } else {
      rec_init<T, GEN>(ts[r][il], rs, D, w, pm, pc);
    }
#pragma unroll
    for (int d = 0; d < DM; ++d) {
      if (d < dn) {
#pragma unroll
        for (int c = 0; c < CT; ++c) acc[c][d] = fma(pc, yv[c], acc[c][d]);
        rec_step<T, GEN>(w, rs, D, d0 + d + 1, pm, pc);
      }
    }
  }
}

// The dC kernel's body for one recurrence kind (the kind is uniform over the
// launch; one body per kind keeps each one's register allocation its own).
template <typename T, int DM, bool SEEK, bool GEN, bool FULL>
__device__ __forceinline__ void dc_body(const T* __restrict__ t, const T* __restrict__ dy,
                                        T* __restrict__ dC, int64_t B, int I, int O, int D,
                                        int d0, int dn_arg, const DcOut& om, const T* rs,
                                        T (&ts)[32][9], T* sst,
                                        T (&ys)[32][32 * VTile<T, DM>::WC + 1]) {
  constexpr int CT = VTile<T, DM>::WC, BO = 32 * CT;
  const int dn = FULL ? DM : dn_arg;
  const int tid = threadIdx.x, il = tid >> 5, ol = tid & 31;
  const int i0 = blockIdx.x * 8, o0 = blockIdx.y * BO;
  T acc[CT][DM];
#pragma unroll
  for (int c = 0; c < CT; ++c)
#pragma unroll
    for (int d = 0; d < DM; ++d) acc[c][d] = T(0);
  for (int64_t bc = 0; bc < B; bc += 32) {
    __syncthreads();
    {
      const int r = tid >> 3, k = tid & 7;
      const int64_t b = bc + r;
      ts[r][k] = (b < B && i0 + k < I) ? t[b * I + i0 + k] : T(0);
    }
    for (int k = tid; k < 32 * BO; k += 256) {
      const int r = k / BO, o = k % BO;
      const int64_t b = bc + r;
      ys[r][o] = (b < B && o0 + o < O) ? dy[b * O + o0 + o] : T(0);
    }
    __syncthreads();
    if constexpr (SEEK) {  // each thread advances one (row, input) recurrence to degree d0
      const int r = tid >> 3, k = tid & 7;
      T w, pm, pc;
      rec_init<T, GEN>(ts[r][k], rs, D, w, pm, pc);
      for (int n = 1; n <= d0; ++n) rec_step<T, GEN>(w, rs, D, n, pm, pc);
      sst[r * 9 + k] = w;
      sst[288 + r * 9 + k] = pm;
      sst[576 + r * 9 + k] = pc;
      __syncthreads();
    }
    dc_tile<T, DM, GEN, CT, SEEK>(acc, ts, sst, ys, rs, D, d0, dn, il, ol);
  }
  const int i = i0 + il;
  if (i >= I) return;
#pragma unroll
  for (int c = 0; c < CT; ++c) {
    const int o = o0 + ol + 32 * c;
    if (o >= O) continue;
    T* dst = dC + ((size_t)i * O + o) * D + d0;
#pragma unroll
    for (int d = 0; d < DM; ++d)
      if (d < dn) DcWrite<T>::put(dst + d, acc[c][d], om);
  }
}

template <typename T, int DM, bool SEEK>
__global__ void __launch_bounds__(256)
k_dc_v(const T* __restrict__ t, const T* __restrict__ dy, T* __restrict__ dC, int64_t B, int I,
       int O, int D, int d0_arg, int dn_arg, DcOut om, const T* __restrict__ rec) {
  // SEEK: every chunk of the degree axis in one launch, chunk blockIdx.z (the
  // chunks write disjoint degrees of dC, so they run side by side)
  const int d0 = SEEK ? d0_arg + (int)blockIdx.z * DM : 0;
  const int dn = SEEK ? min(DM, D - d0) : dn_arg;
  __shared__ T ts[32][9];
  __shared__ T sst[SEEK ? 3 * 32 * 9 : 1];  // seek states, read only with SEEK
  __shared__ T ys[32][32 * VTile<T, DM>::WC + 1];
  extern __shared__ float rs_l[];  // the fp32 recurrence block (rec_lds_bytes)
  stage_rec<T>(rs_l, rec, D);
  const T* rs = rec_src<T>(rs_l, rec);
  __syncthreads();
  const bool gen = rec_generic<T>(rs, rec, D), full = dn == DM;
  if (gen && full) dc_body<T, DM, SEEK, true, true>(t, dy, dC, B, I, O, D, d0, dn, om, rs, ts, sst, ys);
  else if (gen) dc_body<T, DM, SEEK, true, false>(t, dy, dC, B, I, O, D, d0, dn, om, rs, ts, sst, ys);
  else if (full) dc_body<T, DM, SEEK, false, true>(t, dy, dC, B, I, O, D, d0, dn, om, rs, ts, sst, ys);
  else dc_body<T, DM, SEEK, false, false>(t, dy, dC, B, I, O, D, d0, dn, om, rs, ts, sst, ys);
}

// dst = float(src) (or dst += float(src)), src fp32 or bf16: the coefficient
// copy of this path.
__global__ void __launch_bounds__(256)
k_to_f32(const void* __restrict__ src, int src_bf16, float* __restrict__ dst, int64_t n,
         int accumulate) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x) {
    const float v = src_bf16 ? __uint_as_float((uint32_t)static_cast<const uint16_t*>(src)[q] << 16)
                             : static_cast<const float*>(src)[q];
    dst[q] = accumulate ? dst[q] + v : v;
  }
}

static unsigned vgrid(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (unsigned)(g < 1 ? 1 : g);
}

void launch_to_f32(const void* src, bool src_bf16, float* dst, int64_t n, hipStream_t s,
                   bool accumulate) {
  if (n > 0)
    hipLaunchKernelGGL(k_to_f32, dim3(vgrid(n)), dim3(256), 0, s, src, src_bf16 ? 1 : 0, dst, n,
                       accumulate ? 1 : 0);
}

// Chunk size: the smallest instantiated DM that holds D, 17 above.
static int valu_dm(int D) { return D <= 3 ? 3 : D <= 5 ? 5 : D <= 9 ? 9 : kValuDM; }

template <typename T, int DM>
static void fwd_launch(const T* t, const T* C, T* y, int64_t B, int I, int O, int D,
                       const T* rec, hipStream_t s) {
  constexpr int BR = 16 * VTile<T, DM>::WF;
  const dim3 g((unsigned)((B + BR - 1) / BR), (unsigned)((O + 63) / 64));
  if constexpr (DM == kValuDM) {  // the only chunk size with more degrees than one chunk
    if (D > DM) {
      hipLaunchKernelGGL((k_fwd_v<T, DM, true>), g, dim3(256), rec_lds_bytes(rec, D), s, t, C, y,
                         B, I, O, D, rec);
      return;
    }
  }
  hipLaunchKernelGGL((k_fwd_v<T, DM, false>), g, dim3(256), rec_lds_bytes(rec, D), s, t, C, y, B,
                     I, O, D, rec);
}

template <typename T, int DM>
static void bwd_chunks(const T* t, const T* C, const T* dy, T* dx, T* dC, DcOut om, int64_t B,
                       int I, int O, int D, const T* rec, int imap, float ima, hipStream_t s) {
  for (int d0 = 0; d0 < D; d0 += DM) {
    const int dn = D - d0 < DM ? D - d0 : DM;
    if (dx && B > 0) {
      constexpr int BR = 32 * VTile<T, DM>::WX;
      const dim3 g((unsigned)((B + BR - 1) / BR), (unsigned)((I + 7) / 8));
      if (d0 == 0)
        hipLaunchKernelGGL((k_dx_v<T, DM, false>), g, dim3(256), rec_lds_bytes(rec, D), s, t, C,
                           dy, dx, B, I, O, D, d0, dn, 0, rec, imap, ima);
      else
        hipLaunchKernelGGL((k_dx_v<T, DM, true>), g, dim3(256), rec_lds_bytes(rec, D), s, t, C,
                           dy, dx, B, I, O, D, d0, dn, 1, rec, imap, ima);
    }
  }
  if (dC) {  // one launch: the chunks of the degree axis side by side (grid z)
    constexpr int BO = 32 * VTile<T, DM>::WC;
    const int nch = (D + DM - 1) / DM;
    const dim3 g((unsigned)((I + 7) / 8), (unsigned)((O + BO - 1) / BO), (unsigned)nch);
    if (nch == 1)
      hipLaunchKernelGGL((k_dc_v<T, DM, false>), g, dim3(256), rec_lds_bytes(rec, D), s, t, dy,
                         dC, B, I, O, D, 0, D, om, rec);
    else
      hipLaunchKernelGGL((k_dc_v<T, DM, true>), g, dim3(256), rec_lds_bytes(rec, D), s, t, dy,
                         dC, B, I, O, D, 0, DM, om, rec);
  }
}

template <typename T>
void launch_forward_valu(const T* x, const T* C, T* y, T* t, int64_t B, int I, int O, int deg,
                         hipStream_t s, const T* rec, int imap, float ima, float imb) {
  if (B == 0) return;
  hipLaunchKernelGGL(k_tanh_v<T>, dim3(vgrid(B * I)), dim3(256), 0, s, x, t, B * I, imap, ima, imb);
  const int D = deg + 1;
  switch (valu_dm(D)) {
    case 3: fwd_launch<T, 3>(t, C, y, B, I, O, D, rec, s); break;
    case 5: fwd_launch<T, 5>(t, C, y, B, I, O, D, rec, s); break;
    case 9: fwd_launch<T, 9>(t, C, y, B, I, O, D, rec, s); break;
    default: fwd_launch<T, kValuDM>(t, C, y, B, I, O, D, rec, s); break;
  }
}

template <typename T>
void launch_backward_valu(const T* t, const T* C, const T* dy, T* dx, T* dC, DcOut om, int64_t B,
                          int I, int O, int deg, hipStream_t s, const T* rec, int imap,
                          float ima) {
  const int D = deg + 1;
  switch (valu_dm(D)) {
    case 3: bwd_chunks<T, 3>(t, C, dy, dx, dC, om, B, I, O, D, rec, imap, ima, s); break;
    case 5: bwd_chunks<T, 5>(t, C, dy, dx, dC, om, B, I, O, D, rec, imap, ima, s); break;
    case 9: bwd_chunks<T, 9>(t, C, dy, dx, dC, om, B, I, O, D, rec, imap, ima, s); break;
    default: bwd_chunks<T, kValuDM>(t, C, dy, dx, dC, om, B, I, O, D, rec, imap, ima, s); break;
  }
}

template void launch_forward_valu<float>(const float*, const float*, float*, float*, int64_t, int,
                                         int, int, hipStream_t, const float*, int, float, float);
template void launch_forward_valu<double>(const double*, const double*, double*, double*, int64_t,
                                          int, int, int, hipStream_t, const double*, int, float,
                                          float);
template void launch_backward_valu<float>(const float*, const float*, const float*, float*, float*,
                                          DcOut, int64_t, int, int, int, hipStream_t, const float*,
                                          int, float);
template void launch_backward_valu<double>(const double*, const double*, const double*, double*,
                                           double*, DcOut, int64_t, int, int, int, hipStream_t,
                                           const double*, int, float);

}  // namespace ckan
