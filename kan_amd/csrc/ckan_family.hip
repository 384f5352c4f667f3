// Other orthogonal-polynomial bases of the reference (Jacobi, Hermite) served
// by the Chebyshev kernels.  A family P_0..P_deg evaluated at s * tanh(x) is a
// polynomial of degree <= deg in u = tanh(x), so
//   sum_n C[i, o, n] P_n(s u) = sum_k C'[i, o, k] T_k(u),   C' = C M,
// with the lower-triangular change of basis P_n(s u) = sum_k M[n, k] T_k(u).
// The forward and the input gradient are the ChebyKAN layer's with C'; the
// coefficient gradient is dC = dC' M^T.  M is built here exactly (fp64) from
// the family's three-term recurrence; this file also holds the kernels of
// that transform and of the materialised family basis.
#include "chebykan.h"
#include "ckan_kernels.hpp"

#include <math.h>

#include <vector>

namespace ckan {

// Recurrences of kan/basis/jacobi.py:147-188 (P^(alpha,beta)_n, written as
// (a_n t + b_n) P_{n-1} - c_n P_{n-2}), kan/basis/hermite.py:158-193
// (physicists' H_n) and :195-233 (probabilists' He_n), and T_n itself.
// P_n = (a_n t + b_n) P_{n-1} - c_n P_{n-2} (n >= 1, c_1 = 0): the
// coefficients of degree n of a ckan_basis_family (host and device; the
// families' standard recurrences).  False for an unknown family or invalid
// Jacobi parameters.
__host__ __device__ bool recur_coef(int family, int n, double alpha, double beta, double* a,
                                    double* b, double* c) {
  *a = *b = *c = 0.0;
  if (family == CKAN_BASIS_JACOBI &&
      (!(alpha > -1.0) || !(beta > -1.0) || !isfinite(alpha) || !isfinite(beta)))
    return false;
  if (family != CKAN_BASIS_CHEBYSHEV && family != CKAN_BASIS_JACOBI &&
      family != CKAN_BASIS_HERMITE && family != CKAN_BASIS_HERMITE_E)
    return false;
  if (n < 1) return true;
  switch (family) {
    case CKAN_BASIS_CHEBYSHEV:
      *a = n == 1 ? 1.0 : 2.0;
      *c = n == 1 ? 0.0 : 1.0;
      return true;
    case CKAN_BASIS_JACOBI: {
      const double ab = alpha + beta;
      if (n == 1) {
        *a = (ab + 2.0) / 2.0;
        *b = (alpha - beta) / 2.0;
        return true;
      }
      const double ct = 2.0 * n + ab - 1.0;
      const double den = 2.0 * n * (n + ab) * (2.0 * n + ab - 2.0);
      *a = ct * (2.0 * n + ab) * (2.0 * n + ab - 2.0) / den;
      *b = ct * (alpha * alpha - beta * beta) / den;
      *c = 2.0 * (n + alpha - 1.0) * (n + beta - 1.0) * (2.0 * n + ab) / den;
      return true;
    }
    case CKAN_BASIS_HERMITE:
      *a = 2.0;
      *c = n == 1 ? 0.0 : 2.0 * (n - 1);
      return true;
    case CKAN_BASIS_HERMITE_E:
      *a = 1.0;
      *c = n == 1 ? 0.0 : (double)(n - 1);
      return true;
    default:
      return false;
  }
}

bool family_recurrence(int family, int degree, double alpha, double beta, double* a, double* b,
                       double* c) {
  if (degree < 0 || degree >= kMaxD) return false;
  for (int n = 0; n < kMaxD; ++n) a[n] = b[n] = c[n] = 0.0;
  for (int n = 1; n <= degree; ++n)
    if (!recur_coef(family, n, alpha, beta, a + n, b + n, c + n)) return false;
  return recur_coef(family, 0, alpha, beta, a, b, c);  // also checks the family at degree 0
}

// The recurrence block of a vector-ALU packed buffer: a[D], b[D], c[D], the
// basis scale s (P_n is evaluated at s * t) and the kind: 0 for the Chebyshev
// basis at scale 1 (the kernels' specialised recurrence), 1 otherwise.
__global__ void k_write_recur(float* __restrict__ rec, int family, double alpha, double beta, int D,
                              float scale) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n < D) {
    double a, b, c;
    recur_coef(family, n, alpha, beta, &a, &b, &c);
    rec[n] = (float)a;
    rec[D + n] = (float)b;
    rec[2 * D + n] = (float)c;
  }
  if (n == 0) {
    rec[3 * D] = scale;
    rec[3 * D + 1] = (family == CKAN_BASIS_CHEBYSHEV && scale == 1.0f) ? 0.0f : 1.0f;
  }
}

void launch_write_recur(float* rec, int family, double alpha, double beta, int degree, float scale,
                        hipStream_t s) {
  const int D = degree + 1;
  hipLaunchKernelGGL(k_write_recur, dim3((unsigned)((D + 255) / 256)), dim3(256), 0, s, rec, family,
                     alpha, beta, D, scale);
}

// The same block in fp64, for the fp64 family layers.
__global__ void k_write_recur_f64(double* __restrict__ rec, int family, double alpha, double beta,
                                  int D, double scale) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n < D) {
    double a, b, c;
    recur_coef(family, n, alpha, beta, &a, &b, &c);
    rec[n] = a;
    rec[D + n] = b;
    rec[2 * D + n] = c;
  }
  if (n == 0) {
    rec[3 * D] = scale;
    rec[3 * D + 1] = (family == CKAN_BASIS_CHEBYSHEV && scale == 1.0) ? 0.0 : 1.0;
  }
}

void launch_write_recur_f64(double* rec, int family, double alpha, double beta, int degree,
                            double scale, hipStream_t s) {
  const int D = degree + 1;
  hipLaunchKernelGGL(k_write_recur_f64, dim3((unsigned)((D + 255) / 256)), dim3(256), 0, s, rec,
                     family, alpha, beta, D, scale);
}

// The recurrence run on Chebyshev coefficient vectors: multiplication by u is
// u T_0 = T_1 and u T_k = (T_{k+1} + T_{k-1}) / 2 for k >= 1.
void family_to_chebyshev(const double* a, const double* b, const double* c, int degree,
                         double scale, double* M) {
  const int D = degree + 1;
  std::vector<double> v((size_t)D * D, 0.0);  // v[n * D + k]
  auto mul_u = [&](const double* src, double* dst, int deg_src) {
    for (int k = 0; k <= deg_src + 1 && k < D; ++k) dst[k] = 0.0;
    for (int k = 0; k <= deg_src; ++k) {
      if (src[k] == 0.0) continue;
      if (k == 0) {
        dst[1] += src[0];
      } else {
        dst[k + 1] += 0.5 * src[k];
        dst[k - 1] += 0.5 * src[k];
      }
    }
  };
  v[0] = 1.0;
  std::vector<double> uv(D + 1, 0.0);
  for (int n = 1; n < D; ++n) {
    const double* p1 = &v[(size_t)(n - 1) * D];
    double* out = &v[(size_t)n * D];
    mul_u(p1, uv.data(), n - 1);
    for (int k = 0; k <= n; ++k) {
      double x = a[n] * scale * uv[k] + b[n] * (k <= n - 1 ? p1[k] : 0.0);
      if (n >= 2 && k <= n - 2) x -= c[n] * v[(size_t)(n - 2) * D + k];
      out[k] = x;
    }
  }
  for (int i = 0; i < D * D; ++i) M[i] = v[i];
}

// d/dx of a Chebyshev series in t = tanh x: p -> (1 - t^2) p'(t).  p' by the
// Chebyshev derivative recurrence b_{k-1} = b_{k+1} + 2 k a_k (b_0 halved);
// (1 - t^2) q = q - u (u q) with the multiplication by u of family_to_chebyshev.
static void chebyshev_dx(const double* a, int deg, double* out /* deg + 2 */) {
  std::vector<double> b(deg + 2, 0.0), u1(deg + 2, 0.0), u2(deg + 3, 0.0);
  for (int k = deg; k >= 1; --k) b[k - 1] = b[k + 1] + 2.0 * k * a[k];
  b[0] *= 0.5;  // p' has degree deg - 1
  auto mul_u = [](const double* src, int dsrc, double* dst) {
    for (int k = 0; k <= dsrc + 1; ++k) dst[k] = 0.0;
    for (int k = 0; k <= dsrc; ++k) {
      if (k == 0) dst[1] += src[0];
      else { dst[k + 1] += 0.5 * src[k]; dst[k - 1] += 0.5 * src[k]; }
    }
  };
  const int dq = deg - 1;  // degree of p'
  if (dq < 0) {
    for (int k = 0; k <= deg + 1; ++k) out[k] = 0.0;
    return;
  }
  mul_u(b.data(), dq, u1.data());      // degree dq + 1
  mul_u(u1.data(), dq + 1, u2.data()); // degree dq + 2 = deg + 1
  for (int k = 0; k <= deg + 1; ++k) out[k] = (k <= dq ? b[k] : 0.0) - u2[k];
}

bool affine_derivative_to_chebyshev(const double* M, int degree, int order, double a,
                                    double* R) {
  if (degree < 0 || order < 0) return false;
  const int D = degree + 1, DO = D + order;
  double am = 1.0;
  for (int s = 0; s < order; ++s) am *= a;
  std::vector<double> cur(D + 2, 0.0), nxt(D + 2, 0.0);
  for (int n = 0; n < D; ++n) {
    for (int k = 0; k < D + 2; ++k) cur[k] = k < D ? M[n * D + k] : 0.0;
    for (int s = 0; s < order; ++s) {
      // d/du of sum_k c_k T_k(u): e_{k-1} = e_{k+1} + 2 k c_k (k = deg..1), e_0 halved
      for (int k = 0; k < D + 2; ++k) nxt[k] = 0.0;
      for (int k = degree; k >= 1; --k) nxt[k - 1] = nxt[k + 1] + 2.0 * k * cur[k];
      nxt[0] *= 0.5;
      cur.swap(nxt);
    }
    for (int k = 0; k < DO; ++k) R[(size_t)n * DO + k] = k < D ? am * cur[k] : 0.0;
  }
  return true;
}

bool derivative_to_chebyshev(const double* M, int degree, int order, double* R) {
  if (degree < 0 || order < 0) return false;
  const int D = degree + 1, DO = D + order;
  std::vector<double> cur(DO, 0.0), nxt(DO + 1, 0.0);
  for (int n = 0; n < D; ++n) {
    for (int k = 0; k < DO; ++k) cur[k] = k < D ? M[n * D + k] : 0.0;
    int deg = degree;
    for (int s = 0; s < order; ++s) {
      chebyshev_dx(cur.data(), deg, nxt.data());
      ++deg;
      for (int k = 0; k < DO; ++k) cur[k] = k <= deg ? nxt[k] : 0.0;
    }
    for (int k = 0; k < DO; ++k) R[(size_t)n * DO + k] = cur[k];
  }
  return true;
}

// out[q, k] = sum_n in[q, n] r[n][k].  One thread per row; with transposed_o
// the thread of row q = i * O + o writes [o][k][i] (consecutive threads take
// consecutive i, so those stores coalesce).
__global__ void __launch_bounds__(256)
k_coeff_xform(const float* __restrict__ in, float* __restrict__ out, int64_t rows, int din,
              int dout, int tO, BasisXform r) {
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (t >= rows) return;
  int64_t q = t;
  int64_t o = 0, i = 0, I = 0;
  if (tO > 0) {
    I = rows / tO;
    o = t / I;
    i = t - o * I;
    q = i * tO + o;
  }
  float v[kMaxD];
#pragma unroll
  for (int n = 0; n < kMaxD; ++n) v[n] = n < din ? in[q * din + n] : 0.0f;
  for (int k = 0; k < dout; ++k) {
    float acc = 0.0f;
#pragma unroll
    for (int n = 0; n < kMaxD; ++n) acc = fmaf(v[n], r.m[n * kMaxD + k], acc);
    if (tO > 0) out[(o * dout + k) * I + i] = acc;
    else out[q * dout + k] = acc;
  }
}

// jac[b, o, i] = sum_k c1t[o][k][i] T_k(t[b, i]), t the layer's input map of
// x (tanh, or the affine map): block (i-block, b), one input per thread, the
// T_k in registers, a loop over outputs.
template <int DM>
__global__ void __launch_bounds__(256)
k_jacobian(const float* __restrict__ x, const float* __restrict__ c1t, float* __restrict__ jac,
           int64_t B, int I, int O, int dout, int imap, float ima, float imb) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (i >= I) return;
  const float t = input_map(x[b * I + i], imap, ima, imb);
  float T[DM];
  T[0] = 1.0f;
  if (DM > 1) T[1] = t;
#pragma unroll
  for (int k = 2; k < DM; ++k) T[k] = fmaf(2.0f * t, T[k - 1], -T[k - 2]);
  for (int o = 0; o < O; ++o) {
    const float* c = c1t + (size_t)o * dout * I + i;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < DM; ++k)
      if (k < dout) acc = fmaf(c[(size_t)k * I], T[k], acc);
    jac[((size_t)b * O + o) * I + i] = acc;
  }
}

// g[q, n] = sum_{k <= n} dcheb[q, k] m[n][k] over rows q of D values, written
// into dc by om (stored, accumulated, or applied as an SGD / Adam step with dc
// the parameter and om.base == dc).  A block takes 256 consecutive rows: one
// contiguous run of 256 * D floats, moved with float4 accesses when aligned
// and staged in LDS (odd D: the per-row reads hit distinct banks).  Every
// load of a block precedes its stores and blocks own disjoint rows, so dcheb
// may alias dc.
template <int DM>
__global__ void __launch_bounds__(256)
k_coeff_from_cheb(const float* dcheb, float* dc, int64_t rows, int D, DcOut om, int vec,
                  BasisXform xf) {
  __shared__ __attribute__((aligned(16))) float tile[256 * DM];
  const int tid = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * 256;
  const int nr = (int)min<int64_t>(256, rows - r0);
  const int n = nr * D;
  const bool v4 = vec && (n % 4) == 0;
  const float* src = dcheb + r0 * D;
  float* dst = dc + r0 * D;
  if (v4) {
    // every load of the thread in flight before the first LDS store
    constexpr int U = (256 * DM / 4 + 255) / 256;
    f32x4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = tid + u * 256;
      v[u] = k < n / 4 ? __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(src) + k)
                       : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = tid + u * 256;
      if (k < n / 4) reinterpret_cast<f32x4_t*>(tile)[k] = v[u];
    }
  } else {
    for (int k = tid; k < n; k += 256) tile[k] = src[k];
  }
  __syncthreads();
  if (tid < nr) {
    float g[DM];
#pragma unroll
    for (int k = 0; k < DM; ++k) g[k] = k < D ? tile[tid * D + k] : 0.0f;
#pragma unroll
    for (int m = 0; m < DM; ++m) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k <= m; ++k) acc = fmaf(g[k], xf.m[m * kMaxD + k], acc);
      if (m < D) tile[tid * D + m] = acc;
    }
  }
  __syncthreads();
  if (v4) {
    for (int k = tid; k < n / 4; k += 256)
      dc_write4(reinterpret_cast<f32x4_t*>(dst) + k, reinterpret_cast<const f32x4_t*>(tile)[k], om);
  } else {
    for (int k = tid; k < n; k += 256) dc_write(dst + k, tile[k], om);
  }
}

// The recurrence coefficients a_n, b_n, c_n (n <= deg) of a family into LDS,
// rounded to fp32 once per block; ends with the block's barrier.
__device__ __forceinline__ void stage_family(float* ra, float* rb, float* rc, int deg, int family,
                                             double alpha, double beta) {
  for (int k = threadIdx.x; k <= deg; k += blockDim.x) {
    double a, b, c;
    recur_coef(family, k, alpha, beta, &a, &b, &c);
    ra[k] = (float)a;
    rb[k] = (float)b;
    rc[k] = (float)c;
  }
  __syncthreads();
}

// out[q, n] = P_n(t[q]) by the family's recurrence, n = 0..deg.
__global__ void __launch_bounds__(256)
k_basis_family(const float* __restrict__ t, int64_t n, int deg, int family, double alpha,
               double beta, float* __restrict__ out) {
  __shared__ float ra[kValuMaxDegree + 1], rb[kValuMaxDegree + 1], rc[kValuMaxDegree + 1];
  stage_family(ra, rb, rc, deg, family, alpha, beta);
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x) {
    const float tv = t[q];
    float* o = out + q * (deg + 1);
    o[0] = 1.0f;
    if (deg < 1) continue;
    float p0 = 1.0f, p1 = fmaf(ra[1], tv, rb[1]);
    o[1] = p1;
    for (int d = 2; d <= deg; ++d) {
      const float pn = fmaf(fmaf(ra[d], tv, rb[d]), p1, -rc[d] * p0);
      o[d] = pn;
      p0 = p1;
      p1 = pn;
    }
  }
}

// dt[q] = sum_n g[q, n] P_n'(t[q]), with the differentiated recurrence
// P_n' = a_n P_{n-1} + (a_n t + b_n) P_{n-1}' - c_n P_{n-2}'.
__global__ void __launch_bounds__(256)
k_basis_family_bwd(const float* __restrict__ t, const float* __restrict__ g, int64_t n, int deg,
                   int family, double alpha, double beta, float* __restrict__ dt) {
  __shared__ float ra[kValuMaxDegree + 1], rb[kValuMaxDegree + 1], rc[kValuMaxDegree + 1];
  stage_family(ra, rb, rc, deg, family, alpha, beta);
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x) {
    const float tv = t[q];
    const float* gq = g + q * (deg + 1);
    float s = 0.0f;
    if (deg >= 1) {
      float p0 = 1.0f, p1 = fmaf(ra[1], tv, rb[1]);  // P_{n-2}, P_{n-1}
      float d0 = 0.0f, d1 = ra[1];                    // their derivatives
      s = gq[1] * d1;
      for (int d = 2; d <= deg; ++d) {
        const float lin = fmaf(ra[d], tv, rb[d]);
        const float pn = fmaf(lin, p1, -rc[d] * p0);
        const float dn = fmaf(ra[d], p1, fmaf(lin, d1, -rc[d] * d0));
        s = fmaf(gq[d], dn, s);
        p0 = p1; p1 = pn;
        d0 = d1; d1 = dn;
      }
    }
    dt[q] = s;
  }
}

static unsigned grid_of(int64_t work) {
  int64_t g = (work + 255) / 256;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (unsigned)g;
}

void launch_coeff_from_cheb(const float* dcheb, float* dc, const Plan& p, const DcOut& om,
                            const BasisXform& xf, hipStream_t s) {
  const int64_t rows = (int64_t)p.I * p.O;
  const dim3 g((unsigned)((rows + 255) / 256));
  const int vec = is_al16(dcheb) && is_al16(dc);
  switch (p.P) {
    case 2: hipLaunchKernelGGL((k_coeff_from_cheb<3>), g, dim3(256), 0, s, dcheb, dc, rows, p.D, om, vec, xf); break;
    case 4: hipLaunchKernelGGL((k_coeff_from_cheb<5>), g, dim3(256), 0, s, dcheb, dc, rows, p.D, om, vec, xf); break;
    case 8: hipLaunchKernelGGL((k_coeff_from_cheb<9>), g, dim3(256), 0, s, dcheb, dc, rows, p.D, om, vec, xf); break;
    default: hipLaunchKernelGGL((k_coeff_from_cheb<17>), g, dim3(256), 0, s, dcheb, dc, rows, p.D, om, vec, xf); break;
  }
}

void launch_coeff_xform(const float* in, float* out, int64_t rows, int din, int dout,
                        int transposed_o, const BasisXform& r, hipStream_t s) {
  const dim3 g((unsigned)((rows + 255) / 256));
  hipLaunchKernelGGL(k_coeff_xform, g, dim3(256), 0, s, in, out, rows, din, dout, transposed_o, r);
}

// ---- the derivative operator row by row (Chebyshev series of any degree) ---
// For series too long for the operator matrix in the kernel arguments, each
// (i, o) row is transformed on the device, in place in LDS, one derivative
// step at a time (the steps of chebyshev_dx in fp32): the Chebyshev
// derivative recurrence b_{k-1} = b_{k+1} + 2 k a_k (b_0 halved), then the
// product with 1 - t^2, a stencil since t^2 T_k = T_k / 2 + (T_{k+2} +
// T_{|k-2|}) / 4:  r_j = q_j / 2 - (q_{j-2} + q_{j+2}) / 4, less q_1 / 4 at
// j = 1 and q_0 / 4 at j = 2.  The adjoint applies the transposed steps in
// reverse order (the coefficient gradient).
constexpr int kDerivRows = 32;  // rows per block at most, one lane each
constexpr size_t kDerivLds = 48 * 1024;  // a block's LDS at most (high degrees take fewer rows)

// degree deg (r[0..deg]) -> degree deg + 1 (r[0..deg + 1]); r[deg + 1] is 0 on entry
__device__ void cheb_dx_inplace(float* r, int deg) {
  float bnext = 0.0f, bcur = 0.0f, ak = r[deg];  // b_{k+1}, b_k, a_k
  for (int k = deg; k >= 1; --k) {
    const float akm1 = r[k - 1];
    const float bkm1 = fmaf(2.0f * (float)k, ak, bnext);
    r[k - 1] = bkm1;
    bnext = bcur;
    bcur = bkm1;
    ak = akm1;
  }
  r[deg] = 0.0f;
  if (deg >= 1) r[0] *= 0.5f;
  const float q0 = r[0];  // q = r[0 .. deg - 1]
  float qm2 = 0.0f, qm1 = 0.0f;
  for (int j = 0; j <= deg + 1; ++j) {
    const float qj = j <= deg - 1 ? r[j] : 0.0f;
    const float qj2 = j + 2 <= deg - 1 ? r[j + 2] : 0.0f;
    float v = 0.5f * qj - 0.25f * (qm2 + qj2);
    if (j == 1) v -= 0.25f * qj;
    if (j == 2) v -= 0.25f * (deg >= 1 ? q0 : 0.0f);
    r[j] = v;
    qm2 = qm1;
    qm1 = qj;
  }
}

// the transpose of cheb_dx_inplace: r[0..deg + 1] -> r[0..deg] (r[deg + 1] zeroed)
__device__ void cheb_dx_adjoint_inplace(float* r, int deg) {
  float rm2 = 0.0f, rm1 = 0.0f;
  for (int k = 0; k <= deg + 1; ++k) {
    const float rk = r[k];
    const float rk2 = k + 2 <= deg + 1 ? r[k + 2] : 0.0f;
    float v = 0.5f * rk - 0.25f * (rk2 + rm2);
    if (k == 1) v -= 0.25f * rk;
    if (k == 0) v -= 0.25f * rk2;
    r[k] = k < deg ? v : 0.0f;
    rm2 = rm1;
    rm1 = rk;
  }
  float se = 0.0f, so = 0.0f;  // weighted sums of the b-bar of even / odd index below k
  for (int k = 0; k <= deg; ++k) {
    const float qb = k < deg ? r[k] : 0.0f;
    r[k] = 2.0f * (float)k * ((k & 1) ? se : so);
    const float w = k == 0 ? 0.5f : 1.0f;
    if (k & 1) so = fmaf(w, qb, so);
    else se = fmaf(w, qb, se);
  }
}

// in [rows][din] -> out: [rows][dout], or [o][dout][i] for rows q = i * tO + o
// when tO > 0 (the Jacobian's layout).  ADJ: the transposed operator.
template <bool ADJ>
__global__ void __launch_bounds__(64)
k_cheb_deriv_rows(const float* __restrict__ in, float* __restrict__ out, int64_t rows, int din,
                  int dout, int deg0, int order, int pitch, int tO, int rpb) {
  extern __shared__ float sm[];
  const int tid = threadIdx.x;
  const int64_t q0 = (int64_t)blockIdx.x * rpb;
  const int nr = (int)(rows - q0 < rpb ? rows - q0 : rpb);
  for (int idx = tid; idx < rpb * pitch; idx += 64) sm[idx] = 0.0f;
  __syncthreads();
  for (int idx = tid; idx < nr * din; idx += 64) {  // the block's rows are contiguous
    const int r = idx / din, k = idx - r * din;
    sm[r * pitch + k] = in[q0 * din + idx];
  }
  __syncthreads();
  if (tid < nr) {
    float* rr = sm + tid * pitch;
    if constexpr (!ADJ) {
      for (int st = 0; st < order; ++st) cheb_dx_inplace(rr, deg0 + st);
    } else {
      for (int st = order - 1; st >= 0; --st) cheb_dx_adjoint_inplace(rr, deg0 + st);
    }
  }
  __syncthreads();
  if (tO == 0) {
    for (int idx = tid; idx < nr * dout; idx += 64) {
      const int r = idx / dout, k = idx - r * dout;
      out[q0 * dout + idx] = sm[r * pitch + k];
    }
  } else {
    const int64_t I = rows / tO;
    for (int idx = tid; idx < nr * dout; idx += 64) {
      const int r = idx / dout, k = idx - r * dout;
      const int64_t q = q0 + r, i = q / tO, o = q - i * tO;
      out[((size_t)o * dout + k) * I + i] = sm[r * pitch + k];
    }
  }
}

void launch_cheb_deriv_rows(const float* in, float* out, int64_t rows, int degree, int order,
                            bool adjoint, int transposed_o, hipStream_t s) {
  const int D = degree + 1, DO = D + order;
  const int pitch = DO | 1;  // odd: the row lanes hit distinct banks
  int rpb = (int)(kDerivLds / ((size_t)pitch * sizeof(float)));
  if (rpb > kDerivRows) rpb = kDerivRows;
  if (rpb < 1) rpb = 1;
  const size_t lds = (size_t)rpb * pitch * sizeof(float);
  const dim3 g((unsigned)((rows + rpb - 1) / rpb));
  if (adjoint)
    hipLaunchKernelGGL(k_cheb_deriv_rows<true>, g, dim3(64), lds, s, in, out, rows, DO, D, degree,
                       order, pitch, transposed_o, rpb);
  else
    hipLaunchKernelGGL(k_cheb_deriv_rows<false>, g, dim3(64), lds, s, in, out, rows, D, DO, degree,
                       order, pitch, transposed_o, rpb);
}

// jac[b, o, i] for any number of terms: the recurrence runs along k for each o.
__global__ void __launch_bounds__(256)
k_jacobian_any(const float* __restrict__ x, const float* __restrict__ c1t, float* __restrict__ jac,
               int64_t B, int I, int O, int dout, int imap, float ima, float imb) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (i >= I) return;
  const float t = input_map(x[b * I + i], imap, ima, imb), t2 = t + t;
  for (int o = 0; o < O; ++o) {
    const float* c = c1t + (size_t)o * dout * I + i;
    float tp = t, tc = 1.0f, acc = 0.0f;  // T_{-1} = t, T_0
    for (int k = 0; k < dout; ++k) {
      acc = fmaf(c[(size_t)k * I], tc, acc);
      const float nx = fmaf(t2, tc, -tp);
      tp = tc;
      tc = nx;
    }
    jac[((size_t)b * O + o) * I + i] = acc;
  }
}

void launch_jacobian(const float* x, const float* c1t, float* jac, int64_t B, int I, int O,
                     int dout, int imap, float ima, float imb, hipStream_t s) {
  constexpr int64_t kMaxGridY = 65535;
  for (int64_t b0 = 0; b0 < B; b0 += kMaxGridY) {  // rows in chunks of the grid's y limit
    const int64_t nb = B - b0 < kMaxGridY ? B - b0 : kMaxGridY;
    const dim3 g((unsigned)((I + 255) / 256), (unsigned)nb);
    const float* xb = x + b0 * I;
    float* jb = jac + b0 * O * I;
    if (dout <= 5)
      hipLaunchKernelGGL((k_jacobian<5>), g, dim3(256), 0, s, xb, c1t, jb, nb, I, O, dout,
                         imap, ima, imb);
    else if (dout <= 9)
      hipLaunchKernelGGL((k_jacobian<9>), g, dim3(256), 0, s, xb, c1t, jb, nb, I, O, dout,
                         imap, ima, imb);
    else if (dout <= 17)
      hipLaunchKernelGGL((k_jacobian<17>), g, dim3(256), 0, s, xb, c1t, jb, nb, I, O, dout,
                         imap, ima, imb);
    else
      hipLaunchKernelGGL(k_jacobian_any, g, dim3(256), 0, s, xb, c1t, jb, nb, I, O, dout, imap,
                         ima, imb);
  }
}

void launch_basis_family(const float* t, int64_t n, int deg, int family, double alpha,
                         double beta, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_basis_family, dim3(grid_of(n)), dim3(256), 0, s, t, n, deg, family, alpha,
                     beta, out);
}

void launch_basis_family_bwd(const float* t, const float* g, int64_t n, int deg, int family,
                             double alpha, double beta, float* dt, hipStream_t s) {
  hipLaunchKernelGGL(k_basis_family_bwd, dim3(grid_of(n)), dim3(256), 0, s, t, g, n, deg, family,
                     alpha, beta, dt);
}

}  // namespace ckan
