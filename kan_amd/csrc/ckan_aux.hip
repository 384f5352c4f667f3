// Bandwidth-bound kernels around the three MFMA contractions: the tanh cache,
// coefficient packing, the dy re-layout, the dC finalisation, the optimizers
// and the materialised basis.  All are HBM-bound elementwise or re-layout
// passes; each moves its bytes once with coalesced accesses.
#include "ckan_kernels.hpp"

namespace ckan {

// t[b, i] = tanh(x[b, i]) for i < I, 0 for I <= i < I_sg.  Row pitch I_sg.
// Replaces torch.tanh (kan/basis/chebyshev.py:78).  tpr threads per row
// (a power of two dividing 256) take float4 columns; 256/tpr rows per block.
__global__ void __launch_bounds__(256)
k_tanh(const float* __restrict__ x, float* __restrict__ t, int64_t B, int I, int I_sg, int tpr,
       int xal, int imap, float ima, float imb) {
  const int rpb = 256 / tpr;
  const int64_t b = (int64_t)blockIdx.x * rpb + threadIdx.x / tpr;
  if (b >= B) return;
  const int n4 = I_sg / 4;
  const bool vec = xal && (I % 4) == 0;
  const float* xr = x + b * I;
  float* tr = t + b * I_sg;
  for (int c4 = threadIdx.x % tpr; c4 < n4; c4 += tpr) {
    const int i = c4 * 4;
    f32x4_t v;
    if (vec && i < I) {
      v = *reinterpret_cast<const f32x4_t*>(xr + i);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = (i + j < I) ? xr[i + j] : 0.0f;
    }
    f32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = (i + j < I) ? input_map(v[j], imap, ima, imb) : 0.0f;
    *reinterpret_cast<f32x4_t*>(tr + i) = r;
  }
}

// Same, when rows need no padding (I == I_sg, I % 4 == 0): x and t are flat
// arrays of n4 float4.  Each thread issues its kTanhU loads (block-strided, so
// each instruction is one contiguous 4 KiB run per block) before any tanh.
// Two per thread measured fastest (one to eight tried).
constexpr int kTanhU = 2;
__global__ void __launch_bounds__(256)
k_tanh_flat(const f32x4_t* __restrict__ x, f32x4_t* __restrict__ t, int64_t n4, int imap, float ima,
            float imb) {
  const int64_t base = (int64_t)blockIdx.x * (256 * kTanhU) + threadIdx.x;
  f32x4_t v[kTanhU];
  // x, C and dy are read once per launch: non-temporal loads keep them from
  // displacing reused data (pack + tanh 34 -> 28 us, dy re-layout 18 -> 16 us
  // at config 3)
#pragma unroll
  for (int u = 0; u < kTanhU; ++u) {
    const int64_t k = base + u * 256;
    v[u] = k < n4 ? __builtin_nontemporal_load(x + k) : f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int u = 0; u < kTanhU; ++u) {
    const int64_t k = base + u * 256;
    f32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = input_map(v[u][j], imap, ima, imb);
    if (k < n4) t[k] = r;
  }
}

template <typename CT> __device__ __forceinline__ float to_f32(CT v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) {
  return __uint_as_float(((unsigned)v) << 16);
}

// Packs C [I, O, D] into
//   Cf: forward B operand, [NBf][KB][64][8]   (columns o, reduction (i, d>=1))
//   Cb: dX B operand,      [NIB*P][KBx][64][8] (columns (input block, d), reduction o)
//   bias_part[ib][o] = sum_{i in block ib} C[i, o, 0]
// One block per (32 inputs, 32 outputs) tile, staged through LDS so the
// global read of C is one contiguous run of 32*D values per input.  The LDS
// row pitch 32*D+1 is odd, so the column-wise reads of the Cb re-layout hit
// 32 distinct banks.
// With XF, each (input, output) row of D coefficients is first replaced by
// its Chebyshev-basis equivalent c'[k] = sum_n c[n] m[n][k] (another
// polynomial family's coefficients re-expressed for these kernels).
template <bool XF> struct XfArg { BasisXform x; };
template <> struct XfArg<false> {};

// The optional tanh share of a pack launch (t = tanh(x) as flat float4
// arrays, rows unpadded): block k takes float4 [k * per, (k + 1) * per).
struct TanhJob {
  const f32x4_t* x;
  f32x4_t* t;
  int64_t n4, per;
  int imap;
  float ima, imb;
};
constexpr int kPackTanhU = 8;  // tanh float4 per thread in flight at once

// One pack block: input block ib, output block ob; `lin` numbers the block
// for its tanh share.
template <int P, bool BF, typename CT, bool XF>
__device__ __forceinline__ void pack_tile(const CT* __restrict__ C, typename Elem<BF>::type* __restrict__ Cf,
                                          typename Elem<BF>::type* __restrict__ Cb,
                                          float* __restrict__ bias_part, const Plan& p, int cal,
                                          const XfArg<XF>& xf, const TanhJob& tj, int ib, int ob,
                                          int64_t lin) {
  using G = FwdGroup<P>;
  constexpr int RPMAX = 32 * (P + 1) + 1;
  __shared__ float tile[32 * RPMAX];
  __shared__ float bsum[8][32];
  const int tid = threadIdx.x;
  // tanh share: the first chunk's loads go out with the tile's, so both streams
  // are in flight together; the tanh itself runs after the re-layout
  const int64_t tj0 = tj.per * lin;
  const int64_t tj1 = tj.x ? (tj0 + tj.per < tj.n4 ? tj0 + tj.per : tj.n4) : 0;
  f32x4_t tx[kPackTanhU];
#pragma unroll
  for (int u = 0; u < kPackTanhU; ++u) {
    const int64_t k = tj0 + tid + u * 256;
    tx[u] = k < tj1 ? __builtin_nontemporal_load(tj.x + k) : f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // tanh of the chunk at c0 held in tx, stored to t
  auto tanh_chunk = [&](int64_t c0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kPackTanhU; ++u) {
      const int64_t k = c0 + tid + u * 256;
      f32x4_t r;
#pragma unroll
      for (int j = 0; j < 4; ++j) r[j] = input_map(tx[u][j], tj.imap, tj.ima, tj.imb);
      if (k < tj1) tj.t[k] = r;  // read again by the GEMMs: cached store
    }
  };
  bool first_done = false;  // the first chunk is done while the tile loads (float4 path)
  const int i0 = ib * 32, o0 = ob * 32;
  const int D = p.D;
  const int RP = 32 * D + 1;
  const int ocount = min(32, p.O - o0);  // may be <= 0 for the Cb zero-fill blocks
  const int nrow = ocount > 0 ? ocount * D : 0;
  // Each input's run of 32*D values is contiguous in C.  When the run is
  // 16-byte aligned, every thread issues its float4 loads before any use.
  const bool vec = sizeof(CT) == 4 && cal && ((size_t)p.O * D) % 4 == 0 && ocount == 32;
  if (vec) {
    constexpr int MAXV = (32 * 32 * (P + 1) / 4 + 255) / 256;  // float4 per thread
    const int nv = 32 * 8 * D;                                   // float4 in the tile
    f32x4_t buf[MAXV];
#pragma unroll
    for (int q = 0; q < MAXV; ++q) {
      const int v = tid + q * 256;
      const int il = v / (8 * D), k4 = v - il * (8 * D);
      const int i = i0 + il;
      buf[q] = (v < nv && i < p.I)
          ? __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(reinterpret_cast<const float*>(C) + ((size_t)i * p.O + o0) * D + k4 * 4))
          : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    // the tanh share's first chunk (its loads went out before the tile's)
    // while the tile's loads are in flight
    tanh_chunk(tj0);
    first_done = true;
#pragma unroll
    for (int q = 0; q < MAXV; ++q) {
      const int v = tid + q * 256;
      if (v < nv) {
        const int il = v / (8 * D), k4 = v - il * (8 * D);
        float* dst = tile + il * RP + k4 * 4;
        dst[0] = buf[q][0]; dst[1] = buf[q][1]; dst[2] = buf[q][2]; dst[3] = buf[q][3];
      }
    }
  } else {
    // element k of the flattened [32 inputs][32 * D] tile; 16 loads in flight
    // per thread before any is stored (one at a time made small packs
    // latency-bound: 13.7 us for a 64 x 10 x 5 layer)
    const int nt = 32 * 32 * D;
    for (int k0 = 0; k0 < nt; k0 += 256 * 16) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int k = k0 + u * 256 + tid;
        const int il = k / (32 * D), e = k - il * (32 * D);
        const int i = i0 + il;
        v[u] = (k < nt && i < p.I && e < nrow) ? to_f32<CT>(C[((size_t)i * p.O + o0) * D + e]) : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int k = k0 + u * 256 + tid;
        const int il = k / (32 * D), e = k - il * (32 * D);
        if (k < nt) tile[il * RP + e] = v[u];
      }
    }
  }
  __syncthreads();

  if constexpr (XF) {
    for (int row = tid; row < 32 * 32; row += 256) {
      float* r = tile + (row >> 5) * RP + (row & 31) * D;
      float v[P + 1];
#pragma unroll
      for (int n = 0; n <= P; ++n) v[n] = n < D ? r[n] : 0.0f;
#pragma unroll
      for (int k = 0; k <= P; ++k) {
        float acc = 0.0f;
#pragma unroll
        for (int n = k; n <= P; ++n) acc = fmaf(v[n], xf.x.m[n * kMaxD + k], acc);  // m[n][k] = 0 for k > n
        if (k < D) r[k] = acc;
      }
    }
    __syncthreads();
  }

  {  // bias partial: 8 groups of 4 inputs, then a fixed-order sum
    const int ol = tid & 31, grp = tid >> 5;
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) s += tile[(grp * 4 + q) * RP + ol * D];
    bsum[grp][ol] = s;
  }
  __syncthreads();
  if (tid < 32 && o0 + tid < p.O32) {
    float s = 0.0f;
#pragma unroll
    for (int grp = 0; grp < 8; ++grp) s += bsum[grp][tid];
    bias_part[(size_t)ib * p.O32 + o0 + tid] = s;
  }

  if (ob < p.NBf) {
    const int kb_base = ib * 2 * P;  // 32 inputs * P values / 16 per k-block
    for (int item = tid; item < 2 * P * 64; item += 256) {
      const int kbl = item >> 6, lane = item & 63;
      const int kb = kb_base + kbl;
      if (kb >= p.KB) continue;
      const int ol = lane & 31, g = lane >> 5;
      const int r = kb / G::SGK, q = kb - r * G::SGK;
      const int s = q / G::KBG, h = q - s * G::KBG;
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int vv = 8 * h + j;
        const int u = vv / P, d = vv % P + 1;
        const int i = r * G::SGI + g * 2 * G::IPG + s * (G::IPG / 2) + u;
        v[j] = (d <= p.deg) ? tile[(i - i0) * RP + ol * D + d] : 0.0f;
      }
      store_frag<BF>(Cf + cf_elem<BF>(p.KB, ob, kb, lane) - (size_t)lane * 8, lane, v);
    }
  }

  for (int item = tid; item < P * 2 * 64; item += 256) {
    const int e = item >> 7, rem = item & 127;
    const int kbl = rem >> 6, lane = rem & 63;
    const int il = lane & 31, g = lane >> 5;
    const int kbx = ob * 2 + kbl;
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int ol = 16 * kbl + 8 * g + j;
      // scaled by the degree d = e + 1, the factor of dT_d/dt = d U_{d-1}(t)
      v[j] = (e + 1 <= p.deg) ? tile[il * RP + ol * D + e + 1] * (float)(e + 1) : 0.0f;
    }
    store_frag<BF>(Cb + ((size_t)(ib * P + e) * p.KBx + kbx) * kFragElems, lane, v);
  }

  for (int64_t c0 = first_done ? tj0 + 256 * kPackTanhU : tj0; c0 < tj1; c0 += 256 * kPackTanhU) {
    if (c0 > tj0) {
#pragma unroll
      for (int u = 0; u < kPackTanhU; ++u) {
        const int64_t k = c0 + tid + u * 256;
        tx[u] = k < tj1 ? __builtin_nontemporal_load(tj.x + k) : f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    }
    tanh_chunk(c0);
  }
}

template <int P, bool BF, typename CT, bool XF>
__global__ void __launch_bounds__(256)
k_pack(const CT* __restrict__ C, typename Elem<BF>::type* __restrict__ Cf,
       typename Elem<BF>::type* __restrict__ Cb, float* __restrict__ bias_part, Plan p, int cal,
       XfArg<XF> xf, TanhJob tj) {
  pack_tile<P, BF, CT, XF>(C, Cf, Cb, bias_part, p, cal, xf, tj, blockIdx.x, blockIdx.y,
                           blockIdx.x + (int64_t)gridDim.x * blockIdx.y);
}

// Two layers' packs in one launch (fp32 coefficients, the Chebyshev basis):
// blocks [0, a.nblocks) pack layer a, the rest layer b.  For stacks of small
// layers, where each pack is a latency-bound launch of a few blocks.
template <bool BF> struct PackJob {
  const float* C;
  typename Elem<BF>::type* Cf;
  typename Elem<BF>::type* Cb;
  float* bias;
  Plan p;
  int cal, nx, nblocks;
  TanhJob tj;
};
template <int P, bool BF>
__global__ void __launch_bounds__(256)
k_pack2(PackJob<BF> a, PackJob<BF> b) {
  const int bid = blockIdx.x;
  if (bid < a.nblocks)
    pack_tile<P, BF, float, false>(a.C, a.Cf, a.Cb, a.bias, a.p, a.cal, XfArg<false>{}, a.tj,
                                   bid % a.nx, bid / a.nx, bid);
  else
    pack_tile<P, BF, float, false>(b.C, b.Cf, b.Cb, b.bias, b.p, b.cal, XfArg<false>{}, b.tj,
                                   (bid - a.nblocks) % b.nx, (bid - a.nblocks) / b.nx, bid - a.nblocks);
}

// out[o] = sum_k part[k][o] for k < nparts (row pitch `pitch`): 4 interleaved
// partial sums per column keep independent loads in flight; they are added in
// a fixed order, so the result is deterministic.  Used for the forward bias
// (sum_i C[i, o, 0] over input blocks) and the dC column sums of dy.
__global__ void __launch_bounds__(256)
k_col_reduce(const float* __restrict__ part, int nparts, int pitch, int n, float* __restrict__ out) {
  __shared__ float q4[4][64];
  const int ol = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int o = blockIdx.x * 64 + ol;
  float s = 0.0f;
  if (o < n) {
#pragma unroll 8
    for (int k = q; k < nparts; k += 4) s += part[(size_t)k * pitch + o];
  }
  q4[q][ol] = s;
  __syncthreads();
  if (q == 0 && o < n) out[o] = ((q4[0][ol] + q4[1][ol]) + q4[2][ol]) + q4[3][ol];
}

// Re-lays dy [B, O] (fp32) into
//   dYx: dX A operand  [B32/32][KBx][64][8]  (rows b, reduction o)
//   dYc: dC B operand  [NBf][KBc][64][8]     (columns o, reduction b)
// and writes colsum_part[bb][o] = sum of dy over rows [64 bb, 64 bb + 64).
// A wave's unit is (32 columns, 64 rows): it reads that tile of dy once, each
// load instruction covering 8 whole 128-byte row segments, writes it to a
// private LDS tile and reads it back in both fragment orders: 8 consecutive
// columns of a row per lane (dYx) and 8 consecutive rows of a column (dYc).
// Waves stride over the units with the next unit's loads in flight while
// they re-lay and store the current one, so reads and writes overlap instead
// of every wave loading first and storing after.
#ifndef CKAN_PREP_BLOCKS
#define CKAN_PREP_BLOCKS 512
#endif
constexpr int kPrepBlocks = CKAN_PREP_BLOCKS;  // grid cap: 2 blocks (8 waves) per CU
template <bool BF>
__global__ void __launch_bounds__(256)
k_prep_dy(const float* __restrict__ dy, typename Elem<BF>::type* __restrict__ dYx,
           typename Elem<BF>::type* __restrict__ dYc, float* __restrict__ colsum_part,
           Plan p, int need_dx, int need_dc, int nob, int nbb, int64_t dx_rows, int dyal) {
  constexpr int TP = 36;  // row pitch (floats): 16-byte aligned rows
  constexpr int NL = kPrepRows / 8;
  __shared__ __attribute__((aligned(16))) float tile[4][kPrepRows * TP];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nw = nob * nbb, stride = (int)gridDim.x * 4;
  int w = blockIdx.x * 4 + wv;
  if (w >= nw) return;
  const int g = lane >> 5, c = lane & 31;
  const int rs = lane >> 3, q = lane & 7;
  float* t = tile[wv];

  auto load = [&](int wu, f32x4_t (&v)[NL]) __attribute__((always_inline)) {
    const int ob = wu % nob, bb = wu / nob;
    const int64_t r0 = (int64_t)bb * kPrepRows;
    const int o = ob * 32 + 4 * q;
    const bool vec = dyal && (p.O & 3) == 0 && o + 4 <= p.O;
#pragma unroll
    for (int m = 0; m < NL; ++m) {
      const int64_t b = r0 + m * 8 + rs;
      if (b < p.B && vec) {
        v[m] = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(dy + b * p.O + o));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[m][j] = (b < p.B && o + j < p.O) ? dy[b * p.O + o + j] : 0.0f;
      }
    }
  };
  auto process = [&](int wu, const f32x4_t (&v)[NL]) __attribute__((always_inline)) {
    const int ob = wu % nob, bb = wu / nob;
    const int64_t r0 = (int64_t)bb * kPrepRows;
    // the tile is private to this wave, whose LDS accesses are performed in
    // issue order; the compiler barriers keep the previous unit's reads
    // before these writes and these writes before the reads below
    asm volatile("" ::: "memory");
#pragma unroll
    for (int m = 0; m < NL; ++m) *reinterpret_cast<f32x4_t*>(t + (m * 8 + rs) * TP + 4 * q) = v[m];
    asm volatile("" ::: "memory");
    if (need_dx) {
#pragma unroll
      for (int mbl = 0; mbl < kPrepRows / 32; ++mbl) {
        const int64_t b0 = r0 + mbl * 32;
        if (b0 < dx_rows) {
#pragma unroll
          for (int kbl = 0; kbl < 2; ++kbl) {
            const float* src = t + (mbl * 32 + c) * TP + 16 * kbl + 8 * g;
            const f32x4_t a = *reinterpret_cast<const f32x4_t*>(src);
            const f32x4_t e = *reinterpret_cast<const f32x4_t*>(src + 4);
            const float vv[8] = {a[0], a[1], a[2], a[3], e[0], e[1], e[2], e[3]};
            store_frag<BF>(dYx + ((size_t)(b0 / 32) * p.KBx + ob * 2 + kbl) * kFragElems, lane, vv);
          }
        }
      }
    }
    if (need_dc && ob < p.NBf) {
      float u[kPrepRows / 16][8];
#pragma unroll
      for (int kbl = 0; kbl < kPrepRows / 16; ++kbl)
#pragma unroll
        for (int j = 0; j < 8; ++j) u[kbl][j] = t[(kbl * 16 + 8 * g + j) * TP + c];
      float cs = 0.0f;
#pragma unroll
      for (int kbl = 0; kbl < kPrepRows / 16; ++kbl) {
        const int64_t b0 = r0 + kbl * 16;
#pragma unroll
        for (int j = 0; j < 8; ++j) cs += u[kbl][j];
        if (b0 < p.Bc) store_frag<BF>(dYc + ((size_t)ob * p.KBc + b0 / 16) * kFragElems, lane, u[kbl]);
      }
      // rows of lane halves interleave in blocks of 8; add the halves in a fixed order
      const float other = __shfl_xor(cs, 32);
      if (g == 0 && bb < p.NBB) colsum_part[(size_t)bb * p.O32 + ob * 32 + c] = cs + other;
    }
  };

  f32x4_t va[NL], vb[NL];
  load(w, va);
  for (;;) {  // two units per pass, alternating register sets
    int wn = w + stride;
    if (wn < nw) load(wn, vb);
    process(w, va);
    if (wn >= nw) break;
    w = wn;
    wn = w + stride;
    if (wn < nw) load(wn, va);
    process(w, vb);
    if (wn >= nw) break;
    w = wn;
  }
}

// dC[i, o, d] (stored, added or applied as an SGD step, by om) for d = 0: sum_b dy[b, o] (from the colsum partials);
// for d >= 1: sum over the S split partials part[s][d-1][i][o].
// One block per (16 inputs, 64 outputs); the tile is transposed through LDS
// so the write of dC is one contiguous run of 64*D values per input.
template <int P>
__global__ void __launch_bounds__(256)
k_dc_finalize(const float* __restrict__ part, int S, const float* __restrict__ colsum,
              float* __restrict__ dC, DcOut om, Plan p) {
  __shared__ float tile[16 * 64 * (P + 1)];
  __shared__ float csq[1][64];
  const int tid = threadIdx.x;
  const int i0 = blockIdx.x * 16, o0 = blockIdx.y * 64;
  const int D = p.D;
  const int ol = tid & 63, q = tid >> 6;
  const int o = o0 + ol;
  if (tid < 64) csq[0][ol] = (o < p.O) ? colsum[o] : 0.0f;
  const size_t sstride = (size_t)p.P * p.I32 * p.O32;
#pragma unroll 4
  for (int il = 0; il < 16; ++il) {
    const int i = i0 + il;
    const bool ok = i < p.I && o < p.O;
#pragma unroll
    for (int e = q; e < P; e += 4) {
      float v = 0.0f;
      if (ok && e < p.deg) {
        const float* src = part + ((size_t)e * p.I32 + i) * p.O32 + o;
        for (int s0 = 0; s0 < S; s0 += 4) {  // 4 loads in flight, added in split order
          float w[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = (s0 + j < S) ? src[(size_t)(s0 + j) * sstride] : 0.0f;
#pragma unroll
          for (int j = 0; j < 4; ++j) v += w[j];
        }
      }
      if (e < p.deg) tile[(il * 64 + ol) * D + e + 1] = v;
    }
  }
  __syncthreads();
  for (int idx = tid; idx < 16 * 64; idx += 256) tile[idx * D] = csq[0][idx & 63];
  __syncthreads();
  const int ocount = (p.O - o0) < 64 ? (p.O - o0) : 64;
  const int nrow = ocount * D;
  for (int il = 0; il < 16; ++il) {
    const int i = i0 + il;
    if (i >= p.I) break;
    float* dst = dC + ((size_t)i * p.O + o0) * D;
    const float* src = tile + il * 64 * D;
    for (int idx = tid; idx < nrow; idx += 256) {
      const float v = src[idx];
      dc_write(dst + idx, v, om);
    }
  }
}

__global__ void __launch_bounds__(256)
k_sgd(float* __restrict__ p, const float* __restrict__ g, int64_t n, float lr, float wd) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x) {
    p[q] = sgd_update(p[q], g[q], lr, wd);
  }
}

// Adam in torch's single-tensor order; scalars are prepared on the host in
// double precision and rounded to fp32 as torch does for fp32 tensors.
__global__ void __launch_bounds__(256)
k_adam(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
       float* __restrict__ v, int64_t n, float w1, float beta2, float one_m_beta2,
       float bc2_sqrt, float eps, float neg_step_size, float wd) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x) {
    float gv = g[q];
    const float pv = p[q];
    if (wd != 0.0f) gv = gv + wd * pv;
    float mv = m[q];
    // lerp(m, g, w1) as torch computes it for |w1| < 0.5 and otherwise
    mv = (w1 < 0.5f) ? mv + w1 * (gv - mv) : gv - (gv - mv) * (1.0f - w1);
    float vv = v[q] * beta2;
    vv = vv + one_m_beta2 * gv * gv;
    const float denom = sqrtf(vv) / bc2_sqrt + eps;
    m[q] = mv;
    v[q] = vv;
    p[q] = pv + neg_step_size * (mv / denom);
  }
}

// out[q, d] = T_d(t[q]), d = 0..deg.
__global__ void __launch_bounds__(256)
k_basis(const float* __restrict__ t, int64_t n, int deg, float* __restrict__ out) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x) {
    const float tv = t[q];
    float* o = out + q * (deg + 1);
    o[0] = 1.0f;
    if (deg >= 1) o[1] = tv;
    float a = 1.0f, b = tv;
    const float t2 = tv + tv;
    for (int d = 2; d <= deg; ++d) {
      const float c = fmaf(t2, b, -a);
      o[d] = c;
      a = b;
      b = c;
    }
  }
}

// dt[q] = sum_d g[q, d] d U_{d-1}(t[q]).
__global__ void __launch_bounds__(256)
k_basis_bwd(const float* __restrict__ t, const float* __restrict__ g, int64_t n, int deg,
            float* __restrict__ dt) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x) {
    const float tv = t[q];
    const float t2 = tv + tv;
    const float* gq = g + q * (deg + 1);
    float up = 0.0f, u = 1.0f, s = 0.0f;  // U_{-1}, U_0
    for (int d = 1; d <= deg; ++d) {
      s = fmaf(gq[d] * (float)d, u, s);
      const float un = fmaf(t2, u, -up);
      up = u;
      u = un;
    }
    dt[q] = s;
  }
}

__global__ void __launch_bounds__(256) k_zero(u32x4_t* __restrict__ p, int64_t n16) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n16;
       q += (int64_t)gridDim.x * blockDim.x)
    p[q] = u32x4_t{0u, 0u, 0u, 0u};
}

__global__ void __launch_bounds__(256) k_zero_f32(float* __restrict__ p, int64_t n) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x)
    p[q] = 0.0f;
}

// ---------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------

static int grid_for(int64_t work, int per_block = 256) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

void launch_tanh(const float* x, float* t, const Plan& p, hipStream_t s) {
  if (p.I == p.I_sg && p.I % 4 == 0 && is_al16(x)) {
    const int64_t n4 = p.B * p.I / 4;
    hipLaunchKernelGGL(k_tanh_flat, dim3((unsigned)ceil_div(n4, 256 * kTanhU)), dim3(256), 0, s,
                       reinterpret_cast<const f32x4_t*>(x), reinterpret_cast<f32x4_t*>(t), n4, p.imap,
                       p.ima, p.imb);
    return;
  }
  int tpr = 1;
  while (tpr < 256 && tpr < p.I_sg / 4) tpr *= 2;
  const int64_t blocks = ceil_div(p.B, 256 / tpr);
  hipLaunchKernelGGL(k_tanh, dim3((unsigned)blocks), dim3(256), 0, s, x, t, p.B, p.I, p.I_sg, tpr,
                     (int)is_al16(x), p.imap, p.ima, p.imb);
}

template <int P, bool BF, bool XF>
static void launch_pack_t(const void* C, bool c_bf16, void* packed, const Plan& p, hipStream_t s,
                          const XfArg<XF>& xf, const TanhJob& tj) {
  typedef typename Elem<BF>::type E;
  E* Cf = reinterpret_cast<E*>(packed);
  E* Cb = Cf + packed_cf_elems(p);
  // with one input block its bias partial is the bias itself
  float* bias = reinterpret_cast<float*>(reinterpret_cast<char*>(packed) +
                                         (p.NIB == 1 ? packed_biasf_offset(p) : packed_bias_offset(p)));
  dim3 grid(p.NIB, p.O64 / 32);
  if (c_bf16)
    hipLaunchKernelGGL((k_pack<P, BF, uint16_t, XF>), grid, dim3(256), 0, s,
                       reinterpret_cast<const uint16_t*>(C), Cf, Cb, bias, p, 0, xf, tj);
  else
    hipLaunchKernelGGL((k_pack<P, BF, float, XF>), grid, dim3(256), 0, s,
                       reinterpret_cast<const float*>(C), Cf, Cb, bias, p, (int)is_al16(C), xf, tj);
}

template <bool XF>
static void launch_pack_x(const void* C, bool c_bf16, void* packed, const Plan& p, hipStream_t s,
                          const XfArg<XF>& xf, const TanhJob& tj) {
  const bool bf = p.esz == 2;
#define CKAN_PK(PP, BB) launch_pack_t<PP, BB>(C, c_bf16, packed, p, s, xf, tj)
  switch (p.P) {
    case 2: bf ? CKAN_PK(2, true) : CKAN_PK(2, false); break;
    case 4: bf ? CKAN_PK(4, true) : CKAN_PK(4, false); break;
    case 8: bf ? CKAN_PK(8, true) : CKAN_PK(8, false); break;
    default: bf ? CKAN_PK(16, true) : CKAN_PK(16, false); break;
  }
#undef CKAN_PK
}

bool pack_tanh_fusable(const Plan& p, const float* x) {
  // and the pack has blocks enough for one pass of tanh each: a pack with few
  // blocks (narrow outputs) would run the tanh stream serially (config 4's
  // 512 -> 64 layer: 639 us fused against ~45 us in two launches)
  const int64_t blocks = (int64_t)p.NIB * (p.O64 / 32);
  return x && p.I == p.I_sg && p.I % 4 == 0 && is_al16(x) &&
         blocks * 256 * kPackTanhU >= p.B * (int64_t)p.I / 4;
}

void launch_pack(const void* C, bool c_bf16, void* packed, const Plan& p, hipStream_t s,
                 const BasisXform* xf, bool reduce_bias, const float* x, float* t) {
  char* base = reinterpret_cast<char*>(packed);
  TanhJob tj{nullptr, nullptr, 0, 0, p.imap, p.ima, p.imb};
  if (x && t) {  // pack_tanh_fusable(p, x) holds: the caller checked
    tj.x = reinterpret_cast<const f32x4_t*>(x);
    tj.t = reinterpret_cast<f32x4_t*>(t);
    tj.n4 = p.B * p.I / 4;
    const int64_t blocks = (int64_t)p.NIB * (p.O64 / 32);
    tj.per = round_up(ceil_div(tj.n4, blocks), 256);
  }
  if (xf) {
    XfArg<true> a;
    a.x = *xf;
    launch_pack_x<true>(C, c_bf16, packed, p, s, a, tj);
  } else {
    launch_pack_x<false>(C, c_bf16, packed, p, s, XfArg<false>{}, tj);
  }
  if (p.NIB > 1 && reduce_bias)  // bias = sum of the per-input-block partials, in block order
    hipLaunchKernelGGL(k_col_reduce, dim3((unsigned)ceil_div(p.O32, 64)), dim3(256), 0, s,
                       reinterpret_cast<const float*>(base + packed_bias_offset(p)), p.NIB,
                       p.O32, p.O32, reinterpret_cast<float*>(base + packed_biasf_offset(p)));
}

template <int P, bool BF>
static void launch_pack2_t(const float* Ca, void* pa, const Plan& qa, const TanhJob& tja,
                           const float* Cb_, void* pb, const Plan& qb, hipStream_t s) {
  typedef typename Elem<BF>::type E;
  auto job = [](const float* C, void* packed, const Plan& q, const TanhJob& tj) {
    PackJob<BF> j;
    j.C = C;
    j.Cf = reinterpret_cast<E*>(packed);
    j.Cb = j.Cf + packed_cf_elems(q);
    j.bias = reinterpret_cast<float*>(reinterpret_cast<char*>(packed) +
                                      (q.NIB == 1 ? packed_biasf_offset(q) : packed_bias_offset(q)));
    j.p = q;
    j.cal = (int)is_al16(C);
    j.nx = q.NIB;
    j.nblocks = q.NIB * (q.O64 / 32);
    j.tj = tj;
    return j;
  };
  const PackJob<BF> a = job(Ca, pa, qa, tja);
  const PackJob<BF> b = job(Cb_, pb, qb, TanhJob{nullptr, nullptr, 0, 0, qb.imap, qb.ima, qb.imb});
  hipLaunchKernelGGL((k_pack2<P, BF>), dim3((unsigned)(a.nblocks + b.nblocks)), dim3(256), 0, s, a, b);
}

bool pack_pair_ok(const Plan& a, const Plan& b) {
  return a.P == b.P && a.esz == b.esz && (int64_t)a.NIB * (a.O64 / 32) + (int64_t)b.NIB * (b.O64 / 32) < (1 << 30);
}

void launch_pack_pair(const float* Ca, void* pa, const Plan& qa, bool reduce_a, const float* xa,
                      float* ta, const float* Cb_, void* pb, const Plan& qb, bool reduce_b,
                      hipStream_t s) {
  TanhJob tj{nullptr, nullptr, 0, 0, qa.imap, qa.ima, qa.imb};
  if (xa && ta) {  // pack_tanh_fusable(qa, xa) holds: the caller checked
    tj.x = reinterpret_cast<const f32x4_t*>(xa);
    tj.t = reinterpret_cast<f32x4_t*>(ta);
    tj.n4 = qa.B * qa.I / 4;
    tj.per = round_up(ceil_div(tj.n4, (int64_t)qa.NIB * (qa.O64 / 32)), 256);
  }
  const bool bf = qa.esz == 2;
#define CKAN_PK2(PP, BB) launch_pack2_t<PP, BB>(Ca, pa, qa, tj, Cb_, pb, qb, s)
  switch (qa.P) {
    case 2: bf ? CKAN_PK2(2, true) : CKAN_PK2(2, false); break;
    case 4: bf ? CKAN_PK2(4, true) : CKAN_PK2(4, false); break;
    case 8: bf ? CKAN_PK2(8, true) : CKAN_PK2(8, false); break;
    default: bf ? CKAN_PK2(16, true) : CKAN_PK2(16, false); break;
  }
#undef CKAN_PK2
  if (qa.NIB > 1 && reduce_a) launch_bias_reduce(pa, qa, s);
  if (qb.NIB > 1 && reduce_b) launch_bias_reduce(pb, qb, s);
}

void launch_bias_reduce(void* packed, const Plan& p, hipStream_t s) {
  char* base = reinterpret_cast<char*>(packed);
  if (p.NIB > 1)
    hipLaunchKernelGGL(k_col_reduce, dim3((unsigned)ceil_div(p.O32, 64)), dim3(256), 0, s,
                       reinterpret_cast<const float*>(base + packed_bias_offset(p)), p.NIB,
                       p.O32, p.O32, reinterpret_cast<float*>(base + packed_biasf_offset(p)));
}

// Small dC: dC[i, o, d] = sum_b T_d(t[b, i]) dy[b, o] in fp32 for problems
// whose MFMA pipeline would be all prologue (config 2: B = 256).  A block
// takes 8 inputs x 8 outputs; its 256 threads are 64 (input, output) pairs x
// 4 row quarters.  t [B][8] and dy [B][8] are staged in LDS, each thread
// accumulates its pair's D sums over its quarter of the rows (Chebyshev
// recurrence in registers), and the quarters are added in order through LDS.
constexpr int kDcSmallRows = 256;  // rows staged at once (all of the batch)

// One 256-thread group's sums for 8 inputs x 8 outputs (DMAX <= 9), from t
// staged as ts[r * TP + input] and dy as ys[r * 8 + output]: thread (lane,
// wave rq) takes input il2 = lane % 8, outputs 4 og .. 4 og + 3 (og = lane /
// 8 % 2) and rows r = rs (mod 16), rs = 4 rq + lane / 16, so the recurrence of
// a (row, input) serves 4 outputs (one per (input, output) pair and row made
// it vector-ALU-bound: config 2's 784 -> 64 layer 11.8 us); the wave's 4 row
// slices are added by a fixed butterfly into red[(rq * 64 + il2 * 8 + 4 og +
// c) * (DMAX + 1) + d], and the caller adds the 4 waves' rows in rq order.
// SYNC: a block barrier before red is written (red may overlay ts).
template <int DMAX, int TP, bool SYNC = false>
__device__ __forceinline__ void dc_small_sums(const float* ts, const float* ys, float* red, int rows,
                                              int gt) {
  const int lane = gt & 63, rq = gt >> 6;
  const int il2 = lane & 7, og = (lane >> 3) & 1, rs = rq * 4 + (lane >> 4);
  float acc[4][DMAX];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int d = 0; d < DMAX; ++d) acc[c][d] = 0.0f;
  for (int r = rs; r < rows; r += 16) {
    const float tv = ts[r * TP + il2], t2 = tv + tv;
    const f32x4_t yv = *reinterpret_cast<const f32x4_t*>(ys + r * 8 + og * 4);
    float pm = tv, pc = 1.0f;  // T_{-1} = t, T_0 = 1
#pragma unroll
    for (int d = 0; d < DMAX; ++d) {
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c][d] = fmaf(pc, yv[c], acc[c][d]);
      const float nx = fmaf(t2, pc, -pm);
      pm = pc;
      pc = nx;
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int d = 0; d < DMAX; ++d) {
      acc[c][d] += __shfl_xor(acc[c][d], 16);
      acc[c][d] += __shfl_xor(acc[c][d], 32);
    }
  if constexpr (SYNC) __syncthreads();
  if ((lane >> 4) == 0) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int d = 0; d < DMAX; ++d) red[(rq * 64 + il2 * 8 + og * 4 + c) * (DMAX + 1) + d] = acc[c][d];
  }
}

template <int DMAX>
__device__ __forceinline__ void dc_small_body(const float* __restrict__ dy, const float* __restrict__ t,
                                              float* __restrict__ dC, const DcOut& om,
                                              const Plan& p, int bx, int by) {
  __shared__ float ts[kDcSmallRows][9];
  __shared__ __attribute__((aligned(16))) float ys[kDcSmallRows][8];
  __shared__ float red[4][64][DMAX + 1];
  const int tid = threadIdx.x, q = tid & 63, rq = tid >> 6;
  const int il = q >> 3, ol = q & 7;
  const int i0 = bx * 8, o0 = by * 8;
  const int D = p.D;
  const int rows = (int)p.B;  // <= kDcSmallRows (dc_small_ok)
  // every load of the staging in flight at once (a rolled loop waited for
  // each pair of loads in turn: 8 round trips at 256 rows)
  constexpr int NLD = kDcSmallRows * 8 / 256;
  float tl[NLD], yl[NLD];
#pragma unroll
  for (int u = 0; u < NLD; ++u) {
    const int k = tid + 256 * u, r = k >> 3, c = k & 7;
    const bool in = r < rows;
    tl[u] = in && i0 + c < p.I ? t[(int64_t)r * p.I_sg + i0 + c] : 0.0f;
    yl[u] = in && o0 + c < p.O ? dy[(int64_t)r * p.O + o0 + c] : 0.0f;
  }
#pragma unroll
  for (int u = 0; u < NLD; ++u) {
    const int k = tid + 256 * u, r = k >> 3, c = k & 7;
    ts[r][c] = tl[u];
    ys[r][c] = yl[u];
  }
  __syncthreads();
  if constexpr (DMAX <= 9) {
    dc_small_sums<DMAX, 9>(&ts[0][0], &ys[0][0], &red[0][0][0], rows, tid);
  } else {
    // rows 4 at a time with 4 accumulator sets: independent recurrences and
    // LDS reads in flight together (one row at a time was latency-bound);
    // the sets are added in order at the end
    constexpr int RU = 4;
    float acc[RU][DMAX];
#pragma unroll
    for (int u = 0; u < RU; ++u)
#pragma unroll
      for (int d = 0; d < DMAX; ++d) acc[u][d] = 0.0f;
    const int per = (rows + 3) / 4, r0 = rq * per, r1 = min(rows, r0 + per);
    for (int r = r0; r < r1; r += RU) {
      float tv[RU], yv[RU];
#pragma unroll
      for (int u = 0; u < RU; ++u) {  // rows past r1 add zero (their dy is masked)
        const bool in = r + u < r1;
        tv[u] = ts[in ? r + u : r][il];
        yv[u] = in ? ys[r + u][ol] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const float t2 = tv[u] + tv[u];
        float pm = tv[u], pc = 1.0f;  // T_{-1} = t, T_0 = 1
#pragma unroll
        for (int d = 0; d < DMAX; ++d) {
          acc[u][d] = fmaf(pc, yv[u], acc[u][d]);
          const float nx = fmaf(t2, pc, -pm);
          pm = pc;
          pc = nx;
        }
      }
    }
#pragma unroll
    for (int d = 0; d < DMAX; ++d) red[rq][q][d] = ((acc[0][d] + acc[1][d]) + acc[2][d]) + acc[3][d];
  }
  __syncthreads();
  // the block's 8 x 8 x D results, spread over all threads: input il's 8
  // outputs are one contiguous run of 8 D floats of dC (one round trip for
  // the read-modify-write modes instead of D)
  const int ovalid = min(8, p.O - o0);
  for (int k = tid; k < 64 * D; k += 256) {
    const int kil = k / (8 * D), rem = k - kil * 8 * D, kol = rem / D, d = rem - kol * D;
    const int i = i0 + kil;
    if (i >= p.I || kol >= ovalid) continue;
    const int kq = kil * 8 + kol;
    const float g = ((red[0][kq][d] + red[1][kq][d]) + red[2][kq][d]) + red[3][kq][d];
    dc_write(dC + ((size_t)i * p.O + o0) * D + rem, g, om);
  }
}

template <int DMAX>
__global__ void __launch_bounds__(256)
k_dc_small(const float* __restrict__ dy, const float* __restrict__ t, float* __restrict__ dC,
           DcOut om, Plan p) {
  dc_small_body<DMAX>(dy, t, dC, om, p, blockIdx.x, blockIdx.y);
}

// The small dC with its optimizer step applied, which also writes the layer's
// packed operands for the next step from the updated coefficients, so that a
// resident training step runs no pack launch.  A block takes 32 inputs (one
// input block of the pack) x 8 outputs with four 256-thread groups; group q
// computes inputs 8q .. 8q + 7 as a k_dc_small block does (dc_small_sums, the
// waves added in the same order, so the same bits).  The updated 32 x 8 x D
// coefficients stay in LDS (zero for inputs and outputs past the layer, as in
// the pack's tile), and from them the block writes the pack's entries for its
// inputs and outputs, each formed as the pack forms it: the forward operand
// Cf (degrees 1..P), the input block's bias partial (groups of 4 inputs
// summed in order, then the 8 groups in order) and the dX operand Cb
// ((e + 1) C[i, o, e + 1]).  A null pointer skips that part.
template <bool BF> struct DcPackJob {
  const float* dy;                   // [B, O]
  const float* t;                    // tanh cache, row pitch I_sg
  float* C;                          // [I, O, D], receives the step by om
  DcOut om;
  Plan p;
  typename Elem<BF>::type* Cf;       // forward operand, or nullptr
  float* bias;                       // bias partials [NIB][O32] (the bias for NIB == 1), or nullptr
  typename Elem<BF>::type* Cb;       // dX operand, or nullptr
  int nx, nblocks;                   // input blocks of 32; blocks of the job
};
constexpr int kDcPackThreads = 1024;
constexpr int kDcPackTP = 40;  // t staging row pitch: a wave's 4 rows x 8 inputs hit distinct banks

template <int DMAX, int P, bool BF>
__device__ __forceinline__ void dc_pack_body(const DcPackJob<BF>& j, int bx, int by) {
  static_assert(DMAX <= 9, "the small dC sums take DMAX <= 9");
  using G = FwdGroup<P>;
  constexpr int TSF = kDcSmallRows * kDcPackTP;  // t [rows][32 inputs], pitch kDcPackTP
  constexpr int RDG = 4 * 64 * (DMAX + 1);       // one group's wave sums [4][64][DMAX + 1]
  static_assert(4 * RDG <= TSF, "the wave sums overlay the t staging");
  constexpr int CNP = 8 * DMAX + 1;              // updated-C row pitch
  __shared__ __attribute__((aligned(16))) float stage[TSF];
  __shared__ __attribute__((aligned(16))) float ys[kDcSmallRows * 8];
  __shared__ float cn[32 * CNP];
  const Plan& p = j.p;
  const int tid = threadIdx.x, grp = tid >> 8;
  const int i0 = bx * 32, o0 = by * 8;
  const int D = p.D;
  const int rows = (int)p.B;  // <= kDcSmallRows (dc_small_ok)
  // staging with every load in flight at once: t of the 32 inputs (one
  // 128-byte run per row), dy of the 8 outputs, and the coefficients the
  // step updates (element k of the tile's 32 x 8D run: input k / 8D)
  constexpr int NT = kDcSmallRows * 32 / kDcPackThreads, NY = kDcSmallRows * 8 / kDcPackThreads;
  constexpr int NE = (32 * 8 * DMAX + kDcPackThreads - 1) / kDcPackThreads;
  const int ne = 32 * 8 * D, ovalid = min(8, p.O - o0);
  float tl[NT], yl[NY], cold[NE];
#pragma unroll
  for (int m = 0; m < NE; ++m) {
    const int k = tid + kDcPackThreads * m;
    const int kil = k / (8 * D), rem = k - kil * 8 * D;
    const bool ok = k < ne && i0 + kil < p.I && rem / D < ovalid && j.om.mode != kDcStore;
    cold[m] = ok ? j.C[((size_t)(i0 + kil) * p.O + o0) * D + rem] : 0.0f;
  }
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    const int k = tid + kDcPackThreads * u, r = k >> 5, c = k & 31;
    tl[u] = r < rows && i0 + c < p.I ? j.t[(int64_t)r * p.I_sg + i0 + c] : 0.0f;
  }
#pragma unroll
  for (int u = 0; u < NY; ++u) {
    const int k = tid + kDcPackThreads * u, r = k >> 3, c = k & 7;
    yl[u] = r < rows && o0 + c < p.O ? j.dy[(int64_t)r * p.O + o0 + c] : 0.0f;
  }
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    const int k = tid + kDcPackThreads * u;
    stage[(k >> 5) * kDcPackTP + (k & 31)] = tl[u];
  }
#pragma unroll
  for (int u = 0; u < NY; ++u) ys[tid + kDcPackThreads * u] = yl[u];
  __syncthreads();
  // group grp: inputs 8 grp .. 8 grp + 7; its wave sums overlay the staging
  // once every group has read it (the barrier inside)
  dc_small_sums<DMAX, kDcPackTP, true>(stage + grp * 8, ys, stage + grp * RDG, rows, tid & 255);
  __syncthreads();
#pragma unroll
  for (int m = 0; m < NE; ++m) {
    const int k = tid + kDcPackThreads * m;
    if (k >= ne) break;
    const int kil = k / (8 * D), rem = k - kil * 8 * D, kol = rem / D, d = rem - kol * D;
    const int i = i0 + kil;
    float v = 0.0f;
    if (i < p.I && kol < ovalid) {
      const float* rd = stage + (kil >> 3) * RDG + ((kil & 7) * 8 + kol) * (DMAX + 1) + d;
      const float g = ((rd[0] + rd[64 * (DMAX + 1)]) + rd[128 * (DMAX + 1)]) + rd[192 * (DMAX + 1)];
      v = dc_apply_from(j.C + ((size_t)i * p.O + o0) * D + rem, cold[m], g, j.om);
    }
    cn[kil * CNP + rem] = v;
  }
  __syncthreads();
  if (j.bias && tid < 8) {
    float s = 0.0f;
    for (int g8 = 0; g8 < 8; ++g8) {
      float sg = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) sg += cn[(g8 * 4 + q) * CNP + tid * D];
      s += sg;
    }
    j.bias[(size_t)bx * p.O32 + o0 + tid] = s;
  }
  if (j.Cf) {  // the pack's k-blocks of input block bx, lanes of these 8 outputs
    const int ob = o0 >> 5, olo = o0 & 31;
    for (int item = tid; item < 2 * P * 16; item += kDcPackThreads) {
      const int kbl = item >> 4, g = (item >> 3) & 1, oj = item & 7;
      const int kb = bx * 2 * P + kbl;
      if (kb >= p.KB) continue;
      const int lane = olo + oj + 32 * g;
      const int r = kb / G::SGK, q = kb - r * G::SGK;
      const int s = q / G::KBG, h = q - s * G::KBG;
      float v[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int vv = 8 * h + jj;
        const int u = vv / P, d = vv % P + 1;
        const int i = r * G::SGI + g * 2 * G::IPG + s * (G::IPG / 2) + u;
        v[jj] = d <= p.deg ? cn[(i - i0) * CNP + oj * D + d] : 0.0f;
      }
      store_frag<BF>(j.Cf + cf_elem<BF>(p.KB, ob, kb, lane) - (size_t)lane * 8, lane, v);
    }
  }
  if (j.Cb) {  // output k-block o0 / 16, half (o0 / 8) % 2
    const int kbx = o0 >> 4, g = (o0 >> 3) & 1;
    for (int item = tid; item < P * 32; item += kDcPackThreads) {
      const int e = item >> 5, il = item & 31;
      float v[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
        v[jj] = (e + 1 <= p.deg) ? cn[il * CNP + jj * D + e + 1] * (float)(e + 1) : 0.0f;
      store_frag<BF>(j.Cb + ((size_t)(bx * P + e) * p.KBx + kbx) * kFragElems, il + 32 * g, v);
    }
  }
}

// Two layers' dC-and-pack in one launch: blocks [0, a.nblocks) take a, the
// next b.nblocks (may be 0) b, and with lm.part one more block the step's
// loss mean.
template <int DMAX, int P, bool BF>
__global__ void __launch_bounds__(kDcPackThreads)
k_dc_pack2(DcPackJob<BF> a, DcPackJob<BF> b, LossMean lm) {
  const int bid = blockIdx.x;
  if (bid < a.nblocks) dc_pack_body<DMAX, P, BF>(a, bid % a.nx, bid / a.nx);
  else if (bid < a.nblocks + b.nblocks)
    dc_pack_body<DMAX, P, BF>(b, (bid - a.nblocks) % b.nx, (bid - a.nblocks) / b.nx);
  else loss_mean_block(lm);
}

// Small dx: dx[b, i] = t'(x) sum_e U_e(t) sum_o dy[b, o] Cb(i, o, e) for
// layers whose reduction over outputs is short (config 2's 64 -> 10 layer),
// where the pipelined kernel would be all prologue.  Cb is the packed dX
// operand, (e + 1) C[i, o, e + 1] in the compute precision, read here in its
// fragment layout.  Block: 32 rows x 8 inputs, one (row, input) per thread;
// dy rows and the block's coefficients are staged in LDS with every load in
// flight at once.
constexpr int kDxSmallO = 64;  // outputs staged at once (all of them)
template <int P, bool BF>
__device__ __forceinline__ void dx_small_body(const float* __restrict__ dy,
                                              const typename Elem<BF>::type* __restrict__ Cb,
                                              const float* __restrict__ t, float* __restrict__ dx,
                                              const Plan& p, int bx, int by) {
  typedef typename Elem<BF>::type E;
  __shared__ float cs[8][kDxSmallO][P + 1];
  __shared__ float ys[32][kDxSmallO + 1];
  const int tid = threadIdx.x;
  const int64_t b0 = (int64_t)bx * 32;
  const int i0 = by * 8;
  constexpr int NC = 8 * kDxSmallO * P / 256, NY = 32 * kDxSmallO / 256;
  float cv[NC], yv[NY];
#pragma unroll
  for (int u = 0; u < NC; ++u) {  // k = (il, o, e): Cb fragment element of (i, o, e)
    const int k = tid + 256 * u, il = k / (kDxSmallO * P), rem = k - il * kDxSmallO * P;
    const int o = rem / P, e = rem - o * P, i = i0 + il;
    float v = 0.0f;
    if (i < p.I && o < p.O) {
      const size_t q = ((size_t)((i >> 5) * P + e) * p.KBx + (o >> 4)) * kFragElems +
                       ((i & 31) + 32 * ((o & 15) >> 3)) * 8 + (o & 7);
      if constexpr (BF) v = __uint_as_float((uint32_t)Cb[q] << 16);
      else v = Cb[q];
    }
    cv[u] = v;
  }
#pragma unroll
  for (int u = 0; u < NY; ++u) {
    const int k = tid + 256 * u, r = k / kDxSmallO, o = k - r * kDxSmallO;
    yv[u] = (b0 + r < p.B && o < p.O) ? dy[(b0 + r) * p.O + o] : 0.0f;
  }
#pragma unroll
  for (int u = 0; u < NC; ++u) {
    const int k = tid + 256 * u, il = k / (kDxSmallO * P), rem = k - il * kDxSmallO * P;
    cs[il][rem / P][rem % P] = cv[u];
  }
#pragma unroll
  for (int u = 0; u < NY; ++u) {
    const int k = tid + 256 * u;
    ys[k / kDxSmallO][k % kDxSmallO] = yv[u];
  }
  __syncthreads();
  const int r = tid >> 3, il = tid & 7;
  const int64_t b = b0 + r;
  const int i = i0 + il;
  if (b >= p.B || i >= p.I) return;
  float g[P];
#pragma unroll
  for (int e = 0; e < P; ++e) g[e] = 0.0f;
  for (int o = 0; o < p.O; ++o) {
    const float a = ys[r][o];
#pragma unroll
    for (int e = 0; e < P; ++e) g[e] = fmaf(a, cs[il][o][e], g[e]);
  }
  const float tv = t[b * p.I_sg + i], t2 = tv + tv;
  float up = 0.0f, u = 1.0f, s = 0.0f;  // U_{e-1}, U_e
#pragma unroll
  for (int e = 0; e < P; ++e) {
    s = fmaf(g[e], u, s);
    const float un = fmaf(t2, u, -up);
    up = u;
    u = un;
  }
  __builtin_nontemporal_store(s * input_slope(tv, p), dx + b * p.I + i);
}

template <int P, bool BF>
__global__ void __launch_bounds__(256)
k_dx_small(const float* __restrict__ dy, const typename Elem<BF>::type* __restrict__ Cb,
           const float* __restrict__ t, float* __restrict__ dx, Plan p) {
  dx_small_body<P, BF>(dy, Cb, t, dx, p, blockIdx.x, blockIdx.y);
}

bool dx_small_ok(const Plan& p) {
  // grid y = input blocks of 8 (launch_dx_small): at most 65535
  return p.O <= kDxSmallO && ceil_div(p.I, 8) <= 65535 &&
         (int64_t)p.B * p.I * p.O * p.P <= ((int64_t)1 << 27);
}

void launch_dx_small(const float* dy, const void* packed, const float* t, float* dx,
                     const Plan& p, hipStream_t s) {
  const dim3 grid((unsigned)ceil_div(p.B, 32), (unsigned)ceil_div(p.I, 8));
#define CKAN_DXS(PP, BB)                                                                       \
  hipLaunchKernelGGL((k_dx_small<PP, BB>), grid, dim3(256), 0, s, dy,                          \
                     reinterpret_cast<const typename Elem<BB>::type*>(packed) + packed_cf_elems(p), \
                     t, dx, p)
  const bool bf = p.esz == 2;
  switch (p.P) {
    case 2: if (bf) CKAN_DXS(2, true); else CKAN_DXS(2, false); break;
    case 4: if (bf) CKAN_DXS(4, true); else CKAN_DXS(4, false); break;
    case 8: if (bf) CKAN_DXS(8, true); else CKAN_DXS(8, false); break;
    default: if (bf) CKAN_DXS(16, true); else CKAN_DXS(16, false); break;
  }
#undef CKAN_DXS
}


// Both small backward kernels of one layer in one launch (they read the same
// dy and tanh cache and write different outputs: dx, and dC or the layer's
// coefficients): blocks [0, ndx) take dx, the next ndc dC, and with lm.part
// one more block takes the step's loss mean.
template <int P, bool BF>
__global__ void __launch_bounds__(256)
k_bwd_small(const float* __restrict__ dy, const typename Elem<BF>::type* __restrict__ Cb,
            const float* __restrict__ t, float* __restrict__ dx, float* __restrict__ dC, DcOut om,
            Plan p, int nx_dx, int ndx, int nx_dc, int ndc, LossMean lm) {
  const int bid = blockIdx.x;
  if (bid < ndx) dx_small_body<P, BF>(dy, Cb, t, dx, p, bid % nx_dx, bid / nx_dx);
  else if (bid < ndx + ndc) dc_small_body<P + 1>(dy, t, dC, om, p, (bid - ndx) % nx_dc, (bid - ndx) / nx_dc);
  else loss_mean_block(lm);
}

// One round of the fused launch: larger layers keep the two launches, each at
// its own occupancy.  A k_bwd_small block holds the static LDS of all three
// bodies at once (about 55 KB at P = 8, 80 KB at P = 16), so the blocks one CU
// holds are read from the runtime's occupancy calculation for the
// instantiation, not assumed.
// The loss mean alone, where the backward takes no small one-launch path.
__global__ void __launch_bounds__(256) k_loss_mean(LossMean lm) { loss_mean_block(lm); }

void launch_loss_mean(const LossMean& lm, hipStream_t s) {
  hipLaunchKernelGGL(k_loss_mean, dim3(1), dim3(256), 0, s, lm);
}

template <int P, bool BF>
static int bwd_small_blocks_per_cu() {
  static const int n = [] {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, k_bwd_small<P, BF>, 256, 0) != hipSuccess ||
        v < 1)
      v = 1;
    return v;
  }();
  return n;
}

bool bwd_small_one_launch(const Plan& p) {
  const int64_t ndx = ceil_div(p.B, 32) * ceil_div(p.I, 8), ndc = ceil_div(p.I, 8) * ceil_div(p.O, 8);
  const bool bf = p.esz == 2;
  int per_cu;
  switch (p.P) {
    case 2: per_cu = bf ? bwd_small_blocks_per_cu<2, true>() : bwd_small_blocks_per_cu<2, false>(); break;
    case 4: per_cu = bf ? bwd_small_blocks_per_cu<4, true>() : bwd_small_blocks_per_cu<4, false>(); break;
    case 8: per_cu = bf ? bwd_small_blocks_per_cu<8, true>() : bwd_small_blocks_per_cu<8, false>(); break;
    default: per_cu = bf ? bwd_small_blocks_per_cu<16, true>() : bwd_small_blocks_per_cu<16, false>(); break;
  }
  return ndx + ndc <= (int64_t)per_cu * kNumCUs;
}

void launch_bwd_small(const float* dy, const void* packed, const float* t, float* dx, float* dC,
                      DcOut om, const Plan& p, hipStream_t s, LossMean lm) {
  const int nx_dx = (int)ceil_div(p.B, 32), nx_dc = (int)ceil_div(p.I, 8);
  const int ndx = nx_dx * (int)ceil_div(p.I, 8), ndc = nx_dc * (int)ceil_div(p.O, 8);
  const dim3 grid((unsigned)(ndx + ndc + (lm.part ? 1 : 0)));
#define CKAN_BWS(PP, BB)                                                                        \
  hipLaunchKernelGGL((k_bwd_small<PP, BB>), grid, dim3(256), 0, s, dy,                          \
                     reinterpret_cast<const typename Elem<BB>::type*>(packed) + packed_cf_elems(p), \
                     t, dx, dC, om, p, nx_dx, ndx, nx_dc, ndc, lm)
  const bool bf = p.esz == 2;
  switch (p.P) {
    case 2: if (bf) CKAN_BWS(2, true); else CKAN_BWS(2, false); break;
    case 4: if (bf) CKAN_BWS(4, true); else CKAN_BWS(4, false); break;
    case 8: if (bf) CKAN_BWS(8, true); else CKAN_BWS(8, false); break;
    default: if (bf) CKAN_BWS(16, true); else CKAN_BWS(16, false); break;
  }
#undef CKAN_BWS
}

bool dc_small_ok(const Plan& p) {
  // fp32 work ~ pairs * rows * (2 D + 2) lane-instructions: below ~2^28 the
  // vector ALU finishes in a few microseconds, ahead of the pipelined kernel's
  // prologue (and its split sum)
  const int64_t pairs = (int64_t)p.I * p.O;
  // grid y = output blocks of 8 (launch_dc_small): at most 65535
  return p.B >= 1 && p.B <= kDcSmallRows && ceil_div(p.O, 8) <= 65535 &&
         pairs * p.B * (2 * p.D + 2) <= ((int64_t)1 << 28);
}

void launch_dc_small(const float* dy, const float* t, float* dC, DcOut om, const Plan& p,
                     hipStream_t s) {
  const dim3 grid((unsigned)ceil_div(p.I, 8), (unsigned)ceil_div(p.O, 8));
  switch (p.P) {
    case 2: hipLaunchKernelGGL((k_dc_small<3>), grid, dim3(256), 0, s, dy, t, dC, om, p); break;
    case 4: hipLaunchKernelGGL((k_dc_small<5>), grid, dim3(256), 0, s, dy, t, dC, om, p); break;
    case 8: hipLaunchKernelGGL((k_dc_small<9>), grid, dim3(256), 0, s, dy, t, dC, om, p); break;
    default: hipLaunchKernelGGL((k_dc_small<17>), grid, dim3(256), 0, s, dy, t, dC, om, p); break;
  }
}

bool dc_pack_ok(const Plan& p) {
  return dc_small_ok(p) && p.P <= 8 && ceil_div(p.I, 32) * ceil_div(p.O, 8) < (1 << 29);
}

template <int P, bool BF>
static void launch_dc_pack_t(const DcPackArgs& a, const DcPackArgs* b, const LossMean& lm,
                             hipStream_t s) {
  typedef typename Elem<BF>::type E;
  auto job = [](const DcPackArgs& x) {
    DcPackJob<BF> j;
    const Plan& q = x.p;
    char* base = reinterpret_cast<char*>(x.packed);
    j.dy = x.dy;
    j.t = x.t;
    j.C = x.C;
    j.om = x.om;
    j.p = q;
    j.Cf = x.cf ? reinterpret_cast<E*>(base) : nullptr;
    // the pack's bias pointer: the bias itself when there is one input block
    j.bias = x.cf ? reinterpret_cast<float*>(base + (q.NIB == 1 ? packed_biasf_offset(q)
                                                                 : packed_bias_offset(q)))
                  : nullptr;
    j.Cb = x.cb ? reinterpret_cast<E*>(base) + packed_cf_elems(q) : nullptr;
    j.nx = (int)ceil_div(q.I, 32);
    j.nblocks = j.nx * (int)ceil_div(q.O, 8);
    return j;
  };
  const DcPackJob<BF> ja = job(a);
  DcPackJob<BF> jb{};
  if (b) jb = job(*b);
  const dim3 grid((unsigned)(ja.nblocks + jb.nblocks + (lm.part ? 1 : 0)));
  hipLaunchKernelGGL((k_dc_pack2<P + 1, P, BF>), grid, dim3(kDcPackThreads), 0, s, ja, jb, lm);
}

void launch_dc_pack(const DcPackArgs& a, const DcPackArgs* b, hipStream_t s, LossMean lm) {
  const bool bf = a.p.esz == 2;
#define CKAN_DCP(PP) bf ? launch_dc_pack_t<PP, true>(a, b, lm, s) : launch_dc_pack_t<PP, false>(a, b, lm, s)
  switch (a.p.P) {
    case 2: CKAN_DCP(2); break;
    case 4: CKAN_DCP(4); break;
    default: CKAN_DCP(8); break;
  }
#undef CKAN_DCP
}

void launch_prep_dy(const float* dy, void* dYx, void* dYc, float* colsum_part, const Plan& p,
                    bool need_dx, bool need_dc, hipStream_t s) {
  const int64_t dx_rows = need_dx ? dx_row_frags(p) * 32 : 0;  // dYx rows incl. zero padding
  int64_t row_end = p.B32 > p.Bc ? p.B32 : p.Bc;
  if (dx_rows > row_end) row_end = dx_rows;
  const int nob = p.O64 / 32;
  const int nbb = (int)ceil_div(row_end, kPrepRows);
  const int64_t blocks = ceil_div((int64_t)nob * nbb, 4);
  dim3 grid((unsigned)(blocks < kPrepBlocks ? blocks : kPrepBlocks));
  if (p.esz == 2)
    hipLaunchKernelGGL((k_prep_dy<true>), grid, dim3(256), 0, s, dy,
                       reinterpret_cast<uint16_t*>(dYx), reinterpret_cast<uint16_t*>(dYc),
                       colsum_part, p, (int)need_dx, (int)need_dc, nob, nbb, dx_rows, (int)is_al16(dy));
  else
    hipLaunchKernelGGL((k_prep_dy<false>), grid, dim3(256), 0, s, dy,
                       reinterpret_cast<float*>(dYx), reinterpret_cast<float*>(dYc),
                       colsum_part, p, (int)need_dx, (int)need_dc, nob, nbb, dx_rows, (int)is_al16(dy));
}

float* launch_colsum_reduce(float* colsum_part, const Plan& p, hipStream_t s) {
  float* colsum = colsum_part + (size_t)p.NBB * p.O32;
  hipLaunchKernelGGL(k_col_reduce, dim3((unsigned)ceil_div(p.O32, 64)), dim3(256), 0, s,
                     colsum_part, p.NBB, p.O32, p.O32, colsum);
  return colsum;
}

void launch_dc_finalize(const float* part, int S, const float* colsum, float* dC,
                        DcOut om, const Plan& p, hipStream_t s) {
  dim3 grid((unsigned)ceil_div(p.I, 16), (unsigned)ceil_div(p.O, 64));
  switch (p.P) {
    case 2: hipLaunchKernelGGL((k_dc_finalize<2>), grid, dim3(256), 0, s, part, S, colsum, dC, om, p); break;
    case 4: hipLaunchKernelGGL((k_dc_finalize<4>), grid, dim3(256), 0, s, part, S, colsum, dC, om, p); break;
    case 8: hipLaunchKernelGGL((k_dc_finalize<8>), grid, dim3(256), 0, s, part, S, colsum, dC, om, p); break;
    default: hipLaunchKernelGGL((k_dc_finalize<16>), grid, dim3(256), 0, s, part, S, colsum, dC, om, p); break;
  }
}

// dC[q] (stored, added or applied as an SGD step, by om) = sum_z part[z][q],
// z in split order (slices of I*O*D floats).  The split sum is formed first,
// so accumulating adds exactly the gradient a storing call writes.
__global__ void __launch_bounds__(256)
k_dc_sum(const float* __restrict__ part, int S, float* __restrict__ dC, int64_t n, DcOut om) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x) {
    // 16 loads in flight per round trip, added in split order
    float acc = 0.0f;
    for (int z0 = 0; z0 < S; z0 += 16) {
      float v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = z0 + j < S ? part[(size_t)(z0 + j) * n + q] : 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (z0 + j < S) acc += v[j];
    }
    dc_write(dC + q, acc, om);
  }
}

// The same four elements per thread (float4), with the destination's read
// (SGD / accumulate modes) issued together with the partials' loads: config
// 4's 4.5 M-element layers 27 -> 18 us.
__global__ void __launch_bounds__(256)
k_dc_sum4(const f32x4_t* __restrict__ part, int S, f32x4_t* __restrict__ dC, int64_t n4, DcOut om) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n4;
       q += (int64_t)gridDim.x * blockDim.x) {
    const bool rmw = om.mode == kDcSgd || om.mode == kDcAccumulate;
    const f32x4_t c = rmw ? dC[q] : f32x4_t{0.f, 0.f, 0.f, 0.f};
    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int z0 = 0; z0 < S; z0 += 8) {
      f32x4_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v[j] = z0 + j < S ? __builtin_nontemporal_load(part + (size_t)(z0 + j) * n4 + q)
                          : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (z0 + j < S) acc += v[j];
    }
    if (om.mode == kDcAccumulate) {
      dC[q] = c + acc;
    } else if (om.mode == kDcSgd) {
      f32x4_t r;
      r.x = sgd_update(c.x, acc.x, om.lr, om.wd);
      r.y = sgd_update(c.y, acc.y, om.lr, om.wd);
      r.z = sgd_update(c.z, acc.z, om.lr, om.wd);
      r.w = sgd_update(c.w, acc.w, om.lr, om.wd);
      dC[q] = r;
    } else {
      dc_write4(dC + q, acc, om);
    }
  }
}

void launch_dc_sum(const float* part, int S, float* dC, DcOut om, const Plan& p, hipStream_t s) {
  const int64_t n = (int64_t)p.I * p.O * p.D;
  if (n % 4 == 0 && is_al16(part) && is_al16(dC)) {
    hipLaunchKernelGGL(k_dc_sum4, dim3(grid_for(n / 4)), dim3(256), 0, s,
                       reinterpret_cast<const f32x4_t*>(part), S, reinterpret_cast<f32x4_t*>(dC),
                       n / 4, om);
    return;
  }
  hipLaunchKernelGGL(k_dc_sum, dim3(grid_for(n)), dim3(256), 0, s, part, S, dC, n, om);
}

void launch_sgd(float* p, const float* g, int64_t n, float lr, float wd, hipStream_t s) {
  hipLaunchKernelGGL(k_sgd, dim3(grid_for(n)), dim3(256), 0, s, p, g, n, lr, wd);
}

void launch_adam(float* p, const float* g, float* m, float* v, int64_t n, float w1, float beta2,
                 float one_m_beta2, float bc2_sqrt, float eps, float neg_step, float wd,
                 hipStream_t s) {
  hipLaunchKernelGGL(k_adam, dim3(grid_for(n)), dim3(256), 0, s, p, g, m, v, n, w1, beta2,
                     one_m_beta2, bc2_sqrt, eps, neg_step, wd);
}

void launch_basis(const float* t, int64_t n, int deg, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_basis, dim3(grid_for(n)), dim3(256), 0, s, t, n, deg, out);
}

void launch_basis_bwd(const float* t, const float* g, int64_t n, int deg, float* dt,
                      hipStream_t s) {
  hipLaunchKernelGGL(k_basis_bwd, dim3(grid_for(n)), dim3(256), 0, s, t, g, n, deg, dt);
}

void launch_zero_f32(float* ptr, int64_t n, hipStream_t s) {
  if (n > 0) hipLaunchKernelGGL(k_zero_f32, dim3(grid_for(n)), dim3(256), 0, s, ptr, n);
}

void launch_zero(void* ptr, size_t bytes, hipStream_t s) {
  const int64_t n16 = (int64_t)(bytes / 16);
  if (n16 > 0)
    hipLaunchKernelGGL(k_zero, dim3(grid_for(n16)), dim3(256), 0, s,
                       reinterpret_cast<u32x4_t*>(ptr), n16);
}

}  // namespace ckan
