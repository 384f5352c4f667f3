// The three MFMA contractions of the ChebyKAN layer on gfx950.
//
//   forward  y[b,o]        = bias[o] + sum_{i,d>=1} T_d(t[b,i]) C[i,o,d]
//            M = rows, N = outputs, reduction = (input, degree)
//   dX       dT[b,(i,d)]   = sum_o dy[b,o] C[i,o,d]; dx[b,i] = (1-t^2) sum_d d U_{d-1}(t) dT
//            M = rows, N = (input, degree), reduction = outputs
//   dC       dC[i,o,d]     = sum_b T_d(t[b,i]) dy[b,o]
//            M = (input, degree), N = outputs, reduction = rows
//
// The basis T_d(tanh x) never reaches HBM.  In the forward each lane builds
// its MFMA A fragment in registers from 2*IPG tanh values with the three-term
// recurrence; in dC the block builds the basis operand once per stage into
// LDS.  The coefficient operands are pre-packed fragment-major and staged
// through LDS with a register double buffer (one barrier per stage).
#include <atomic>
#include <type_traits>

#include "ckan_kernels.hpp"

namespace ckan {

// s0 + sum_{z < n} src[z * stride] (n >= 1), added in z order.  Every load of
// a round is issued before its first addition, so a long split count does not
// serialise on memory latency: up to 16 terms one round of 16, else rounds of
// 64 (the fused cross-entropy tail sums 49 splits per output).  The loads are
// unconditional, past n from the last term's address (a load under a branch
// is waited for inside that branch, one round trip per term), and a
// scheduling barrier keeps them ahead of the additions (left to itself the
// compiler issued them 8 at a time, each batch waited for).
__device__ __forceinline__ float split_sum(const float* __restrict__ src, size_t stride,
                                           unsigned n, float s0) {
  float s = s0;
  if (n <= 16) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = src[(size_t)((unsigned)j < n ? j : n - 1) * stride];
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the first use
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if ((unsigned)j < n) s += v[j];
    return s;
  }
  for (unsigned z0 = 0; z0 < n; z0 += 64) {
    float v[64];
#pragma unroll
    for (int j = 0; j < 64; ++j) v[j] = src[(size_t)(z0 + j < n ? z0 + j : n - 1) * stride];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 64; ++j)
      if (z0 + j < n) s += v[j];
  }
  return s;
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// Block = 4 waves arranged WGM x WGN; wave tile NM x NN fragments of 32x32.
// The reduction runs over super-groups (SG): SGI inputs = SGK k-blocks.
// With gridDim.z > 1 the SGs are split over blocks; each block writes its
// partial tile to the workspace and k_fwd_reduce, a separate launch, adds the
// partials in fixed split order.
// XT: tc is x itself (rows unpadded, I == I_sg, 16-byte aligned); the block
// maps each value by the input map as it loads it (the arithmetic of
// launch_tanh), and the first column block's first wave column stores the
// mapped values into the tanh cache tout for the backward (each value once).
template <int P, bool BF, int NM, int NN, int WGM, int WGN, bool XT = false>
__global__ void __launch_bounds__(256)
k_fwd(const float* __restrict__ tc, const typename Elem<BF>::type* __restrict__ Cf,
      const float* __restrict__ bias_f, float* __restrict__ y, float* __restrict__ part,
      Plan p, int sg_per_split, const float* __restrict__ bias_part, int nib,
      float* __restrict__ bias_out, float* __restrict__ tout) {
  typedef typename Elem<BF>::type E;
  typedef FwdGroup<P> G;
  static_assert(WGM * WGN == 4, "4 waves per block");
  constexpr int BNF = WGN * NN;
  constexpr int BM = WGM * NM * 32;
  constexpr int STAGE = BNF * G::SGK * kFragElems;
  constexpr int CE = 16 / (int)sizeof(E);
  constexpr int NCHUNK = STAGE / CE;
  constexpr int CPT = NCHUNK / 256;
  constexpr int CPN = G::SGK * kFragElems / CE;  // chunks per N fragment
  static_assert(NCHUNK % 256 == 0, "stage must split evenly over 256 threads");
  __shared__ __attribute__((aligned(16))) E lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int g = lane >> 5;
  const int64_t m_blk = (int64_t)blockIdx.x * BM;
  const int nb0 = blockIdx.y * BNF;
  const int nsg = p.I_sg / G::SGI;
  const int sg0 = blockIdx.z * sg_per_split;
  const int sg1 = min(nsg, sg0 + sg_per_split);

  const float* trow[NM];
  bool rvalid[NM];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi) {
    const int64_t r = m_blk + (wm * NM + mi) * 32 + (lane & 31);
    rvalid[mi] = r < p.B;
    trow[mi] = tc + (rvalid[mi] ? r : 0) * p.I_sg + g * G::LANE_T;
  }

  u32x4_t pre[CPT];
  auto gload = [&](int sg) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      const int c = tid + q * 256;
      const int nbl = c / CPN, off = c - nbl * CPN;
      const int nb = nb0 + nbl;
      // chunk off of the stage: k-block off / CPF, lane-chunk off % CPF (a lane
      // holds 8 values: one chunk for bf16, two for fp32)
      constexpr int CPF = kFragElems / CE;
      const int kbl = off / CPF, lc = off - kbl * CPF;
      if (nb < p.NBf)
        pre[q] = *reinterpret_cast<const u32x4_t*>(
            Cf + cf_elem<BF>(p.KB, nb, sg * G::SGK + kbl, lc * CE / 8) + (size_t)(lc * CE % 8));
      else
        pre[q] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto lstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < CPT; ++q)
      *reinterpret_cast<u32x4_t*>(lds + buf * STAGE + (tid + q * 256) * CE) = pre[q];
  };

  f32x16_t acc[NM][NN];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int ni = 0; ni < NN; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.0f;

  // tanh values of the next super-group, prefetched one stage ahead
  f32x4_t tnext[NM][G::LANE_T / 4];
  auto tload = [&](int sg) __attribute__((always_inline)) {
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      const f32x4_t* src = reinterpret_cast<const f32x4_t*>(trow[mi] + (size_t)sg * G::SGI);
#pragma unroll
      for (int q = 0; q < G::LANE_T / 4; ++q)
        tnext[mi][q] = rvalid[mi] ? src[q] : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  };

  if (sg0 < sg1) {
    gload(sg0);
    tload(sg0);
    lstore(0);
  }
  __syncthreads();

  for (int sg = sg0; sg < sg1; ++sg) {
    const int buf = (sg - sg0) & 1;
    const bool more = sg + 1 < sg1;
    f32x4_t tcur[NM][G::LANE_T / 4];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int q = 0; q < G::LANE_T / 4; ++q) tcur[mi][q] = tnext[mi][q];
    if (more) {
      gload(sg + 1);
      tload(sg + 1);
    }

    Frag<BF> af[NM][G::SGK];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      float tv[G::LANE_T];
#pragma unroll
      for (int q = 0; q < G::LANE_T / 4; ++q) {
        if constexpr (XT) {
          f32x4_t m;
#pragma unroll
          for (int e = 0; e < 4; ++e) m[e] = input_map(tcur[mi][q][e], p.imap, p.ima, p.imb);
          tcur[mi][q] = m;
        }
        tv[4 * q + 0] = tcur[mi][q][0]; tv[4 * q + 1] = tcur[mi][q][1];
        tv[4 * q + 2] = tcur[mi][q][2]; tv[4 * q + 3] = tcur[mi][q][3];
      }
      if constexpr (XT) {  // the waves along N map the same rows: the first stores them
        if (blockIdx.y == 0 && wn == 0 && rvalid[mi]) {
          const int64_t r = m_blk + (wm * NM + mi) * 32 + (lane & 31);
          f32x4_t* dst = reinterpret_cast<f32x4_t*>(tout + r * p.I_sg + (size_t)sg * G::SGI + g * G::LANE_T);
#pragma unroll
          for (int q = 0; q < G::LANE_T / 4; ++q) dst[q] = tcur[mi][q];
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float vals[8 * G::KBG];
#pragma unroll
        for (int u = 0; u < G::IPG / 2; ++u) cheb_T<P>(tv[s * (G::IPG / 2) + u], vals + u * P);
#pragma unroll
        for (int h = 0; h < G::KBG; ++h) af[mi][s * G::KBG + h] = make_frag<BF>(vals + 8 * h);
      }
    }

    const E* sb = lds + buf * STAGE;
#pragma unroll
    for (int kbl = 0; kbl < G::SGK; ++kbl) {
#pragma unroll
      for (int ni = 0; ni < NN; ++ni) {
        const Frag<BF> bfr = load_frag<BF>(sb + ((wn * NN + ni) * G::SGK + kbl) * kFragElems, lane);
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) mma(acc[mi][ni], af[mi][kbl], bfr);
      }
    }
    if (more) lstore(buf ^ 1);
    __syncthreads();
  }

  const bool split = gridDim.z > 1;
  if (!split) {
    // nib > 0: the bias from its per-input-block partials (and the first row
    // of blocks fills the packed bias slot for later forwards)
    if (nib > 0 && blockIdx.x == 0)
      for (int idx = threadIdx.x; idx < BNF * 32; idx += 256) {
        const int o = nb0 * 32 + idx;
        if (o < p.O32) bias_out[o] = bias_from_parts(bias_part, nib, p.O32, o);
      }
#pragma unroll
    for (int ni = 0; ni < NN; ++ni) {
      const int o = (nb0 + wn * NN + ni) * 32 + (lane & 31);
      if (o >= p.O) continue;
      const float bias = nib > 0 ? bias_from_parts(bias_part, nib, p.O32, o) : bias_f[o];
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) {
        const int64_t r0 = m_blk + (wm * NM + mi) * 32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t r = r0 + acc_row(v, g);
          if (r < p.B) y[r * p.O + o] = acc[mi][ni][v] + bias;
        }
      }
    }
    return;
  }

  // split-K: write the partial tile; k_fwd_reduce adds the splits in order
#pragma unroll
  for (int ni = 0; ni < NN; ++ni) {
    const int nb = nb0 + wn * NN + ni;
    if (nb >= p.NBf) continue;
    const int o = nb * 32 + (lane & 31);
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      const int64_t r0 = m_blk + (wm * NM + mi) * 32;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t r = r0 + acc_row(v, g);
        if (r < p.B32)
          part[((size_t)blockIdx.z * p.B32 + r) * p.O32 + o] = acc[mi][ni][v];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Forward, large-batch pipeline.  Block tile 256 rows x 128 outputs, 8 waves
// (2 per SIMD): waves 0-3 ("half 0") take the even super-groups of the
// reduction and waves 4-7 the odd ones, each half covering the whole tile
// (4 waves along rows, 2 x 4 fragments each); the two partial tiles are summed
// through LDS at the end.  Two waves per SIMD let one wave's MFMAs run while
// the other generates its basis fragments or waits on LDS, within the
// 256-register budget, without global split-K partials.
//
// Each super-group stage (coefficient fragments for 128 outputs and the
// 256 x SGI tanh tile) is copied global -> LDS by global_load_lds_dwordx4
// into a ring of NPB stage pairs, issued one pair-iteration ahead; a pair
// costs one barrier.  Out-of-range rows and output fragments read a clamped
// in-bounds address; their results are never stored.
// ---------------------------------------------------------------------------
// Workgroups go to the 8 XCDs round-robin by linear id, and each XCD has its
// own L2.  When the grid is exactly 256 tiles of (8a) x (4b), give each XCD an
// 8 x 4 patch (8 values of the x tile index, 4 of y) so that the operands the
// patch shares stay in one L2; otherwise keep the launch order.
__device__ __forceinline__ void xcd_patch(int& bx, int& by) {
  bx = blockIdx.x;
  by = blockIdx.y;
  if (gridDim.x * gridDim.y == 256 && gridDim.x % 8 == 0 && gridDim.y % 4 == 0 && gridDim.z == 1) {
    const int lin = blockIdx.x + gridDim.x * blockIdx.y;
    const int xcd = lin & 7, loc = lin >> 3;
    const int px = gridDim.x / 8;  // patches along x
    bx = (xcd % px) * 8 + (loc & 7);
    by = (xcd / px) * 4 + (loc >> 3);
  }
}

// BNF_: output fragments (32 columns each) per block; 2 for layers of at most
// 64 outputs, whose 4-fragment tile would run half its MFMAs on padding.
template <int P, bool BF, int BNF_ = 4>
struct FwdPipe {
  typedef typename Elem<BF>::type E;
  typedef FwdGroup<P> G;
  static constexpr int NM = 2, NN = BNF_, BM = 256, BNF = BNF_, THREADS = 512;
  static constexpr int B_BYTES = BNF * G::SGK * kFragElems * (int)sizeof(E);
  static constexpr int T_BYTES = BM * G::SGI * 4;
  static constexpr int STAGE_BYTES = B_BYTES + T_BYTES;
  static constexpr int PAIR_BYTES = 2 * STAGE_BYTES;
  static constexpr int RED_BYTES = BM * BNF * 32 * 4;  // one partial tile, fp32
  static constexpr int NPB_FIT = (160 * 1024) / PAIR_BYTES;
  static constexpr int NPB = NPB_FIT > 3 ? 3 : NPB_FIT;
  static constexpr int RING_BYTES = NPB * PAIR_BYTES;
  // bias sums of the block's outputs (epilogue only, after the halves' tiles)
  static constexpr int BIAS_OFF = RED_BYTES + 16;
  static constexpr int BIAS_END = BIAS_OFF + BNF * 32 * 4;
  static constexpr int LDS_BYTES = RING_BYTES > BIAS_END ? RING_BYTES : BIAS_END;
  // dma16 ops per thread per stage (each op moves 512 x 16 bytes per block)
  static constexpr int B_OPS = B_BYTES / (16 * THREADS);
  static constexpr int T_OPS = T_BYTES / (16 * THREADS);
  static constexpr int OPS = 2 * (B_OPS + T_OPS);  // per pair
  static constexpr bool kOk = NPB >= 2 && LDS_BYTES <= 160 * 1024 && RED_BYTES + 16 <= LDS_BYTES &&
                              B_BYTES % (16 * THREADS) == 0 && T_BYTES % (16 * THREADS) == 0;
};

// XOR applied to the 16-byte chunk index of row r of the forward kernel's tanh
// tile (CR chunks per row).  A wave reads one chunk of 32 consecutive rows per
// instruction; with it, every 16-lane (64 banks) and 8-lane (32 banks) group of
// a 16-byte read covers distinct banks.  XOR-linear in the row bits.
template <int CR> __device__ __forceinline__ int fwd_t_xor(int r) {
  if constexpr (CR == 2) return ((r >> 2) ^ (r >> 3)) & 1;
  else if constexpr (CR == 4) return ((r >> 2) & 1) | ((((r >> 1) ^ (r >> 3)) & 1) << 1);
  else return ((r >> 1) & 1) | (((r >> 2) & 1) << 1) | (((r ^ (r >> 3)) & 1) << 2);
}

// The bias: bias_f[o] when nib == 0; otherwise the block sums the nib
// per-input-block partials bias_part[ib][o] itself (in the order k_col_reduce
// adds them, so the two give the same bits), and the first row tile also
// writes the sums to bias_out.  OT (unsplit launches only): store tanh(y)
// in place of y, for the next layer of a stack.
template <int P, bool BF, bool OT, int BNF_ = 4>
__global__ void __launch_bounds__(512)
k_fwd_pipe(const float* __restrict__ tc, const typename Elem<BF>::type* __restrict__ Cf,
           const float* __restrict__ bias_f, float* __restrict__ y, float* __restrict__ part,
           Plan p, int sg_per_split, const float* __restrict__ bias_part, int nib,
           float* __restrict__ bias_out) {
  typedef FwdPipe<P, BF, BNF_> K;
  typedef typename K::E E;
  typedef typename K::G G;
  constexpr int NM = K::NM, NN = K::NN, BM = K::BM, BNF = K::BNF, NPB = K::NPB;
  constexpr int TH = K::THREADS;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = wave >> 2, wq = wave & 3;
  const int g = lane >> 5;
  int bx, by;
  xcd_patch(bx, by);
  const int64_t m_blk = (int64_t)bx * BM;
  const int nb0 = by * BNF;
  const int nsg = p.I_sg / G::SGI;
  const int sg0 = blockIdx.z * sg_per_split;
  const int sg1 = min(nsg, sg0 + sg_per_split);
  const int npair = (sg1 - sg0 + 1) / 2;

  // DMA: the 4 waves of half 0 issue every copy of a stage (HB_OPS coefficient
  // and HT_OPS tanh copies per thread); chunk c = (q*4 + wq)*64 + lane lands at
  // byte 16*c of the stage's coefficient or tanh area.  Sources are a
  // wave-uniform base (the block's first output fragment / row, plus the
  // stage) and a per-lane 32-bit offset fixed for the kernel.
  constexpr int HB_OPS = 2 * K::B_OPS, HT_OPS = 2 * K::T_OPS, HOPS = 2 * (HB_OPS + HT_OPS);
  constexpr int CPF = kFragElems * (int)sizeof(E) / 16;  // 16-byte chunks per fragment
  const int wqs = __builtin_amdgcn_readfirstlane(wq);
  const E* cf0 = Cf + cf_elem<BF>(p.KB, nb0, 0, 0);
  const char* bbase = reinterpret_cast<const char*>(cf0);
  uint32_t boff[HB_OPS];
#pragma unroll
  for (int q = 0; q < HB_OPS; ++q) {
    const int c = (q * 4 + wq) * 64 + lane;
    const int nbl = c / (G::SGK * CPF), off = c - nbl * (G::SGK * CPF);
    const int nb = min(nb0 + nbl, p.NBf - 1);
    const int kbl = off / CPF, lc = off - kbl * CPF;  // k-block of the stage, lane-chunk
    constexpr int CE = 16 / (int)sizeof(E);
    const E* src = Cf + cf_elem<BF>(p.KB, nb, kbl, lc * CE / 8) + (lc * CE % 8);
    boff[q] = (uint32_t)((size_t)(src - cf0) * sizeof(E));
  }
  const char* tbase = reinterpret_cast<const char*>(tc) + (size_t)m_blk * p.I_sg * 4;
  uint32_t toff[HT_OPS];
#pragma unroll
  for (int q = 0; q < HT_OPS; ++q) {
    const int c = (q * 4 + wq) * 64 + lane;
    const int rl = c / (G::SGI / 4), part4 = c - rl * (G::SGI / 4);  // stored chunk
    int64_t r = m_blk + rl;
    if (r >= p.B) r = p.B - 1;
    toff[q] = (uint32_t)(((size_t)(r - m_blk) * p.I_sg + (part4 ^ fwd_t_xor<G::SGI / 4>(rl)) * 4) * 4);
  }
  // one super-group further: SGK k-blocks, in every stream (bf16) or fragment column
  const size_t b_stride =
      (cf_elem<BF>(p.KB, 0, G::SGK, 0) - cf_elem<BF>(p.KB, 0, 0, 0)) * sizeof(E);
  const size_t t_stride = (size_t)G::SGI * 4;
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

  // stage `sg` (if it exists) into ring slot `slot` (0 .. 2*NPB-1); half 0 only
  auto issue = [&](int sg, int slot) __attribute__((always_inline)) {
    if (sg >= sg1) return;
    const uint32_t l = lds0 + slot * K::STAGE_BYTES + wqs * 1024;
#pragma unroll
    for (int q = 0; q < HB_OPS; ++q)
      dma16s_salu(bbase + (size_t)sg * b_stride, boff[q], l + q * 4096);
#pragma unroll
    for (int q = 0; q < HT_OPS; ++q)
      dma16s_salu(tbase + (size_t)sg * t_stride, toff[q], l + K::B_BYTES + q * 4096);
  };
  auto issue_pair = [&](int j) __attribute__((always_inline)) {
    const int slot = (j % NPB) * 2;
    issue(sg0 + 2 * j, slot);
    issue(sg0 + 2 * j + 1, slot + 1);
  };

  f32x16_t acc[NM][NN];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int ni = 0; ni < NN; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.0f;

  // One super-group of this wave's rows.  Software-pipelined one k-block
  // ahead: the B fragments of k-block k+1 are read from LDS and the basis
  // fragments of the next sub-step generated (VALU) while the MFMAs of
  // k-block k run; scheduling barriers keep that order and interleave the
  // generation with the MFMAs.
  auto compute = [&](int slot) __attribute__((always_inline)) {
    const char* base = smem + slot * K::STAGE_BYTES;
    const float* tl = reinterpret_cast<const float*>(base + K::B_BYTES);
    const E* bl = reinterpret_cast<const E*>(base);
    constexpr int SGK = G::SGK, KBG = G::KBG;
    float tv[NM][G::LANE_T];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      const int rl = (wq * NM + mi) * 32 + (lane & 31);
      const f32x4_t* src = reinterpret_cast<const f32x4_t*>(tl + rl * G::SGI);
      const int sx = fwd_t_xor<G::SGI / 4>(rl);
#pragma unroll
      for (int q = 0; q < G::LANE_T / 4; ++q) {
        const f32x4_t w = src[(g * (G::LANE_T / 4) + q) ^ sx];
        tv[mi][4 * q + 0] = w[0]; tv[mi][4 * q + 1] = w[1];
        tv[mi][4 * q + 2] = w[2]; tv[mi][4 * q + 3] = w[3];
      }
    }
    Frag<BF> bq[2][NN];
#pragma unroll
    for (int ni = 0; ni < NN; ++ni) bq[0][ni] = load_frag<BF>(bl + (ni * SGK) * kFragElems, lane);
    Frag<BF> af[2][NM][KBG];
    auto gen = [&](int s, Frag<BF> (&dst)[NM][KBG]) __attribute__((always_inline)) {
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) {
        float vals[8 * KBG];
#pragma unroll
        for (int u = 0; u < G::IPG / 2; ++u) cheb_T<P>(tv[mi][s * (G::IPG / 2) + u], vals + u * P);
#pragma unroll
        for (int h = 0; h < KBG; ++h) dst[mi][h] = make_frag<BF>(vals + 8 * h);
      }
    };
    gen(0, af[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int h = 0; h < KBG; ++h) {
        const int kbl = s * KBG + h;
        if (kbl + 1 < SGK) {
#pragma unroll
          for (int ni = 0; ni < NN; ++ni)
            bq[(kbl + 1) & 1][ni] = load_frag<BF>(bl + (ni * SGK + kbl + 1) * kFragElems, lane);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (h == KBG - 1 && s < 3) gen(s + 1, af[(s + 1) & 1]);
#pragma unroll
        for (int ni = 0; ni < NN; ++ni)
#pragma unroll
          for (int mi = 0; mi < NM; ++mi) mma(acc[mi][ni], af[s & 1][mi][h], bq[kbl & 1][ni]);
#pragma unroll
        for (int q = 0; q < NN * NM; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // then up to four VALU
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // Pair j is copied by half 0: pairs 0 .. NPB-2 before the loop, pair
  // j + NPB - 1 right after half 0's MFMAs of iteration j, while half 1's
  // MFMAs of that iteration still run (the older waves of a SIMD are issued
  // first, so half 0 reaches the end of its super-group first).  Copies
  // interleaved with the MFMAs of every wave measured slower: each copy
  // occupies the CU's address unit ~20 clk and stalls its wave meanwhile.
  pin_sgpr(y);  // used after the loop
  pin_sgpr(part);
  pin_sgpr(bias_f);
  pin_sgpr(bias_part);
  pin_sgpr(bias_out);
  pin_sgpr(nib);
  if (half == 0) {
#pragma unroll
    for (int j = 0; j < NPB - 1; ++j)
      if (j < npair) issue_pair(j);
  }
  for (int j = 0; j < npair; ++j) {
    // half 0: pair j has landed once only the copies of pairs j+1 .. j+NPB-2
    // (HOPS each) remain; only the last pair can be a single stage, so near
    // the end wait for all.  The barrier publishes the copies to half 1.
    if (half == 0) {
      if (j + NPB - 2 < npair - 1) wait_vmcnt<HOPS * (NPB - 2)>();
      else wait_vmcnt<0>();
    }
    block_barrier();
    if (sg0 + 2 * j + half < sg1) compute((j % NPB) * 2 + half);
    if (half == 0 && j + NPB - 1 < npair) issue_pair(j + NPB - 1);
  }

  // Sum the two halves' tiles through LDS (the ring is free once all waves
  // pass the barrier).  Each half keeps NN/2 column blocks: it hands the
  // other half's column blocks over, adds the ones it receives, and stores
  // its own, so all 8 waves share the stores.  Every barrier is reached by
  // all 8 waves.
  constexpr int NH = NN / 2;
  // bias from the partials: thread t sums partials k = t % 4, t % 4 + 4, ... of
  // output nb0 * 32 + t / 4 (loads issued here, ahead of the LDS hand-over);
  // the block's outputs are the first BNF * 32 of them
  float bsum = 0.0f;
  const int bo = nb0 * 32 + (tid >> 2);
  const bool bown = (tid >> 2) < BNF * 32 && bo < p.O32;
  if (nib > 0 && bown)
    for (int k = tid & 3; k < nib; k += 4) bsum += bias_part[(size_t)k * p.O32 + bo];
  wait_lgkmcnt<0>();
  block_barrier();
  float* bias_l = reinterpret_cast<float*>(smem + K::BIAS_OFF);
  if (nib > 0) {
    const int q0 = lane & ~3;
    const float s0 = __shfl(bsum, q0), s1 = __shfl(bsum, q0 + 1);
    const float s2 = __shfl(bsum, q0 + 2), s3 = __shfl(bsum, q0 + 3);
    const float tot = ((s0 + s1) + s2) + s3;
    if ((tid & 3) == 0 && (tid >> 2) < BNF * 32) {
      bias_l[tid >> 2] = tot;
      if (bias_out && bx == 0 && blockIdx.z == 0 && bown) bias_out[bo] = tot;
    }
  }
  float* red = reinterpret_cast<float*>(smem);
  auto red_at = [&](int giver, int mi, int j, int v) __attribute__((always_inline)) {
    return red + ((((giver * 4 + wq) * NM + mi) * NH + j) * 16 + v) * 64 + lane;
  };
  auto exchange = [&](auto KEEP) __attribute__((always_inline)) {
    constexpr int keep0 = decltype(KEEP)::value, give0 = NH - keep0;
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int j = 0; j < NH; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) *red_at(half, mi, j, v) = acc[mi][give0 + j][v];
    wait_lgkmcnt<0>();
    block_barrier();
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int j = 0; j < NH; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[mi][keep0 + j][v] += *red_at(half ^ 1, mi, j, v);
  };
  const bool split = gridDim.z > 1;
  const bool full_rows = m_blk + BM <= (split ? p.B32 : p.B);
  auto store = [&](auto KEEP) __attribute__((always_inline)) {
    constexpr int keep0 = decltype(KEEP)::value;
#pragma unroll
    for (int j = 0; j < NH; ++j) {
      const int nb = nb0 + keep0 + j;
      const int o = nb * 32 + (lane & 31);
      if (split ? nb >= p.NBf : o >= p.O) continue;
      const float add = split ? 0.0f : (nib > 0 ? bias_l[(keep0 + j) * 32 + (lane & 31)] : bias_f[o]);
      const int64_t pitch = split ? p.O32 : p.O;
      const int64_t nrow = split ? p.B32 : p.B;
      float* out = split ? part + (size_t)blockIdx.z * p.B32 * p.O32 : y;
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) {
        const int64_t r0 = m_blk + (wq * NM + mi) * 32 + 4 * g;
        float* op = out + r0 * pitch + o;
        if (full_rows) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            float* a = op + (8 * (v >> 2) + (v & 3)) * pitch;
            const float yv = acc[mi][keep0 + j][v] + add;
            if (split) *a = yv;
            else if constexpr (OT) *a = tanhf(yv);  // read again soon, by the next layer
            else __builtin_nontemporal_store(yv, a);
          }
        } else {
#pragma unroll
          for (int v = 0; v < 16; ++v)
            if (r0 + 8 * (v >> 2) + (v & 3) < nrow) {
              const float yv = acc[mi][keep0 + j][v] + add;
              op[(8 * (v >> 2) + (v & 3)) * pitch] = OT && !split ? tanhf(yv) : yv;
            }
        }
      }
    }
  };
  // split-K blocks write partial tiles; k_fwd_reduce adds the splits in order
  if (half == 0) {
    exchange(std::integral_constant<int, 0>{});
    store(std::integral_constant<int, 0>{});
  } else {
    exchange(std::integral_constant<int, NH>{});
    store(std::integral_constant<int, NH>{});
  }
}

// ---------------------------------------------------------------------------
// Forward, small batch (B <= 64): coefficient streaming.  The work is the
// HBM stream of Cf; the MFMAs run at a few percent of their peak.  Each wave
// takes one 32-output column block and SPW super-groups (16 k-blocks) of the
// reduction and issues all of its loads at once: the coefficient fragments
// straight into registers (one coalesced 1 KiB wave load per fragment, no
// LDS) and its rows of x.  With up to 32 rows it computes tanh itself
// (writing the tanh cache from the blocks of column block 0); with 33..64
// (TPRE) it reads the cache written by launch_tanh instead, since every
// column block needs the same values.  It builds its basis fragments, and
// accumulates NMS x 32 rows.  The 4 waves of a block reduce through LDS and
// write one partial tile; k_fwd_reduce adds the partials in order.
// ---------------------------------------------------------------------------
template <int P, bool BF> struct FwdStream {
  typedef FwdGroup<P> G;
  static constexpr int SPW = 16 / G::SGK;         // super-groups per wave
  static constexpr int KPW = SPW * G::SGK;        // k-blocks per wave (16)
  static constexpr int WAVES = 4;
};

// Waves per SIMD the streaming kernel asks the compiler to fit.  The grid
// runs 16 waves per CU; at more than 128 registers a lane only 3 fit per
// SIMD and the last quarter of the waves runs as a second round.  The bf16
// kernels of degree 8 and 16 fit 4 per SIMD without spilling; the others
// keep the default (they would spill).
template <int P, bool BF> struct StreamWaves { static constexpr int v = (BF && P >= 8) ? 4 : 1; };

template <int P, bool BF, int NMS, bool TPRE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(StreamWaves<P, BF>::v)))
k_fwd_stream(const float* __restrict__ x, float* __restrict__ tc,
             const typename Elem<BF>::type* __restrict__ Cf, float* __restrict__ part, Plan p,
             int bpn, int xal) {
  typedef FwdGroup<P> G;
  typedef FwdStream<P, BF> K;
  constexpr int SPW = K::SPW, KPW = K::KPW, LT = G::LANE_T;
  __shared__ float red[K::WAVES][NMS * 32][33];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5;
  const int nb = blockIdx.x / bpn, blk = blockIdx.x - nb * bpn;
  const int nsg = p.I_sg / G::SGI;
  const int sg0 = (blk * K::WAVES + wave) * SPW;

  // every load of this wave, in flight together: its rows of x first, so
  // that tanh and the basis (which need only x) can run while the
  // coefficient fragments are still streaming in (vector loads retire in
  // issue order, so each MFMA then waits only for its own fragment).  The
  // loads are unconditional, from clamped in-range addresses; values past B,
  // I or the last super-group are zeroed only after every load is issued (a
  // use of a loaded value between the loads made the compiler wait for it).
  float xv[NMS][SPW][LT];
  const bool xvec = xal && (p.I & 3) == 0;  // LT is a multiple of 4, so are the lane offsets
  f32x4_t xraw[NMS][SPW][LT / 4];
  if constexpr (TPRE) {
    // the tanh values come from the cache (pitch I_sg, zero past I): one
    // 16-byte load each, rows past B clamped and zeroed below
#pragma unroll
    for (int mi = 0; mi < NMS; ++mi) {
      const int r = mi * 32 + (lane & 31);
      const float* tr = tc + (size_t)(r < p.B ? r : (int)p.B - 1) * p.I_sg;
#pragma unroll
      for (int j = 0; j < SPW; ++j) {
        const int i0 = min(sg0 + j, nsg - 1) * G::SGI + g * LT;
#pragma unroll
        for (int q = 0; q < LT; q += 4) xraw[mi][j][q / 4] = *reinterpret_cast<const f32x4_t*>(tr + i0 + q);
      }
    }
  } else
#pragma unroll
  for (int mi = 0; mi < NMS; ++mi) {
    const int r = mi * 32 + (lane & 31);
    const float* xr = x + (size_t)(r < p.B ? r : (int)p.B - 1) * p.I;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int i0 = (sg0 + j) * G::SGI + g * LT;
#pragma unroll
      for (int q = 0; q < LT; q += 4) {
        if (xvec) {  // I % 4 == 0: a float4 is all in or all out
          xraw[mi][j][q / 4] = *reinterpret_cast<const f32x4_t*>(xr + (i0 + q + 4 <= p.I ? i0 + q : p.I - 4));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) xraw[mi][j][q / 4][e] = xr[min(i0 + q + e, p.I - 1)];
        }
      }
    }
  }
  Frag<BF> bfr[KPW];
#pragma unroll
  for (int q = 0; q < KPW; ++q) {
    const int sg = min(sg0 + q / G::SGK, nsg - 1);
    bfr[q] = load_frag_nt<BF>(Cf + cf_elem<BF>(p.KB, nb, sg * G::SGK + q % G::SGK, lane) - (size_t)lane * 8, lane);
  }
#pragma unroll
  for (int q = 0; q < KPW; ++q)
    if (sg0 + q / G::SGK >= nsg) bfr[q] = zero_frag<BF>();
#pragma unroll
  for (int mi = 0; mi < NMS; ++mi) {
    const int r = mi * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int i0 = (sg0 + j) * G::SGI + g * LT;
#pragma unroll
      for (int q = 0; q < LT; ++q)
        xv[mi][j][q] = (r < p.B && i0 + q < p.I) ? xraw[mi][j][q / 4][q % 4] : 0.0f;
    }
  }
  f32x16_t acc[NMS];
#pragma unroll
  for (int mi = 0; mi < NMS; ++mi)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[mi][v] = 0.0f;

#pragma unroll
  for (int mi = 0; mi < NMS; ++mi) {
    const int r = mi * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int sg = sg0 + j;
      float tv[LT];
#pragma unroll
      for (int q = 0; q < LT; ++q) tv[q] = TPRE ? xv[mi][j][q] : input_map(xv[mi][j][q], p.imap, p.ima, p.imb);
      if (!TPRE && nb == 0 && r < p.B && sg < nsg) {  // the tanh cache, written once
        f32x4_t* dst = reinterpret_cast<f32x4_t*>(tc + (size_t)r * p.I_sg + (size_t)sg * G::SGI + g * LT);
#pragma unroll
        for (int q = 0; q < LT / 4; ++q)
          dst[q] = f32x4_t{tv[4 * q], tv[4 * q + 1], tv[4 * q + 2], tv[4 * q + 3]};
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        float vals[8 * G::KBG];
#pragma unroll
        for (int u = 0; u < G::IPG / 2; ++u) cheb_T<P>(tv[s4 * (G::IPG / 2) + u], vals + u * P);
#pragma unroll
        for (int h = 0; h < G::KBG; ++h)
          mma(acc[mi], make_frag<BF>(vals + 8 * h), bfr[j * G::SGK + s4 * G::KBG + h]);
      }
    }
  }

  // reduce the 4 waves' tiles (valid rows only) and write this block's partial
#pragma unroll
  for (int mi = 0; mi < NMS; ++mi)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int r = mi * 32 + acc_row(v, g);
      if (r < p.B) red[wave][r][lane & 31] = acc[mi][v];
    }
  __syncthreads();
  const int nrow = p.B < NMS * 32 ? (int)p.B : NMS * 32;
  for (int idx = tid; idx < nrow * 32; idx += 256) {
    const int r = idx >> 5, c = idx & 31;
    part[((size_t)blk * p.B32 + r) * p.O32 + nb * 32 + c] =
        ((red[0][r][c] + red[1][r][c]) + red[2][r][c]) + red[3][r][c];
  }
}

// y[r, o] = bias[o] + sum_z part[z][r][o], z in split order.  nib > 0: the
// bias comes from its per-input-block partials (summed per element: the host
// chooses this only for small outputs) and the packed bias slot is filled.
// out_tanh: tanh(y) is stored instead (the next layer's tanh cache).
__global__ void __launch_bounds__(256)
k_fwd_reduce(const float* __restrict__ part, int S, const float* __restrict__ bias_f,
             float* __restrict__ y, Plan p, const float* __restrict__ bias_part, int nib,
             float* __restrict__ bias_out, int out_tanh) {
  const int64_t n = p.B * (int64_t)p.O;
  const int64_t nn = n > p.O32 ? n : p.O32;
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < nn;
       q += (int64_t)gridDim.x * blockDim.x) {
    if (nib > 0 && q < p.O32) bias_out[q] = bias_from_parts(bias_part, nib, p.O32, (int)q);
    if (q >= n) continue;
    const int64_t r = q / p.O;
    const int o = (int)(q - r * p.O);
    const float bias = nib > 0 ? bias_from_parts(bias_part, nib, p.O32, o) : bias_f[o];
    const float v = split_sum(part + (size_t)r * p.O32 + o, (size_t)p.B32 * p.O32, (unsigned)S, bias);
    y[q] = out_tanh ? tanhf(v) : v;
  }
}

// The end of a stack's training forward, one row per wave: layer a's split
// sum (the bits of k_fwd_reduce with out_tanh: tanh(y_a) into layer b's
// tanh cache tb, pitch a.O = b's inputs), then the last layer b on the vector
// ALU from its fp32 coefficients Cb [Ib, Ob, Db] (lane i takes input i: its
// T_d(t_i) by the three-term recurrence, times Cb[i, k, d]; the lanes'
// partials are summed per class through LDS), then the row's softmax
// cross-entropy: yb, dyb = (softmax - onehot) / B and the row's loss into
// loss_part[r], whose mean is taken in k_sum_scalar's order by the caller's
// next launch.  Ib <= 64, Ob <= kTailO; the
// block stages Cb in LDS (Ib Ob Db <= kTailC floats), its coalesced loads
// issued ahead of the split sums so that both latencies overlap.
// With dxa, lane i also writes layer b's dX for the row, dL/dy_a[r, i] =
// (1 - t_i^2) sum_e U_e(t_i) sum_k dy[k] (e + 1) Cb[i, k, e + 1] over e < Pb
// (b's padded degree), in k_dx_small's arithmetic (the same bits): the row's
// gradient dy[k] is broadcast from lane k, and the operand (e + 1) Cb is
// formed as the pack forms it.
constexpr int kTailO = 16, kTailRows = 4, kTailC = 8192, kTailCL = 16;

// Lane i's dX of the row for b's padded degree PB: c = Cb[i] staged [Ob][Db],
// dmine the row's dy of this lane's class (read from lane k for class k), t
// its input.  Reads are unconditional from in-range addresses and classes
// past Ob leave g unchanged, so g[e] takes k_dx_small's additions in its
// order.  b's input map is tanh (the tail's precondition): dt/dy_a = 1 - t^2.
template <int PB>
__device__ __forceinline__ float tail_dx(const float* c, int Ob, int Db, float dmine, float t) {
  float g[PB];
#pragma unroll
  for (int e = 0; e < PB; ++e) g[e] = 0.0f;
#pragma unroll
  for (int k = 0; k < kTailO; ++k) {
    const int kk = k < Ob ? k : 0;
    const float a = __shfl(dmine, kk);
#pragma unroll
    for (int e = 0; e < PB; ++e) {
      const float cc = c[kk * Db + (e + 1 < Db ? e + 1 : 0)];
      const float w = e + 1 < Db ? cc * (float)(e + 1) : 0.0f;  // the packed dX operand's value
      g[e] = k < Ob ? fmaf(a, w, g[e]) : g[e];
    }
  }
  const float t2 = t + t;
  float up = 0.0f, u = 1.0f, sd = 0.0f;  // U_{e-1}, U_e
#pragma unroll
  for (int e = 0; e < PB; ++e) {
    sd = fmaf(g[e], u, sd);
    const float un = fmaf(t2, u, -up);
    up = u;
    u = un;
  }
  return sd * (1.0f - t * t);
}

__global__ void __launch_bounds__(256)
k_fwd_tail_ce(const float* __restrict__ part, int S, const float* __restrict__ bias_f, Plan pa,
              const float* __restrict__ bias_part, int nib, float* __restrict__ bias_out,
              float* __restrict__ tb, const float* __restrict__ Cb, int Ob, int Db,
              float* __restrict__ yb, const int64_t* __restrict__ labels, float* __restrict__ dyb,
              float* __restrict__ loss_part, float* __restrict__ dxa, int Pb) {
  extern __shared__ float csh[];  // Cb [Ib][Ob][Db]
  __shared__ float red[kTailRows][64 * (kTailO + 1)];  // each wave's [input][class] partials
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t r = (int64_t)blockIdx.x * kTailRows + (tid >> 6);
  const bool active = r < pa.B;
  const int Ib = pa.O, nC = Ib * Ob * Db;
  float cv[kTailCL];
#pragma unroll
  for (int u = 0; u < kTailCL; ++u) {
    const int q = tid + u * 256;
    cv[u] = q < nC ? Cb[q] : 0.0f;
  }
  if (nib > 0 && blockIdx.x == 0)
    for (int q = tid; q < pa.O32; q += blockDim.x) bias_out[q] = bias_from_parts(bias_part, nib, pa.O32, q);
  float t = 0.0f;
  if (active && lane < Ib) {
    const float bias = nib > 0 ? bias_from_parts(bias_part, nib, pa.O32, lane) : bias_f[lane];
    t = tanhf(split_sum(part + (size_t)r * pa.O32 + lane, (size_t)pa.B32 * pa.O32, (unsigned)S, bias));
    tb[r * Ib + lane] = t;
  }
#pragma unroll
  for (int u = 0; u < kTailCL; ++u) {
    const int q = tid + u * 256;
    if (q < nC) csh[q] = cv[u];
  }
  for (int q0 = kTailCL * 256; q0 < nC; q0 += kTailCL * 256) {
#pragma unroll
    for (int u = 0; u < kTailCL; ++u) {
      const int q = q0 + tid + u * 256;
      cv[u] = q < nC ? Cb[q] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kTailCL; ++u) {
      const int q = q0 + tid + u * 256;
      if (q < nC) csh[q] = cv[u];
    }
  }
  __syncthreads();
  if (!active) return;
  float acc[kTailO];
#pragma unroll
  for (int k = 0; k < kTailO; ++k) acc[k] = 0.0f;
  if (lane < Ib) {
    const float* c = csh + lane * Ob * Db;
    const float t2 = t + t;
    float tm = 1.0f, tc = t;  // T_{d-1}, T_d from d = 0
    for (int d = 0; d < Db; ++d) {
      const float td = d == 0 ? 1.0f : tc;
      // reads from in-range addresses, unconditional: an LDS read under a
      // branch is waited for inside it (one round trip per read)
      float cv[kTailO];
#pragma unroll
      for (int k = 0; k < kTailO; ++k) cv[k] = c[(k < Ob ? k : 0) * Db + d];
#pragma unroll
      for (int k = 0; k < kTailO; ++k) acc[k] = k < Ob ? fmaf(cv[k], td, acc[k]) : acc[k];
      if (d > 0) {
        const float tn = fmaf(t2, tc, -tm);
        tm = tc;
        tc = tn;
      }
    }
  }
  // the sums over the 64 inputs: the lanes' class partials go through the
  // wave's LDS area (odd pitch: writes and reads hit 64 distinct banks), lane
  // (k, q) = (lane % 16, lane / 16) adds inputs 16q .. 16q + 15 of class k in
  // order, and two exchanges add the quarters, so lanes k, k + 16, k + 32 and
  // k + 48 hold y_k (a 64-lane butterfly per class was 96 dependent exchanges)
  float* rw = red[tid >> 6];
#pragma unroll
  for (int k = 0; k < kTailO; ++k) rw[lane * (kTailO + 1) + k] = acc[k];
  wait_lgkmcnt<0>();  // the wave reads other lanes' writes of its own area
  __builtin_amdgcn_wave_barrier();
  const int kc = lane & 15, qq = lane >> 4;
  float yk = 0.0f;
#pragma unroll
  for (int u = 0; u < 16; ++u) yk += rw[(qq * 16 + u) * (kTailO + 1) + kc];
  yk += __shfl_xor(yk, 16);
  yk += __shfl_xor(yk, 32);
  // the cross-entropy of row r: max and sum of the exponentials over the
  // classes by butterflies within each 16-lane row (every row the same)
  const bool valid = kc < Ob;
  float m = valid ? yk : -INFINITY;
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1) m = fmaxf(m, __shfl_xor(m, w));
  const float ek = valid ? expf(yk - m) : 0.0f;
  float sm = ek;
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1) sm += __shfl_xor(sm, w);
  const int64_t lab = labels[r];
  const float inv_b = 1.0f / (float)pa.B;
  const bool lab_ok = lab >= 0 && lab < Ob;
  const float yl = __shfl(yk, lab_ok ? (int)lab : 0);
  // lane k < 16: class k's gradient (read by the dX below from lane k)
  const float dmine = (ek / sm - (kc == lab ? 1.0f : 0.0f)) * inv_b;
  if (lane < Ob) {
    yb[r * Ob + lane] = yk;
    dyb[r * Ob + lane] = dmine;
  }
  if (lane == 0) loss_part[r] = (logf(sm) + m) - (lab_ok ? yl : 0.0f);
  if (dxa) {
    const float* c = csh + (lane < Ib ? lane : 0) * Ob * Db;
    float dx;
    switch (Pb) {
      case 2: dx = tail_dx<2>(c, Ob, Db, dmine, t); break;
      case 4: dx = tail_dx<4>(c, Ob, Db, dmine, t); break;
      case 8: dx = tail_dx<8>(c, Ob, Db, dmine, t); break;
      default: dx = tail_dx<16>(c, Ob, Db, dmine, t); break;
    }
    if (lane < Ib) __builtin_nontemporal_store(dx, dxa + r * Ib + lane);
  }
}

// ---------------------------------------------------------------------------
// Forward, very small batch (B <= 16), one launch: column-owning blocks.
// Block b owns one 8-output stream of the bf16 coefficients (cf_bf16_elem)
// and the whole reduction, so no split-K partials and no second launch; with
// 2048 outputs that is 256 blocks, one per CU.  Its 16 waves split the
// reduction into batches of 2 U k-blocks (U MFMA steps: 16, or 8 from 4
// rows), read as U / 2 contiguous 1 KiB loads: lane (c, G) = (lane % 16,
// lane / 16) of load l gets column c % 8 of half c / 8 of k-block 4 l + G.
// Each load feeds two
// v_mfma_f32_16x16x32_bf16 steps whose k-group G is that k-block: the first
// half directly (columns 0..7), the second half rotated in from lanes 8..15
// by a DPP row rotate; columns 8..15 of every step are duplicates whose sums
// are not stored.  The wave's lanes build each of the batch's R x 4U distinct
// basis vectors (row, k-group run of 8 values) once, from coalesced loads of
// x, into a per-wave LDS area, and every MFMA lane reads its vector there
// (rows past R read row R - 1; their sums are never stored).  Loads go out
// one batch ahead of the MFMAs.  The 16 waves' tiles are added in wave order
// through LDS, with the bias.
// ---------------------------------------------------------------------------
template <int P, int R>
struct FwdCols {
  typedef FwdGroup<P> G;
  static constexpr int WAVES = 16;
  static constexpr int NU = P <= 8 ? 8 / P : 1;        // inputs per basis vector
  // MFMA steps per batch (measured at config 5: 16 best for 1 row, 8 for 4)
  static constexpr int U = R >= 4 ? 8 : 16;
  static constexpr int NL = U / 2;                     // 1 KiB loads per batch
  static constexpr int KBB = 4 * NL;                   // k-blocks per batch (4 per load)
  static constexpr int SGB = KBB / G::SGK;             // super-groups per batch
  static constexpr int VPR = 4 * U;                    // vectors per row per batch
  static constexpr int NV = R * VPR;                   // vectors per batch
  static constexpr int PASSES = (NV + 63) / 64;
  // LDS slots of a wave: vector (step j, k-group gg, row r) at (4 j + gg) RP + r.
  // The vector-building lanes of one row write 4U different (j, gg) at once;
  // an odd pitch spreads them over the banks (pitch R >= 4: 16-byte slots a
  // multiple of 64 bytes apart, 16 lanes on one bank group).
  static constexpr int RP = R >= 4 ? R + 1 : R;
  static constexpr int SLOTS = 4 * U * RP;
  // Above kColsTanhRows rows the tanh values come from the tanh cache
  // (written by launch_tanh): tanh per vector makes the kernel
  // vector-ALU-bound at 16 rows.
  static constexpr bool TPRE = R > kColsTanhRows;
};

__device__ __forceinline__ void mma16(f32x4_t& acc, const bf16x8_t& a, const bf16x8_t& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}

// v rotated by 8 lanes within each row of 16 (lane c takes lane (c + 8) % 16).
__device__ __forceinline__ bf16x8_t row_rotate8(const bf16x8_t& v) {
  const u32x4_t u = __builtin_bit_cast(u32x4_t, v);
  u32x4_t r;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    r[e] = (unsigned)__builtin_amdgcn_update_dpp(0, (int)u[e], 0x128, 0xF, 0xF, false);  // row_ror:8
  return __builtin_bit_cast(bf16x8_t, r);
}

template <int P, int R>
__global__ void __launch_bounds__(1024)
k_fwd_cols(const float* __restrict__ x, float* __restrict__ tc, const uint16_t* __restrict__ Cf,
           const float* __restrict__ bias_f, float* __restrict__ y, Plan p,
           const float* __restrict__ bias_part, int nib, float* __restrict__ bias_out) {
  typedef FwdCols<P, R> K;
  typedef FwdGroup<P> G;
  constexpr int U = K::U, NL = K::NL, NU = K::NU, SGK = G::SGK, PASSES = K::PASSES;
  static_assert(K::KBB % SGK == 0, "a batch holds whole super-groups");
  __shared__ bf16x8_t vec[K::WAVES][K::SLOTS];
  __shared__ float red[K::WAVES][16][8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 15, G4 = lane >> 4;
  // Blocks go to the 8 XCDs round-robin (block b on XCD b % 8).  With the
  // number of 32-output blocks a multiple of 8, the 4 streams of one 32-output
  // block get the same XCD and neighbouring dispatch slots; otherwise blocks
  // take streams in order.
  int nb, sub;
  if ((p.NBf & 7) == 0) {
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    sub = slot & 3;
    nb = (slot >> 2) * 8 + xcd;
  } else {
    nb = blockIdx.x >> 2;
    sub = blockIdx.x & 3;
  }
  const int nsg = p.I_sg / G::SGI;
  const int nbat = (nsg + K::SGB - 1) / K::SGB;           // batches of the whole reduction
  const int bpw = (nbat + K::WAVES - 1) / K::WAVES;        // batches per wave
  const int b0 = wave * bpw;
  const int nb_w = max(0, min(b0 + bpw, nbat) - b0);       // this wave's batches
  const int rl = c < R ? c : R - 1;                        // row whose vector this lane reads
  const bool writes_t = nb == 0 && sub == 0;
  // this block's stream; load l of batch bb covers its k-blocks bb KBB + 4 l .. + 3
  const uint16_t* stream = Cf + cf_bf16_elem(p.KB, nb, 0, sub * 8) + (size_t)lane * 8;
  const int kbmax = p.KB - 4;                              // last whole load (KB % 4 == 0)

  // vector-building lane, pass q: vector v = lane + 64 q -> (row, k) with k
  // ordered by input, so the x loads of consecutive lanes are contiguous
  struct VecJob { int r, sgl, j, gg, off; bool on; };
  auto vjob = [&](int q) {
    VecJob jb;
    const int v = lane + 64 * q;
    jb.on = v < K::NV;
    const int vv = jb.on ? v : 0;
    jb.r = vv / K::VPR;
    const int k = vv - jb.r * K::VPR;
    jb.sgl = k / (2 * SGK);                 // super-group within the batch
    const int e = k - jb.sgl * 2 * SGK;
    int g, sidx, h;
    if constexpr (P <= 8) { g = e / 4; sidx = e % 4; h = 0; }
    else { g = e / 8; sidx = (e % 8) / 2; h = e % 2; }
    const int kbl = jb.sgl * SGK + sidx * G::KBG + h;  // k-block within the batch
    jb.j = 2 * (kbl >> 2) + g;                         // MFMA step: load kbl / 4, half g
    jb.gg = kbl & 3;                                   // its k-group
    jb.off = g * 2 * G::IPG + sidx * (G::IPG / 2);     // first input within the super-group
    return jb;
  };

  bf16x8_t fb[2][NL];
  float xv[2][PASSES][NU];
  auto load = [&](int buf, int bt) {
    const int bb = min(b0 + bt, nbat - 1);
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const VecJob jb = vjob(q);
      const int64_t r = jb.r < p.B ? jb.r : p.B - 1;
      const int i0 = (bb * K::SGB + jb.sgl) * G::SGI + jb.off;
#pragma unroll
      for (int u = 0; u < NU; ++u)
        xv[buf][q][u] = K::TPRE ? tc[r * p.I_sg + min(i0 + u, p.I_sg - 1)]
                                : x[r * p.I + min(i0 + u, p.I - 1)];
    }
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      const int kb = min(bb * K::KBB + 4 * l, kbmax);
      fb[buf][l] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8_t*>(stream + (size_t)kb * 128));
    }
  };

  f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int buf, int bt) {
    const bool live = bt < nb_w;
    const int bb = min(b0 + bt, nbat - 1);
    // this batch's basis vectors into the wave's LDS area
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const VecJob jb = vjob(q);
      const int sg = bb * K::SGB + jb.sgl;
      const int i0 = sg * G::SGI + jb.off;
      float tv[NU];
#pragma unroll
      for (int u = 0; u < NU; ++u)
        tv[u] = (sg < nsg && i0 + u < p.I)
            ? (K::TPRE ? xv[buf][q][u] : input_map(xv[buf][q][u], p.imap, p.ima, p.imb))
            : 0.0f;
      if (!K::TPRE && writes_t && live && jb.on && jb.r < p.B && sg < nsg) {
        if constexpr (P <= 8) {
#pragma unroll
          for (int u = 0; u < NU; ++u) tc[(int64_t)jb.r * p.I_sg + i0 + u] = tv[u];
        } else if ((jb.gg & 1) == 0) {  // degree-16 vectors come in degree-half pairs
          tc[(int64_t)jb.r * p.I_sg + i0] = tv[0];
        }
      }
      float vals[8 * G::KBG];
      if constexpr (P <= 8) {
#pragma unroll
        for (int u = 0; u < NU; ++u) cheb_T<P>(tv[u], vals + u * P);
      } else {
        cheb_T<P>(tv[0], vals);
        if (jb.gg & 1) {
#pragma unroll
          for (int e = 0; e < 8; ++e) vals[e] = vals[8 + e];
        }
      }
      // batches past the wave's range, and super-groups past the last, add nothing
      const bf16x8_t a = (live && sg < nsg) ? make_frag_bf(vals).v : bf16x8_t{};
      if (jb.on) vec[wave][(4 * jb.j + jb.gg) * K::RP + jb.r] = a;
    }
    // the wave reads other lanes' writes of its own area: wait for them to
    // complete (without the wait, reads have returned stale vectors on
    // gfx950) and keep the compiler from moving accesses across
    wait_lgkmcnt<0>();
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      mma16(acc, vec[wave][(4 * (2 * l) + G4) * K::RP + rl], fb[buf][l]);
      mma16(acc, vec[wave][(4 * (2 * l + 1) + G4) * K::RP + rl], row_rotate8(fb[buf][l]));
    }
  };

  // two register buffers, each batch loaded one batch ahead of its MFMAs.
  // Inside the loop every load is unconditional, so the wait before each use
  // counts only the loads issued after it; the last one or two batches are
  // peeled, so no wave loads past its range.
  int bt = 0;
  if (nb_w > 0) load(0, 0);
  for (; bt + 2 < nb_w; bt += 2) {
    load(1, bt + 1);
    compute(0, bt);
    load(0, bt + 2);
    compute(1, bt + 1);
  }
  if (bt + 1 < nb_w) {
    load(1, bt + 1);
    compute(0, bt);
    compute(1, bt + 1);
  } else if (bt < nb_w) {
    compute(0, bt);
  }

  // the 16 waves' tiles (rows 0..15, columns 0..7), added in wave order with the bias
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (c < 8) red[wave][G4 * 4 + e][c] = acc[e];
  __syncthreads();
  // nib > 0: the bias from its per-input-block partials; the block fills its
  // 8 entries of the packed bias slot
  if (nib > 0 && tid < 8)
    bias_out[nb * 32 + sub * 8 + tid] = bias_from_parts(bias_part, nib, p.O32, nb * 32 + sub * 8 + tid);
  for (int idx = tid; idx < R * 8; idx += 1024) {
    const int r = idx >> 3, cc = idx & 7;
    const int o = nb * 32 + sub * 8 + cc;
    if (r < p.B && o < p.O) {
      float sum = nib > 0 ? bias_from_parts(bias_part, nib, p.O32, o) : bias_f[o];
#pragma unroll
      for (int w = 0; w < K::WAVES; ++w) sum += red[w][r][cc];
      y[(size_t)r * p.O + o] = sum;
    }
  }
}

// ---------------------------------------------------------------------------
// dX, pipelined.  A block's tile is 256 rows (4 waves x NM fragments) x one
// input block (32 inputs x P degrees).  Both operands (dy fragments for the
// wave's rows, coefficient fragments for the input block) are copied
// global -> LDS by global_load_lds_dwordx4 into a ring of NBUF stages of KI
// k-blocks (16 outputs each), NBUF-1 stages ahead; each wave reads the next
// k-block's fragments into registers while its MFMAs run on the current one.
// The epilogue sums over degrees with d U_{d-1}(t) and the tanh chain factor
// in registers.
// ---------------------------------------------------------------------------
template <int P, bool BF>
struct DxPipe {
  typedef typename Elem<BF>::type E;
  static constexpr int NM = BwdTile<P>::NM, WGM = 4, KI = 2;  // KI even (loop unroll)
  static constexpr int FB = kFragElems * (int)sizeof(E);  // bytes per fragment
  static constexpr int A_BYTES = WGM * NM * KI * FB;
  static constexpr int B_BYTES = P * KI * FB;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int NBUF_FIT = (160 * 1024) / STAGE_BYTES;
  static constexpr int NBUF = NBUF_FIT > 5 ? 5 : NBUF_FIT;
  static constexpr int OPS = STAGE_BYTES / 4096;  // dma16 per thread per stage
  static constexpr int A_OPS = A_BYTES / 4096;
  static constexpr bool kOk = NBUF >= 3 && STAGE_BYTES % 4096 == 0 && A_BYTES % 4096 == 0 &&
                              OPS * (NBUF - 2) < 64;
};

template <int P, bool BF>
__global__ void __launch_bounds__(256)
k_dx_pipe(const typename Elem<BF>::type* __restrict__ dYx,
          const typename Elem<BF>::type* __restrict__ Cb, const float* __restrict__ tc,
          float* __restrict__ dx, Plan p, int n_rb) {
  typedef DxPipe<P, BF> K;
  typedef typename K::E E;
  constexpr int NM = K::NM, WGM = K::WGM, KI = K::KI, FB = K::FB, NBUF = K::NBUF;
  constexpr int RUN = KI * FB / 16;  // 16-byte chunks per contiguous fragment run
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5;
  const int nst = p.KBx / KI;
  const int rb = blockIdx.x % n_rb, ib = blockIdx.x / n_rb;

  // per-op source offsets (bytes); dYx rows are padded to whole tiles
  const char* abase = reinterpret_cast<const char*>(dYx) + (size_t)rb * WGM * NM * p.KBx * FB;
  const char* bbase = reinterpret_cast<const char*>(Cb) + (size_t)ib * P * p.KBx * FB;
  uint32_t off[K::OPS];
#pragma unroll
  for (int q = 0; q < K::OPS; ++q) {
    const int c = (q * 4 + wave) * 64 + lane;
    if (q < K::A_OPS) {
      const int run = c / RUN, w = c - run * RUN;  // run = wave' * NM + mi
      off[q] = (uint32_t)(run * p.KBx * FB + w * 16);
    } else {
      const int cc = c - K::A_OPS * 256;
      const int e = cc / RUN, w = cc - e * RUN;
      off[q] = (uint32_t)(e * p.KBx * FB + w * 16);
    }
  }
  auto issue = [&](int st) __attribute__((always_inline)) {
    if (st >= nst) return;
    const size_t sb = (size_t)st * KI * FB;
    char* dst = smem + (st % NBUF) * K::STAGE_BYTES + wave * 1024;
#pragma unroll
    for (int q = 0; q < K::OPS; ++q)
      dma16((q < K::A_OPS ? abase : bbase) + sb + off[q], dst + q * 4096);
  };

  struct Regs {
    Frag<BF> a[NM];
    Frag<BF> b[P];
  };
  auto lds_read = [&](int kb, Regs& R) __attribute__((always_inline)) {
    const int kk = kb % KI;
    const char* base = smem + ((kb / KI) % NBUF) * K::STAGE_BYTES;
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
      R.a[mi] = load_frag<BF>(reinterpret_cast<const E*>(base + ((wave * NM + mi) * KI + kk) * FB), lane);
#pragma unroll
    for (int e = 0; e < P; ++e)
      R.b[e] = load_frag<BF>(reinterpret_cast<const E*>(base + K::A_BYTES + (e * KI + kk) * FB), lane);
  };

  f32x16_t acc[NM][P];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int e = 0; e < P; ++e)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][e][v] = 0.0f;

#pragma unroll
  for (int q = 0; q < NBUF - 1; ++q) issue(q);
  if (NBUF - 2 <= nst - 1) wait_vmcnt<K::OPS * (NBUF - 2)>();
  else wait_vmcnt<0>();
  block_barrier();
  // the transition into stage st refills with st + NBUF - 1; stage 0 has no
  // transition, so its refill (stage NBUF - 1) is issued here
  issue(NBUF - 1);
  Regs R0, R1;
  lds_read(0, R0);

  const int nkb = nst * KI;
  auto step = [&](int kb, const Regs& Rc, Regs& Rn) __attribute__((always_inline)) {
    const int nxt = kb + 1;
    if (nxt < nkb) {
      if (nxt % KI == 0) {
        const int st = nxt / KI;
        wait_lgkmcnt<0>();  // this wave's reads of the slot being refilled are done
        if (st + NBUF - 2 <= nst - 1) wait_vmcnt<K::OPS * (NBUF - 2)>();
        else wait_vmcnt<0>();
        block_barrier();
        issue(st + NBUF - 1);
      }
      lds_read(nxt, Rn);
    }
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int e = 0; e < P; ++e) mma(acc[mi][e], Rc.a[mi], Rc.b[e]);
  };
  for (int kb = 0; kb < nkb; kb += 2) {
    step(kb, R0, R1);
    step(kb + 1, R1, R0);
  }

  const int i = ib * 32 + (lane & 31);
  const bool icol = i < p.I;
#pragma unroll
  for (int mi = 0; mi < NM; ++mi) {
    const int64_t r0 = ((int64_t)rb * WGM * NM + wave * NM + mi) * 32 + 4 * g;
    float tv[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t r = r0 + 8 * (v >> 2) + (v & 3);
      tv[v] = (icol && r < p.B) ? tc[r * p.I_sg + i] : 0.0f;
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t r = r0 + 8 * (v >> 2) + (v & 3);
      const float t2 = tv[v] + tv[v];
      float up = 0.0f, u = 1.0f, sum = 0.0f;  // U_{-1}, U_0
#pragma unroll
      for (int e = 0; e < P; ++e) {
        sum = fmaf(acc[mi][e][v], u, sum);
        const float un = fmaf(t2, u, -up);
        up = u;
        u = un;
      }
      if (icol && r < p.B) __builtin_nontemporal_store(sum * input_slope(tv[v], p), dx + r * p.I + i);
    }
  }
}

// ---------------------------------------------------------------------------
// dX for degrees up to 8 (and fp32 at degree 16, with NM = 1: 128-row
// blocks; bf16 at degree 16 takes k_dx16 below).  One block = 2*RG waves
// (dh, rg): wave rg takes NM = 2 fragments of 32 rows, wave dh half of the P
// degrees, for one input block (32 inputs); acc = NM x P/2 fragments, two
// waves per SIMD.  RG = 4
// (256 rows per block, one block per CU) streams a third less operand data
// per MFMA than RG = 2 (two 128-row blocks per CU, whose epilogues overlap
// each other's MFMAs) and measures faster.  Both operands (dy rows and the
// degree-scaled coefficients) arrive by LDS DMA in a ring of NBUF stages of
// KI k-blocks.  Epilogue: each wave sums its degrees with U_{d-1}(t), the dh
// pair exchanges halves through LDS, and each wave stores one fragment row of
// dx = (1 - t^2) sum_d d C U_{d-1}(t) dy.
// ---------------------------------------------------------------------------
template <int P, bool BF>
struct DxDh {
  typedef typename Elem<BF>::type E;
  static constexpr int RG = 4;  // row groups: 2 * RG waves
  static constexpr int NM = P == 16 ? 1 : 2, PH = P / 2, THR = 2 * RG * 64;
  static constexpr int FB = kFragElems * (int)sizeof(E);
  static constexpr int KI = BF ? 2 : 1;
  static constexpr int A_BYTES = RG * NM * KI * FB;
  static constexpr int B_BYTES = P * KI * FB;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int NBUF = 3;
  static constexpr int LDS_BYTES = NBUF * STAGE_BYTES;
  static constexpr int OPS = STAGE_BYTES / (THR * 16);  // dma16 per thread per stage
  static constexpr int A_OPS = A_BYTES / (THR * 16);
  static constexpr bool kOk = P >= 2 && LDS_BYTES <= 160 * 1024 &&
                              A_BYTES % (THR * 16) == 0 && B_BYTES % (THR * 16) == 0 &&
                              2 * RG * 16 * 64 * 4 <= LDS_BYTES;
};

template <int P, bool BF>
__global__ void __launch_bounds__(512)
k_dx_dh(const typename Elem<BF>::type* __restrict__ dYx,
         const typename Elem<BF>::type* __restrict__ Cb, const float* __restrict__ tc,
         float* __restrict__ dx, Plan p, int n_rb) {
  typedef DxDh<P, BF> K;
  typedef typename K::E E;
  constexpr int NM = K::NM, PH = K::PH, KI = K::KI, FB = K::FB, NBUF = K::NBUF, OPS = K::OPS;
  constexpr int RUN = KI * FB / 16;  // 16-byte chunks per fragment run of a stage
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int dh = wave & 1, rg = wave >> 1;
  const int g = lane >> 5;
  const int nst = p.KBx / KI;
  const int rb = blockIdx.x % n_rb, ib = blockIdx.x / n_rb;

  // DMA: the copies of a stage are HOPS per thread of one 256-thread half,
  // chunk c = q*256 + (tid & 255) landing at byte 16*c of the stage (dy rows
  // first, then the coefficient fragments).  Waves 0-3 issue q < H0, waves
  // 4-7 the rest (see the loop for when).  Sources: a wave-uniform base (block
  // operand + stage) and a per-lane 32-bit offset; dYx rows are padded to
  // whole row blocks.
  constexpr int RG = K::RG, THR = K::THR;
  static_assert(THR == 512, "launch bounds");
  constexpr int HOPS = 2 * OPS, HA_OPS = 2 * K::A_OPS;
  constexpr int H0 = HOPS / 2, H1 = HOPS - H0;  // copies per thread of waves 0-3 / 4-7
  const char* abase = reinterpret_cast<const char*>(dYx) + (size_t)rb * RG * NM * p.KBx * FB;
  const char* bbase = reinterpret_cast<const char*>(Cb) + (size_t)ib * P * p.KBx * FB;
  const int hw = __builtin_amdgcn_readfirstlane(wave) >> 2;  // 0: waves 0-3, 1: waves 4-7
  const int q0 = hw ? H0 : 0, nq = hw ? H1 : H0;
  uint32_t off[H1];
#pragma unroll
  for (int qi = 0; qi < H1; ++qi) {
    const int q = q0 + qi;
    const int c = q * 256 + (tid & 255);
    if (q < HA_OPS) {
      const int run = c / RUN, w = c - run * RUN;
      off[qi] = (uint32_t)((size_t)run * p.KBx * FB + w * 16);
    } else {
      const int cc = c - HA_OPS * 256;
      const int e = cc / RUN, w = cc - e * RUN;
      off[qi] = (uint32_t)((size_t)e * p.KBx * FB + w * 16);
    }
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem + (uint32_t)__builtin_amdgcn_readfirstlane(wave & 3) * 1024;
  auto issue = [&](int st) __attribute__((always_inline)) {
    if (st >= nst) st = nst - 1;  // past the end: in-range data, never read
    const size_t sb = (size_t)st * KI * FB;
    const uint32_t l = lds0 + (st % NBUF) * K::STAGE_BYTES;
#pragma unroll
    for (int qi = 0; qi < H1; ++qi)
      if (qi < nq)
        dma16s_salu((q0 + qi < HA_OPS ? abase : bbase) + sb, off[qi], l + (q0 + qi) * 4096);
  };

  // epilogue tanh values, loaded up front (they complete long before use)
  const int i = ib * 32 + (lane & 31);
  const bool icol = i < p.I;
  float tt[NM][16];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi) {
    const int64_t r0 = ((int64_t)rb * RG * NM + rg * NM + mi) * 32 + 4 * g;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t r = r0 + 8 * (v >> 2) + (v & 3);
      tt[mi][v] = (icol && r < p.B) ? tc[r * p.I_sg + i] : 0.0f;
    }
  }

  f32x16_t acc[NM][PH];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int e = 0; e < PH; ++e)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][e][v] = 0.0f;

  // The copies of stage st + NBUF - 1 are split between the two waves of each
  // SIMD and issued apart in time: waves 4-7 (the younger wave of a SIMD,
  // issued second) right after their fragment reads of stage st, while waves
  // 0-3 run their MFMAs; waves 0-3 after their MFMAs, while waves 4-7 still run
  // theirs.  A copy stalls its wave while the CU's address unit takes it, so
  // neither wave carries all of a stage's copies.  The slot was last read in
  // stage st - 1, whose reads every wave completed before this stage's
  // barrier.  Each wave waits only for its own copies (vmcnt).
  pin_sgpr(dx);  // used after the loop
#pragma unroll
  for (int q = 0; q < NBUF - 1; ++q) issue(q);
  for (int st = 0; st < nst; ++st) {
    // stage st landed (this wave's copies of st+1 may be in flight)
    if (hw) wait_vmcnt<H1 * (NBUF - 2)>();
    else wait_vmcnt<H0 * (NBUF - 2)>();
    block_barrier();
    const char* base = smem + (st % NBUF) * K::STAGE_BYTES;
    // all reads first, in k-block order; the MFMAs of k-block kk wait only for
    // its own reads (LDS returns in order)
    Frag<BF> fa[KI][NM], fb[KI][PH];
#pragma unroll
    for (int kk = 0; kk < KI; ++kk) {
#pragma unroll
      for (int mi = 0; mi < NM; ++mi)
        fa[kk][mi] = load_frag<BF>(reinterpret_cast<const E*>(base + ((rg * NM + mi) * KI + kk) * FB), lane);
#pragma unroll
      for (int e = 0; e < PH; ++e)
        fb[kk][e] = load_frag<BF>(reinterpret_cast<const E*>(base + K::A_BYTES + ((dh * PH + e) * KI + kk) * FB), lane);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (hw) issue(st + NBUF - 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < KI; ++kk) {
#pragma unroll
      for (int mi = 0; mi < NM; ++mi)
#pragma unroll
        for (int e = 0; e < PH; ++e) mma(acc[mi][e], fa[kk][mi], fb[kk][e]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!hw) issue(st + NBUF - 1);
  }
  wait_vmcnt<0>();
  wait_lgkmcnt<0>();
  block_barrier();  // the ring is free

  // partial sums over this wave's degrees d = dh*PH + e + 1 (weights U_{d-1})
  float part[NM][16];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float t2 = tt[mi][v] + tt[mi][v];
      float up = 0.0f, u = 1.0f;  // U_{-1}, U_0; advanced to U_{dh*PH}
#pragma unroll
      for (int k = 0; k < PH; ++k) {
        const float un = fmaf(t2, u, -up);
        up = dh ? u : up;
        u = dh ? un : u;
      }
      float sum = 0.0f;
#pragma unroll
      for (int e = 0; e < PH; ++e) {
        sum = fmaf(acc[mi][e][v], u, sum);
        const float un = fmaf(t2, u, -up);
        up = u;
        u = un;
      }
      part[mi][v] = sum;
    }
  // with NM = 2 wave (dh, rg) keeps fragment row mi = dh and hands mi = 1 - dh
  // to its pair; with NM = 1 the dh = 1 wave hands its sums to the dh = 0 wave
  float* xch = reinterpret_cast<float*>(smem);
  auto finish = [&](auto DH) __attribute__((always_inline)) {
    constexpr int d = decltype(DH)::value;
    constexpr int keep = NM == 2 ? d : 0, give = NM == 2 ? 1 - d : 0;
    if (NM == 2 || d == 1) {
#pragma unroll
      for (int v = 0; v < 16; ++v) xch[((rg * 2 + d) * 16 + v) * 64 + lane] = part[give][v];
    }
    wait_lgkmcnt<0>();
    block_barrier();
    if (NM == 1 && d == 1) return;  // no barrier follows
    const int64_t r0 = ((int64_t)rb * RG * NM + rg * NM + keep) * 32 + 4 * g;
    float res[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float other = xch[((rg * 2 + (d ^ 1)) * 16 + v) * 64 + lane];
      const float t = tt[keep][v];
      // fixed order: the lower degrees' half first
      const float sum = d ? other + part[keep][v] : part[keep][v] + other;
      res[v] = sum * input_slope(t, p);
    }
    float* dp = dx + r0 * p.I + i;
    if (icol && r0 - 4 * g + 32 <= p.B) {
#pragma unroll
      for (int v = 0; v < 16; ++v) __builtin_nontemporal_store(res[v], dp + (int64_t)(8 * (v >> 2) + (v & 3)) * p.I);
    } else if (icol) {
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (r0 + 8 * (v >> 2) + (v & 3) < p.B) dp[(int64_t)(8 * (v >> 2) + (v & 3)) * p.I] = res[v];
    }
  };
  if (dh) finish(std::integral_constant<int, 1>{});
  else finish(std::integral_constant<int, 0>{});
}

// ---------------------------------------------------------------------------
// dX, bf16, degrees 3..8, persistent, with copy waves.  The tiles, MFMAs and
// accumulation order of k_dx_dh: waves 0-7 only read fragments and run
// MFMAs (wave (rg, dh) = (wave / 2, wave % 2): fragment rows 2 rg, 2 rg + 1,
// degrees dh PH .. + PH - 1) and waves 8-11 (one per SIMD) only issue the
// global -> LDS copies.  12 waves make three per SIMD, so every wave fits 168
// registers: the MFMA waves hold one k-block's fragments at a time and read
// the tile's tanh values from LDS in the epilogue.
//
// Persistent: block b walks tiles b, b + G, ... (tile = (row block rb, input
// block ib), rb fastest) as one stream of stages of KI = 2 k-blocks; the
// copies run three stages ahead in a ring of four.  Barrier B_s starts stage
// s; before it the copy waves have waited for stage s + 1 and every MFMA wave
// has finished reading stage s - 1, so after it the copy waves fill slot
// (s + 3) % 4 = (s - 1) % 4, and an MFMA wave reads the first k-block of
// stage s + 1 before B_{s+1}, overlapping the barrier.  A tile's epilogue:
// its tanh values (copied into a 32 KiB buffer after the previous tile's
// epilogue) are read and each wave's degree sums formed and scaled by their
// rows' input slope; the next stage barrier frees the buffer, which then
// carries the dh pairs' exchange (one more barrier, X).  The next tile's tanh
// copies follow the barrier after that.  A tile needs at least 4 stages
// (tanh copies waited two stages after their issue, before the tile's last).
//
// Measured at config 3 (cuts of a scratch copy): the MFMA loop alone takes
// 84 us of the kernel's ~115; the copies and fragment reads ~18 us; the
// epilogue ~14 us when it held the kept row's tanh values across the
// exchange (register spills whose reloads waited behind the tile's stores),
// about half that with the sums scaled before the exchange.  A 16x16x32
// version whose waves own every degree (no exchange) ran its MFMA loop 27 %
// slower, and one with the copies issued between the MFMA waves' MFMAs ran
// 20 % slower than k_dx_dh.
// ---------------------------------------------------------------------------
template <int P>
struct DxWs {
  static constexpr int PH = P / 2, KI = 2, FB = 1024;
  static constexpr int NMW = 8, NDW = 4, THR = (NMW + NDW) * 64;
  static constexpr int A_FR = 8 * KI, B_FR = P * KI, STAGE_FR = A_FR + B_FR;
  static constexpr int STAGE_BYTES = STAGE_FR * FB;
  static constexpr int CPW = STAGE_FR / NDW;   // stage copies per copy wave
  static constexpr int NBUF = 4;
  static constexpr int RING = NBUF * STAGE_BYTES;
  static constexpr int TBUF = 256 * 32 * 4;    // tanh tile [256 rows][32 inputs] fp32
  static constexpr int TCPW = TBUF / FB / NDW;  // tanh copies per copy wave
  static constexpr int XCH = NMW * 16 * 64 * 4;  // the dh pairs' exchange (in the tanh buffer)
  static constexpr int LDS_BYTES = RING + TBUF;
  static constexpr int MIN_STAGES = 4;
  static constexpr bool kOk = (P == 4 || P == 8) && STAGE_FR % NDW == 0 && XCH <= TBUF &&
                              CPW + TCPW < 64 && LDS_BYTES <= 160 * 1024;
};

template <int P>
__global__ void __launch_bounds__(768)
k_dx_ws(const uint16_t* __restrict__ dYx, const uint16_t* __restrict__ Cb,
        const float* __restrict__ tc, float* __restrict__ dx, Plan p, int n_rb, int ntiles) {
  typedef DxWs<P> K;
  constexpr int PH = K::PH, KI = K::KI, FB = K::FB, NBUF = K::NBUF, CPW = K::CPW, TCPW = K::TCPW;
  static_assert(K::kOk, "shape");
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nst = p.KBx / KI;  // stages per tile (>= MIN_STAGES, checked on the host)
  const int G = gridDim.x;
  const int mine = (ntiles - (int)blockIdx.x + G - 1) / G;  // tiles of this block (>= 1)
  const int total = mine * nst;
  float* tbuf = reinterpret_cast<float*>(smem + K::RING);

  if (wave >= K::NMW) {
    // ---- copy waves ----
    const int dw = wave - K::NMW;
    const uint32_t ring = (uint32_t)(uintptr_t)smem, tb = ring + K::RING;
    const uint32_t voff = (uint32_t)lane * 16;
    const char* const a0 = reinterpret_cast<const char*>(dYx);
    const char* const b0 = reinterpret_cast<const char*>(Cb);
    const size_t run = (size_t)p.KBx * FB;  // one fragment row / degree, all k-blocks
    // stage cursor of the next issue: tile ik, stage ist (clamped at the end)
    int ik = 0, ist = 0, islot = 0;
    auto issue = [&]() __attribute__((always_inline)) {
      const int tix = (int)blockIdx.x + (ik < mine ? ik : mine - 1) * G;
      const int st = ik < mine ? ist : nst - 1;  // past the end: in-range data, never read
      const int rb = tix % n_rb, ib = tix / n_rb;
      const char* a = a0 + (size_t)rb * 8 * run + (size_t)st * KI * FB;
      const char* b = b0 + (size_t)ib * P * run + (size_t)st * KI * FB;
      const uint32_t l = ring + (uint32_t)islot * K::STAGE_BYTES;
#pragma unroll
      for (int q = 0; q < CPW; ++q) {
        const int f = dw * CPW + q;  // wave-uniform
        const char* src = f < K::A_FR ? a + (size_t)(f / KI) * run + (f % KI) * FB
                                      : b + (size_t)((f - K::A_FR) / KI) * run + ((f - K::A_FR) % KI) * FB;
        dma16s(src, voff, l + (uint32_t)f * FB);
      }
      if (++ist == nst) { ist = 0; ++ik; }
      islot = islot == NBUF - 1 ? 0 : islot + 1;
    };
    // the tanh values of tile k: copy (dw, j) = tile rows 8 (dw TCPW + j) ..
    // + 7, lane -> row lane / 8, 16-byte chunk lane % 8 (32 inputs per row)
    auto issue_t = [&](int k) __attribute__((always_inline)) {
      const int tix = (int)blockIdx.x + k * G;
      const int rb = tix % n_rb, ib = tix / n_rb;
      const int ch = ib * 32 + 4 * (lane & 7) < p.I_sg ? 4 * (lane & 7) : 0;  // past the pitch: unused
#pragma unroll
      for (int j = 0; j < TCPW; ++j) {
        const int64_t r = (int64_t)rb * 256 + 8 * (dw * TCPW + j) + (lane >> 3);
        const int64_t rr = r < p.B ? r : p.B - 1;  // rows past B: unused
        dma16s(tc, (uint32_t)((rr * p.I_sg + ib * 32 + ch) * 4), tb + (uint32_t)(dw * TCPW + j) * FB);
      }
    };
    issue_t(0);
    issue();
    issue();
    issue();
    wait_vmcnt<2 * CPW>();  // tanh tile 0 and stage 0
    block_barrier();        // P
    wait_vmcnt<CPW>();      // stage 1
    block_barrier();        // B_0
    int st = 0, k = 0;      // the stage just started
    for (int s = 0; s < total; ++s) {
      // the next tile's tanh values, after the barrier that follows its
      // predecessor's exchange (B_{S+1}, S = the tile's first stage)
      const bool tcopy = st == 1 && k > 0;
      if (tcopy) issue_t(k);
      issue();  // stage s + 3
      if (tcopy) wait_vmcnt<CPW + TCPW>();  // stage s + 2
      else wait_vmcnt<CPW>();
      block_barrier();  // B_{s+1}
      if (++st == nst) {
        st = 0;
        ++k;
        block_barrier();  // X: the exchange of tile k - 1
      }
    }
    wait_vmcnt<0>();
    return;
  }

  // ---- MFMA waves ----
  const int dh = wave & 1, rg = wave >> 1, g = lane >> 5;
  const char* const ring = smem;
  auto read = [&](int slot, int kk, Frag<true>* fa, Frag<true>* fb) __attribute__((always_inline)) {
    const char* base = ring + slot * K::STAGE_BYTES;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
      fa[mi] = load_frag<true>(reinterpret_cast<const uint16_t*>(base + ((rg * 2 + mi) * KI + kk) * FB), lane);
#pragma unroll
    for (int e = 0; e < PH; ++e)
      fb[e] = load_frag<true>(reinterpret_cast<const uint16_t*>(base + (K::A_FR + (dh * PH + e) * KI + kk) * FB), lane);
  };

  f32x16_t acc[2][PH];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int e = 0; e < PH; ++e)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][e][v] = 0.0f;

  pin_sgpr(dx);
  Frag<true> fa[2], fb[PH];
  block_barrier();  // P: stage 0 landed
  read(0, 0, fa, fb);
  block_barrier();  // B_0
  int slot = 0;
  for (int k = 0; k < mine; ++k) {
    for (int st = 0; st < nst; ++st) {
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int e = 0; e < PH; ++e) mma(acc[mi][e], fa[mi], fb[e]);
      read(slot, 1, fa, fb);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int e = 0; e < PH; ++e) mma(acc[mi][e], fa[mi], fb[e]);
      slot = slot == NBUF - 1 ? 0 : slot + 1;
      if (st + 1 < nst) {
        read(slot, 0, fa, fb);  // stage s + 1 landed before B_s
        block_barrier();        // B_{s+1}
      }
    }

    // epilogue of tile k: degree sums with U_{d-1}(t) over this wave's
    // degrees d = dh PH + e + 1 (k_dx_dh's arithmetic), one fragment row at a
    // time; dh is made a constant so that no register array is indexed at run
    // time
    const int tix = (int)blockIdx.x + k * G;
    const int rb = tix % n_rb, ib = tix / n_rb;
    auto epilogue = [&](auto DH) __attribute__((always_inline)) {
      constexpr int d = decltype(DH)::value, keep = d, give = 1 - d;
      // the row handed to the pair first (its accumulators die before the
      // kept row's are read), each sum scaled by its row's input slope here,
      // so no tanh value is held across the exchange
      float part[2][16];  // [0]: the row handed over, [1]: the row kept
      int toff = (rg * 64 + 4 * g) * 32 + (lane & 31);
      asm volatile("" : "+v"(toff));
      const float* tl = tbuf + toff;
#pragma unroll
      for (int step = 0; step < 2; ++step) {
        const int mi = step == 0 ? give : keep;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float tv = tl[(mi * 32 + 8 * (v >> 2) + (v & 3)) * 32];
          const float t2 = tv + tv;
          float up = 0.0f, u = 1.0f;  // U_{-1}, U_0; advanced to U_{d*PH}
#pragma unroll
          for (int j = 0; j < PH; ++j) {
            const float un = fmaf(t2, u, -up);
            up = d ? u : up;
            u = d ? un : u;
          }
          float sum = 0.0f;
#pragma unroll
          for (int e = 0; e < PH; ++e) {
            sum = fmaf(acc[mi][e][v], u, sum);
            const float un = fmaf(t2, u, -up);
            up = u;
            u = un;
          }
          part[step][v] = sum * input_slope(tv, p);
          if ((v & 3) == 3) __builtin_amdgcn_sched_barrier(0);  // 168-register budget
        }
      }
      // the sums are formed here, before the barriers
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) asm volatile("" ::"v"(part[q][v]));
      wait_lgkmcnt<0>();
      block_barrier();  // B_S: every wave has read its tanh values; the buffer is free
      // wave (rg, d) keeps fragment row d and hands row 1 - d to its pair
      int xoff = rg * 2 * 16 * 64 + lane;
      asm volatile("" : "+v"(xoff));
      float* xw = tbuf + xoff + d * 16 * 64;
      const float* xr = tbuf + xoff + (d ^ 1) * 16 * 64;
#pragma unroll
      for (int v = 0; v < 16; ++v) xw[v * 64] = part[0][v];
      wait_lgkmcnt<0>();
      block_barrier();  // X
      float res[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float other = xr[v * 64];
        // fixed order: the lower degrees' half first
        res[v] = d ? other + part[1][v] : part[1][v] + other;
      }
      // row r0u + 4 g + 8 (v / 4) + v % 4, input i, by buffer stores: the
      // descriptor's base is row r0u and its size ends at row B (the unit
      // drops stores past it, the rows of a partial tile), a wave-uniform
      // row offset and a per-lane 32-bit offset (no 64-bit address registers)
      const int i = ib * 32 + (lane & 31);
      const int64_t r0u = ((int64_t)rb * 8 + rg * 2 + d) * 32;
      const int64_t rows_left = p.B - r0u;
      if (rows_left > 0) {
        const __amdgpu_buffer_rsrc_t rs =
            buffer_rsrc(dx + r0u * p.I, (int)((rows_left < 32 ? rows_left : 32) * p.I * 4));
        const int loff = (4 * g * p.I + i) * (int)sizeof(float);
        if (i < p.I) {
#pragma unroll
          for (int v = 0; v < 16; ++v)
            buffer_store_f32_nt(res[v], rs, loff, (8 * (v >> 2) + (v & 3)) * p.I * 4);
        }
      }
    };
    if (dh) epilogue(std::integral_constant<int, 1>{});
    else epilogue(std::integral_constant<int, 0>{});
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int e = 0; e < PH; ++e)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[mi][e][v] = 0.0f;
    // the next tile's first stage (landed before B_S); after the last tile a
    // read of in-range LDS whose values are never used (unconditional, so the
    // last stage's fragments are not kept live through the epilogue)
    read(slot, 0, fa, fb);
  }
}

// ---------------------------------------------------------------------------
// dX at degree 16, bf16: v_mfma_f32_16x16x32_bf16 on 16-input column
// fragments.  A 32-input block carries 16 x 32 = 512 GEMM columns, so the
// 32x32 kernel above fits only 128 rows per block and each wave reads 9 KiB
// of fragments per 8 MFMAs, which made LDS reads its bound at degree 16 (40 %
// MFMA busy).  Here a tile is 256 rows x 16 inputs x 16 degrees, as big as
// degree 8's, and each wave reads 12 KiB per 32 (half-size) MFMAs.  Both
// operands keep their 32-row / 32-input fragment layouts: a 16x16x32
// fragment (16 rows or inputs, 32 k = two 16-k fragments) is four 256-byte
// runs of them, gathered by one LDS-DMA copy into 1 KiB ordered by lane, so
// every fragment read is one contiguous ds_read_b128.  Lane l of a 16x16x32
// operand holds row (or input) l % 16 at k 8 (l / 16) .. + 7, i.e. 16-k block
// l / 32, half (l / 16) % 2 of the stored fragments.
//
// Persistent: one block per CU walks tiles blockIdx.x, + gridDim.x, ... as one
// stream of stages, so the copies of a tile's first stages are in flight
// while the previous tile finishes (its last MFMAs and epilogue) instead of
// after a new block's launch; with 16 stages per tile (512 outputs) or 2 (64)
// that start-up was a large share of each tile.  Consecutive tiles of a block
// keep their input block when the input blocks divide the grid, so each XCD
// (blocks round-robin over 8) keeps the same few coefficient blocks in L2.
//
// Stage (32 k): copies 0-15 = A fragments (rows 16 q .. + 15 of the tile),
// copies 16-31 = B fragments of degrees 0..15 (16 inputs).  Waves 0-3 issue
// the A copies after their MFMAs, waves 4-7 the B copies after their fragment
// reads (each wave four).  The tile's tanh values (256 rows x 16 inputs, for
// the epilogue) come by 16 more copies, two per wave, issued just before the
// copies of the tile's first stage, into one of two LDS buffers.  Every wait
// is on this wave's own copies (vmcnt, in issue order): at each stage only the
// copies issued one stage earlier may be pending.  The dx stores of a tile go out
// after the next tile's first barrier, so no wait ever covers stores issued
// just before it.  Wave (rg, dh) = (wave / 2, wave % 2) owns rows
// 64 rg .. + 63 (four 16-row fragments) and degrees 8 dh .. + 7.
// ---------------------------------------------------------------------------
struct Dx16 {
  static constexpr int THR = 512, NBUF = 3, ROWS = 256;
  static constexpr int STAGE_BYTES = 32 * 1024;
  static constexpr int RING = NBUF * STAGE_BYTES;          // 96 KiB
  static constexpr int TBUF = ROWS * 16 * 4;               // tanh values of a tile
  static constexpr int XCH = 8 * 2 * 4 * 64 * 4;           // the dh pairs' exchange
  static constexpr int LDS_BYTES = RING + 2 * TBUF + XCH;  // 144 KiB
};

__global__ void __launch_bounds__(512)
k_dx16(const uint16_t* __restrict__ dYx, const uint16_t* __restrict__ Cb,
       const float* __restrict__ tc, float* __restrict__ dx, Plan p, int nib16, int ntiles) {
  typedef Dx16 K;
  constexpr int P = 16, NBUF = K::NBUF;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int dh = wave & 1, rg = wave >> 1, hw = wave >> 2;
  const int nst = p.KBx / 2;
  const int G = gridDim.x;
  const int mine = (ntiles - (int)blockIdx.x + G - 1) / G;  // tiles of this block (>= 1)
  const int c4 = lane >> 4, kbl = c4 >> 1, gq = c4 & 1, l16 = lane & 15;
  const size_t frag_run = (size_t)p.KBx * 1024;  // bytes of one fragment row (all k)

  // per-lane copy offsets, the same for every tile and stage
  uint32_t off[4];
#pragma unroll
  for (int qi = 0; qi < 4; ++qi) {
    const int q = (wave & 3) * 4 + qi;  // A: 16-row fragment q; B: degree q
    off[qi] = hw ? (uint32_t)(((size_t)q * p.KBx + kbl) * 1024 + (l16 + 32 * gq) * 16)
                 : (uint32_t)(((size_t)(q >> 1) * p.KBx + kbl) * 1024 + (16 * (q & 1) + l16 + 32 * gq) * 16);
  }
  const uint32_t lring = (uint32_t)(uintptr_t)smem + (uint32_t)(hw * 16 + (wave & 3) * 4) * 1024;
  const uint32_t ltb = (uint32_t)(uintptr_t)smem + K::RING + (uint32_t)wave * 2048;
  const float* tbuf = reinterpret_cast<const float*>(smem + K::RING);
  float* xch = reinterpret_cast<float*>(smem + K::RING + 2 * K::TBUF);
  // tanh copy j (rows 16 (2 wave + j) .. + 15 of the tile): lane -> row
  // lane / 4, 16-byte chunk lane % 4 of the tile's 16 inputs
  const int trow = lane >> 2, tch = lane & 3;

  // issue cursor: tile ik of this block, stage ist, ring slot islot
  int ik = 0, ist = 0, islot = 0;
  const char* isrc = nullptr;  // copy base of tile ik (stage 0)
  auto tile_base = [&](int k) __attribute__((always_inline)) {
    const int tix = (int)blockIdx.x + (k < mine ? k : mine - 1) * G;
    const int rb = tix / nib16, ib = tix - rb * nib16;
    return hw ? reinterpret_cast<const char*>(Cb) + (size_t)(ib >> 1) * P * frag_run + (ib & 1) * 256
              : reinterpret_cast<const char*>(dYx) + (size_t)rb * 8 * frag_run;
  };
  auto issue = [&]() __attribute__((always_inline)) {
    if (ist == 0) {
      // the tile's tanh values, ahead of its first stage; past the last tile
      // the last tile's again, into the buffer no epilogue reads any more
      // (always two copies, so the waits below can count them)
      isrc = tile_base(ik);
      const int tix = (int)blockIdx.x + (ik < mine ? ik : mine - 1) * G;
      const int rb = tix / nib16, ib = tix - rb * nib16;
      const int ich = ib * 16 + 4 * tch < p.I_sg ? 4 * tch : 0;  // chunks past the pitch: unused
      const char* tb = reinterpret_cast<const char*>(tc + ib * 16);
      const uint32_t l = ltb + (uint32_t)(ik & 1) * K::TBUF;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t r = (int64_t)rb * K::ROWS + 16 * (2 * wave + j) + trow;
        const int64_t rr = r < p.B ? r : p.B - 1;  // rows past B: unused
        dma16s(tb, (uint32_t)((rr * p.I_sg + ich) * 4), l + j * 1024);
      }
    }
    // past the last tile: its last stage again (in range, never read)
    const char* sb = isrc + (size_t)(ik < mine ? ist : nst - 1) * 2048;
    const uint32_t l = lring + islot * K::STAGE_BYTES;
#pragma unroll
    for (int qi = 0; qi < 4; ++qi) dma16s(sb, off[qi], l + qi * 1024);
    islot = islot + 1 == NBUF ? 0 : islot + 1;
    if (++ist == nst) {
      ist = 0;
      ++ik;
    }
  };

  f32x4_t acc[4][8];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[mi][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // the previous tile's results, stored after the next tile's first barrier
  float res[2][4];
  int64_t rrow0 = 0;   // first row of the pending results (+ 16 m + v)
  int pend = 0;        // results pending
  int pcol = 0;        // their input column
  auto store_pending = [&]() __attribute__((always_inline)) {
    if (pend) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t r = rrow0 + 16 * m + v;
          if (pcol < p.I && r < p.B) __builtin_nontemporal_store(res[m][v], dx + r * p.I + pcol);
        }
      pend = 0;
    }
  };

  pin_sgpr(dx);
#pragma unroll
  for (int q = 0; q < NBUF - 1; ++q) issue();
  int k = 0, st = 0, slot = 0;
  const int total = mine * nst;
  for (int gs = 0; gs < total; ++gs) {
    // this wave's copies of this stage (and everything older) landed; issued
    // after them: the next stage's four copies, and before a tile's last stage
    // also the next tile's two tanh copies
    if (st == nst - 1) wait_vmcnt<4 * (NBUF - 2) + 2>();
    else wait_vmcnt<4 * (NBUF - 2)>();
    block_barrier();
    store_pending();
    const char* base = smem + slot * K::STAGE_BYTES;
    bf16x8_t fa[4], fb[8];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
      fa[mi] = *reinterpret_cast<const bf16x8_t*>(base + (rg * 4 + mi) * 1024 + lane * 16);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      fb[j] = *reinterpret_cast<const bf16x8_t*>(base + (16 + dh * 8 + j) * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);
    if (hw) issue();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) mma16(acc[mi][j], fa[mi], fb[j]);
    __builtin_amdgcn_sched_barrier(0);
    if (!hw) issue();
    slot = slot + 1 == NBUF ? 0 : slot + 1;
    if (++st < nst) continue;

    // ---- tile k done: epilogue ----
    const int tix = (int)blockIdx.x + k * G;
    const int rb = tix / nib16, ib = tix - rb * nib16;
    const float* tt = tbuf + (size_t)(k & 1) * K::ROWS * 16;
    const int rl0 = rg * 64 + 4 * c4;  // tile row of (mi, v) = rl0 + 16 mi + v
    // partial sums over this wave's degrees d = 8 dh + j + 1 (weights U_{d-1})
    float part[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float t = tt[(rl0 + 16 * mi + v) * 16 + l16];
        const float t2 = t + t;
        float up = 0.0f, u = 1.0f;  // U_{-1}, U_0; advanced to U_{8 dh}
        if (dh) {
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const float un = fmaf(t2, u, -up);
            up = u;
            u = un;
          }
        }
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          sum = fmaf(acc[mi][j][v], u, sum);
          const float un = fmaf(t2, u, -up);
          up = u;
          u = un;
        }
        part[mi][v] = sum;
      }
    // wave (rg, dh) keeps row fragments 2 dh, 2 dh + 1 and hands the other
    // two to its pair
    const int keep = 2 * dh, give = 2 - 2 * dh;
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int v = 0; v < 4; ++v) xch[(((rg * 2 + dh) * 2 + m) * 4 + v) * 64 + lane] = part[give + m][v];
    wait_lgkmcnt<0>();
    block_barrier();
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float other = xch[(((rg * 2 + (dh ^ 1)) * 2 + m) * 4 + v) * 64 + lane];
        const float mine_v = part[keep + m][v];
        // fixed order: the lower degrees' half first
        const float sum = dh ? other + mine_v : mine_v + other;
        res[m][v] = sum * input_slope(tt[(rl0 + 16 * (keep + m) + v) * 16 + l16], p);
      }
    rrow0 = (int64_t)rb * K::ROWS + rl0 + 16 * keep;
    pcol = ib * 16 + l16;
    pend = 1;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[mi][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    st = 0;
    ++k;
  }
  store_pending();
  wait_vmcnt<0>();  // the copies past the last tile
}

// ---------------------------------------------------------------------------
// dX: one block = 4 waves along rows x one input block (32 inputs x P degrees).
// B fragments (coefficients, all P degrees of the input block) are shared
// through LDS; A fragments (dy) are per-wave global loads, prefetched a stage
// ahead.  Epilogue: per (row, input), sum over degrees with d U_{d-1}(t) and
// the tanh chain factor, all in registers.
// ---------------------------------------------------------------------------
template <int P, bool BF, int NM, int KI>
__global__ void __launch_bounds__(256)
k_dx(const typename Elem<BF>::type* __restrict__ dYx, const typename Elem<BF>::type* __restrict__ Cb,
     const float* __restrict__ tc, float* __restrict__ dx, Plan p) {
  typedef typename Elem<BF>::type E;
  constexpr int WGM = 4;
  constexpr int STAGE = P * KI * kFragElems;
  constexpr int CE = 16 / (int)sizeof(E);
  constexpr int NCHUNK = STAGE / CE;
  constexpr int CPT = NCHUNK / 256;
  constexpr int CPE = KI * kFragElems / CE;  // chunks per degree
  static_assert(NCHUNK % 256 == 0, "stage must split evenly over 256 threads");
  __shared__ __attribute__((aligned(16))) E lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5;
  const int ib = blockIdx.y;
  const int64_t mf0 = (int64_t)blockIdx.x * WGM * NM + wave * NM;  // first 32-row fragment
  const int64_t nmf = p.B32 / 32;
  const int nst = p.KBx / KI;

  u32x4_t pre[CPT];
  auto gload = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      const int c = tid + q * 256;
      const int e = c / CPE, off = c - e * CPE;
      pre[q] = *reinterpret_cast<const u32x4_t*>(
          Cb + ((size_t)(ib * P + e) * p.KBx + (size_t)st * KI) * kFragElems + (size_t)off * CE);
    }
  };
  auto lstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < CPT; ++q)
      *reinterpret_cast<u32x4_t*>(lds + buf * STAGE + (tid + q * 256) * CE) = pre[q];
  };
  Frag<BF> apre[NM][KI];
  auto aload = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int k = 0; k < KI; ++k) {
        const int64_t mf = mf0 + mi;
        apre[mi][k] = (mf < nmf)
            ? load_frag<BF>(dYx + ((size_t)mf * p.KBx + (size_t)st * KI + k) * kFragElems, lane)
            : zero_frag<BF>();
      }
  };

  f32x16_t acc[NM][P];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int e = 0; e < P; ++e)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][e][v] = 0.0f;

  gload(0);
  lstore(0);
  aload(0);
  __syncthreads();

  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    const bool more = st + 1 < nst;
    Frag<BF> a[NM][KI];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int k = 0; k < KI; ++k) a[mi][k] = apre[mi][k];
    if (more) {
      gload(st + 1);
      aload(st + 1);
    }
    const E* sb = lds + buf * STAGE;
#pragma unroll
    for (int k = 0; k < KI; ++k) {
#pragma unroll
      for (int e = 0; e < P; ++e) {
        const Frag<BF> bfr = load_frag<BF>(sb + (e * KI + k) * kFragElems, lane);
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) mma(acc[mi][e], a[mi][k], bfr);
      }
    }
    if (more) lstore(buf ^ 1);
    __syncthreads();
  }

  const int i = ib * 32 + (lane & 31);
#pragma unroll
  for (int mi = 0; mi < NM; ++mi) {
    const int64_t r0 = (mf0 + mi) * 32;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t r = r0 + acc_row(v, g);
      const bool ok = r < p.B && i < p.I;
      const float tv = ok ? tc[r * p.I_sg + i] : 0.0f;
      const float t2 = tv + tv;
      float up = 0.0f, u = 1.0f, s = 0.0f;  // U_{-1}, U_0
#pragma unroll
      for (int e = 0; e < P; ++e) {
        s = fmaf(acc[mi][e][v], u, s);
        const float un = fmaf(t2, u, -up);
        up = u;
        u = un;
      }
      if (ok) __builtin_nontemporal_store(s * input_slope(tv, p), dx + r * p.I + i);
    }
  }
}

// ---------------------------------------------------------------------------
// dC: one block = 4 waves along outputs x one input block (32 inputs x P
// degrees) x one batch split.  The basis operand (rows = inputs, one fragment
// per degree) is generated by the block into LDS once per stage of KI
// k-blocks (16*KI batch rows); the dy operand (columns = outputs) is a
// per-wave global load prefetched a stage ahead.  Output: fp32 partials
// part[split][d-1][i][o], reduced by k_dc_finalize.
// ---------------------------------------------------------------------------
template <int P, bool BF, int NM, int KI>
__global__ void __launch_bounds__(256)
k_dc(const typename Elem<BF>::type* __restrict__ dYc, const float* __restrict__ tc,
     float* __restrict__ part, Plan p, int st_per_split) {
  typedef typename Elem<BF>::type E;
  constexpr int WGM = 4;
  static_assert(KI * 64 <= 256, "at most one generated lane-slot per thread per stage");
  constexpr int GEN = KI * 64;  // threads that generate the basis operand
  constexpr int STAGE = P * KI * kFragElems;
  __shared__ __attribute__((aligned(16))) E lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5;
  const int ib = blockIdx.y;
  const int mf0 = blockIdx.x * WGM * NM + wave * NM;  // first 32-output fragment
  const int nst = (int)(p.KBc / KI);
  const int st0 = blockIdx.z * st_per_split;
  const int st1 = min(nst, st0 + st_per_split);

  // generator slot of this thread: k-block kg of the stage, fragment lane ln
  const int kg = (tid >> 6) % KI, ln = tid & 63;
  const int gi = ib * 32 + (ln & 31);
  const bool gvalid = gi < p.I;
  float tpre[8];
  auto tload = [&](int st) __attribute__((always_inline)) {
    const int64_t b0 = ((int64_t)st * KI + kg) * 16 + 8 * (ln >> 5);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t b = b0 + j;
      tpre[j] = (gvalid && b < p.B) ? tc[b * p.I_sg + gi] : 0.0f;
    }
  };
  auto generate = [&](int buf) __attribute__((always_inline)) {
    float ta[8], tb[8], t2[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ta[j] = 1.0f;
      tb[j] = tpre[j];
      t2[j] = tpre[j] + tpre[j];
    }
    E* dst = lds + buf * STAGE + kg * kFragElems;
    store_frag<BF>(dst, ln, tb);  // T_1
#pragma unroll
    for (int e = 1; e < P; ++e) {
      float tn[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        tn[j] = fmaf(t2[j], tb[j], -ta[j]);
        ta[j] = tb[j];
        tb[j] = tn[j];
      }
      store_frag<BF>(dst + e * KI * kFragElems, ln, tn);
    }
  };
  Frag<BF> bpre[NM][KI];
  auto bload = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int k = 0; k < KI; ++k) {
        const int mf = mf0 + mi;
        bpre[mi][k] = (mf < p.NBf)
            ? load_frag<BF>(dYc + ((size_t)mf * p.KBc + (size_t)st * KI + k) * kFragElems, lane)
            : zero_frag<BF>();
      }
  };

  f32x16_t acc[P][NM];
#pragma unroll
  for (int e = 0; e < P; ++e)
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[e][mi][v] = 0.0f;

  const bool gen = tid < GEN;
  if (st0 < st1) {
    if (gen) {
      tload(st0);
      generate(0);
    }
    bload(st0);
  }
  __syncthreads();

  for (int st = st0; st < st1; ++st) {
    const int buf = (st - st0) & 1;
    const bool more = st + 1 < st1;
    Frag<BF> b[NM][KI];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int k = 0; k < KI; ++k) b[mi][k] = bpre[mi][k];
    if (more) {
      if (gen) tload(st + 1);
      bload(st + 1);
    }
    const E* sb = lds + buf * STAGE;
#pragma unroll
    for (int k = 0; k < KI; ++k) {
#pragma unroll
      for (int e = 0; e < P; ++e) {
        const Frag<BF> afr = load_frag<BF>(sb + (e * KI + k) * kFragElems, lane);
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) mma(acc[e][mi], afr, b[mi][k]);
      }
    }
    if (more && gen) generate(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int mi = 0; mi < NM; ++mi) {
    const int mf = mf0 + mi;
    if (mf >= p.NBf) continue;
    const int o = mf * 32 + (lane & 31);
#pragma unroll
    for (int e = 0; e < P; ++e) {
      float* dst = part + (((size_t)blockIdx.z * p.P + e) * p.I32 + ib * 32) * p.O32 + o;
#pragma unroll
      for (int v = 0; v < 16; ++v) dst[(size_t)acc_row(v, g) * p.O32] = acc[e][mi][v];
    }
  }
}

// ---------------------------------------------------------------------------
// dC, pipelined: dC[i, o, d] = sum_b T_d(t[b, i]) dy[b, o] for d >= 1.
// One block = 8 waves in H groups ("halves") that take alternate stages of KI
// k-blocks (16 batch rows each) of the reduction; in a group, wave (dq, og)
// accumulates PH = min(P, 4) degrees (group dq) x NN output fragments (group
// og) for the block's 32 inputs, always 8 accumulator fragments.  H = 2 (a
// K split inside the block), or H = 1 for degree 16 with at least 4 output
// fragments: 4 output fragments per block keep basis generation at 3 VALU
// per MFMA.
// Both streamed operands arrive by LDS DMA, with no vector-register loads in
// the loop: tanh tiles three pairs of stages ahead, dy fragments two pairs
// ahead.  The basis operand (P fragments per k-block) is generated from the
// tanh tile into LDS one pair ahead, interleaved with the MFMAs.  The halves'
// tiles are summed through LDS, then each output group is staged as
// [input][output][degree] (d = 0 from the reduced dy column sums) so that the
// block writes contiguous runs of dC, or of its split-K slice.
// ---------------------------------------------------------------------------
template <int P, bool BF, int H_>
struct DcPipe {
  typedef typename Elem<BF>::type E;
  static constexpr int H = H_;              // stage groups (K split inside the block)
  static constexpr int WG = 8 / H;          // waves per group
  static constexpr int PH = P < 4 ? P : 4;  // degrees per wave
  static constexpr int DQ = P / PH;         // degree groups in a group
  static constexpr int OG = WG / DQ;        // output groups in a group
  static constexpr int NN = 8 / PH;         // output fragments per wave
  static constexpr int NO = OG * NN;        // output fragments per block
  static constexpr int NF = PH * NN;        // accumulator fragments per wave (8)
  static constexpr int KI = (BF && P != 2 && (P != 16 || H == 1)) ? 2 : 1;
  static constexpr int FB = kFragElems * (int)sizeof(E);
  static constexpr int BAS_STAGE = P * KI * FB;
  static constexpr int DY_STAGE = NO * KI * FB;
  static constexpr int DY_CHUNKS = H * DY_STAGE / 16;             // real chunks per step
  static constexpr int DY_OPS = (DY_CHUNKS + 511) / 512;          // dma16 per thread per step
  static constexpr int DY_SLOT = DY_OPS * 8192;                   // bytes per step slot
  static constexpr int T_STAGE = KI * 16 * 32 * 4;                // tanh rows x 32 inputs
  static constexpr int T_CHUNKS = H * T_STAGE / 16;
  static constexpr int T_SLOT = 8192;                             // one dma16 per thread
  static constexpr int BAS_BYTES = 2 * H * BAS_STAGE;             // two steps of H stages
  static constexpr int MAIN_BYTES = BAS_BYTES + 3 * DY_SLOT + 3 * T_SLOT;
  static constexpr int XCH_BYTES = H == 2 ? 8 * (NF / 2) * 16 * 64 * 4 : 0;
  static constexpr int STG_BYTES = 32 * NN * 32 * (P + 1) * 4;  // one output group
  static constexpr int BIG_BYTES = MAIN_BYTES > XCH_BYTES
      ? (MAIN_BYTES > STG_BYTES ? MAIN_BYTES : STG_BYTES)
      : (XCH_BYTES > STG_BYTES ? XCH_BYTES : STG_BYTES);
  static constexpr int CS_BYTES = 512 * 4;  // column-sum partials of the block's outputs
  static constexpr int LDS_BYTES = BIG_BYTES + CS_BYTES;
  static constexpr int RPT = KI * H;  // batch rows per generating thread (of a lane's 8)
  static constexpr bool kOk = LDS_BYTES <= 160 * 1024 && T_CHUNKS <= 512 && NF % 2 == 0;
};

// The change of basis a dC launch applies before its stores (XF = true):
// g[n] = sum_{k <= n} g'[k] m[n][k] per (input, output) row of D values.
template <bool XF> struct DcXf { BasisXform x; };
template <> struct DcXf<false> {};
// LDS for M's rows n <= P, after the pipelined dC's own
template <int P> constexpr int kDcXfBytes = (P + 1) * kMaxD * (int)sizeof(float);
template <int P, bool BF, int H>
constexpr bool dc_xf_fits() { return DcPipe<P, BF, H>::kOk && DcPipe<P, BF, H>::LDS_BYTES + kDcXfBytes<P> <= 160 * 1024; }

template <int P, bool BF, int H_, bool XF = false>
__global__ void __launch_bounds__(512)
k_dc_pipe(const typename Elem<BF>::type* __restrict__ dYc, const float* __restrict__ tc,
          const float* __restrict__ colsum_part, float* __restrict__ out, Plan p, int st_per_split,
          DcOut om, DcXf<XF> xf) {
  typedef DcPipe<P, BF, H_> K;
  typedef typename K::E E;
  constexpr int PH = K::PH, DQ = K::DQ, OG = K::OG, NN = K::NN, NO = K::NO, NF = K::NF;
  constexpr int KI = K::KI, FB = K::FB, H = K::H, WG = K::WG;
  constexpr int RPT = K::RPT, DY_OPS = K::DY_OPS;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = wave / WG, wq = wave % WG, dh = wq % DQ, og = wq / DQ;
  if constexpr (XF) {
    // M (rows n <= P of kMaxD floats) past the kernel's own LDS: read by the
    // epilogue, after the loop's barriers have published it
    static_assert((P + 1) * kMaxD <= 512, "one element per thread");
    if (tid < (P + 1) * kMaxD)
      reinterpret_cast<float*>(smem + K::LDS_BYTES)[tid] = xf.x.m[tid];
  }
  const int g = lane >> 5;
  int ib, obk;
  xcd_patch(ib, obk);
  const int nst_all = (int)(p.KBc / KI);
  const int st0 = blockIdx.z * st_per_split;
  const int st1 = min(nst_all, st0 + st_per_split);
  const int npair = (st1 - st0) / H;  // steps of H stages (split stage counts are even)
  char* bas = smem;
  char* dyr = smem + K::BAS_BYTES;
  char* tlr = dyr + 3 * K::DY_SLOT;

  // DMA: waves 0-3 issue every copy of a step (the H stages of one pair step),
  // DH_OPS dy and TH_OPS tanh copies per thread, after their MFMAs of the
  // step before (see the loop).  Sources are a wave-uniform base plus a
  // per-lane 32-bit offset fixed for the kernel.
  constexpr int CPF = FB / 16;
  constexpr int DH_OPS = (K::DY_CHUNKS + 255) / 256, TH_OPS = (K::T_CHUNKS + 255) / 256;
  constexpr int HOPS = DH_OPS + TH_OPS;  // copies per thread per step
  static_assert(DH_OPS * 4096 <= K::DY_SLOT && TH_OPS * 4096 <= K::T_SLOT, "copy slots");
  const int t256 = tid & 255;
  const uint32_t w1k = (uint32_t)__builtin_amdgcn_readfirstlane(wave & 3) * 1024;
  // dy: chunk c < DY_CHUNKS of a step is [stage hs][fragment f][k-block kk][16 B];
  // chunks past that repeat real ones into the unused end of the slot
  const char* dyb = reinterpret_cast<const char*>(dYc) + (size_t)obk * NO * p.KBc * FB;
  uint32_t doff[DH_OPS];
#pragma unroll
  for (int q = 0; q < DH_OPS; ++q) {
    const int c = (q * 256 + t256) % K::DY_CHUNKS;
    const int hs = c / (NO * KI * CPF), r1 = c - hs * (NO * KI * CPF);
    const int f = r1 / (KI * CPF), r2 = r1 - f * (KI * CPF);
    const int kk = r2 / CPF, piece = r2 - kk * CPF;
    const int mf = min(obk * NO + f, p.NBf - 1);
    doff[q] = (uint32_t)(((size_t)(mf - obk * NO) * p.KBc + kk) * FB + (size_t)piece * 16 +
                         (size_t)hs * KI * FB);
  }
  // tanh tile of a stage: rows of 32 fp32 inputs.  Row rho is stored at row
  // t_row(rho) with its 16-byte chunks XOR-ed by t_xor(rho) / 4, so that the
  // generation reads (G row groups x 64/G columns per wave, see gen) hit 64
  // distinct banks, and each 32-lane half 32 distinct banks.  t_row only flips
  // bit 0 and t_xor reads bits 1..2, so both are unchanged by t_row.
  constexpr int G = 8 / RPT;  // generation row groups
  auto t_row = [](int r) __attribute__((always_inline)) {
    return RPT == 4 ? r ^ ((r >> 2) & 1) : RPT == 2 ? r ^ ((r >> 1) & 1) : r;
  };
  auto t_xor = [](int r) __attribute__((always_inline)) {
    return RPT == 4 ? 16 * ((r >> 2) & 1) : RPT == 2 ? 8 * ((r >> 1) & 3) : 4 * (r & 7);
  };
  // tanh copy q: chunk c = (q*256 + t256) % T_CHUNKS fills [stage ths][stored row trr][chunk c % 8]
  constexpr int SROWS = KI * 16;  // batch rows per stage
  int tsr[TH_OPS], tcl[TH_OPS], tst[TH_OPS];
  uint32_t toff[TH_OPS];
#pragma unroll
  for (int q = 0; q < TH_OPS; ++q) {
    const int c = (q * 256 + t256) % K::T_CHUNKS;
    tst[q] = c / (K::T_STAGE / 16);
    const int trr = (c % (K::T_STAGE / 16)) / 8;
    tsr[q] = t_row(trr);  // t_row is an involution
    tcl[q] = min(ib * 32 + (((c % 8) * 4) ^ t_xor(trr)), p.I_sg - 4);  // inputs past I_sg: never stored
    toff[q] = (uint32_t)(((size_t)tsr[q] * p.I_sg + tcl[q]) * 4);
  }
  const char* tcb = reinterpret_cast<const char*>(tc);
  const uint32_t dyl0 = (uint32_t)(uintptr_t)dyr + w1k, tll0 = (uint32_t)(uintptr_t)tlr + w1k;
  auto dma_dy = [&](int j) __attribute__((always_inline)) {
    int st = st0 + H * j;
    if (st + H > st1) st = st0;  // past the end: any in-range source, never read
    const char* sb = dyb + (size_t)st * KI * FB;
    const uint32_t l = dyl0 + (j % 3) * K::DY_SLOT;
#pragma unroll
    for (int q = 0; q < DH_OPS; ++q) dma16s_salu(sb, doff[q], l + q * 4096);
  };
  auto dma_t = [&](int j) __attribute__((always_inline)) {
    int st = st0 + H * j;
    if (st + H > st1) st = st0;
    const uint32_t l = tll0 + (j % 3) * K::T_SLOT;
#pragma unroll
    for (int q = 0; q < TH_OPS; ++q) {
      const int64_t row0 = (int64_t)(st + tst[q]) * SROWS;
      if (row0 + SROWS <= p.B) {
        dma16s(tcb + (size_t)row0 * p.I_sg * 4, toff[q], l + q * 4096);
      } else {
        // a stage past the last row: rows clamped to B - 1 (dy is zero there)
        const int64_t rb0 = row0 < p.B ? row0 : p.B - 1;
        int64_t b = row0 + tsr[q];
        if (b >= p.B) b = p.B - 1;
        dma16s(tcb + (size_t)rb0 * p.I_sg * 4, (uint32_t)(((size_t)(b - rb0) * p.I_sg + tcl[q]) * 4),
               l + q * 4096);
      }
    }
  };

  // basis generation slot of this thread within its half: k-block gkk,
  // fragment lane gl, rows grh*RPT .. +RPT of the lane's 8.  The G threads of
  // one fragment lane are adjacent, so each wave writes one contiguous run.
  const int th = tid % (512 / H);
  const int grh = th % G, gl = (th / G) % 64, gkk = th / (G * 64);
  const int trow0 = gkk * 16 + 8 * (gl >> 5) + grh * RPT;
  // the generation's tanh reads, issued apart so that they can go ahead of
  // the step's fragment reads (LDS returns in order)
  auto gen_read = [&](int j, float (&tv)[RPT]) __attribute__((always_inline)) {
    const float* tl = reinterpret_cast<const float*>(tlr + (j % 3) * K::T_SLOT + half * K::T_STAGE);
#pragma unroll
    for (int r = 0; r < RPT; ++r) tv[r] = tl[t_row(trow0 + r) * 32 + ((gl & 31) ^ t_xor(trow0 + r))];
  };
  auto gen_write = [&](int j, const float (&tv)[RPT]) __attribute__((always_inline)) {
    char* dst = bas + ((j & 1) * H + half) * K::BAS_STAGE + gkk * FB + (gl * 8 + grh * RPT) * (int)sizeof(E);
    float a[RPT], b[RPT], t2[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r) { a[r] = 1.0f; b[r] = tv[r]; t2[r] = tv[r] + tv[r]; }
#pragma unroll
    for (int e = 0; e < P; ++e) {
      if (e > 0) {
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
          const float n = fmaf(t2[r], b[r], -a[r]);
          a[r] = b[r];
          b[r] = n;
        }
      }
      char* d = dst + e * KI * FB;
      if constexpr (BF) {
        if constexpr (RPT == 4) {
          bf16x4_t w;
#pragma unroll
          for (int r = 0; r < 4; ++r) w[r] = (__bf16)b[r];
          *reinterpret_cast<bf16x4_t*>(d) = w;
        } else if constexpr (RPT == 2) {
          bf16x2_t w;
#pragma unroll
          for (int r = 0; r < 2; ++r) w[r] = (__bf16)b[r];
          *reinterpret_cast<bf16x2_t*>(d) = w;
        } else {
          *reinterpret_cast<__bf16*>(d) = (__bf16)b[0];
        }
      } else {
        if constexpr (RPT == 2) *reinterpret_cast<f32x2_t*>(d) = f32x2_t{b[0], b[1]};
        else *reinterpret_cast<float*>(d) = b[0];
      }
    }
  };

  f32x16_t acc[PH][NN];
#pragma unroll
  for (int e = 0; e < PH; ++e)
#pragma unroll
    for (int ni = 0; ni < NN; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[e][ni][v] = 0.0f;

  // One pair step of this wave: the fragments of all KI k-blocks of its stage
  // are read from LDS up front, and the basis generation for the next pair
  // (VALU + LDS traffic) is interleaved with the MFMAs.
  auto step = [&](int j) __attribute__((always_inline)) {
    const E* ab = reinterpret_cast<const E*>(bas + ((j & 1) * H + half) * K::BAS_STAGE) +
                  (size_t)(dh * PH) * KI * kFragElems;
    const E* bb = reinterpret_cast<const E*>(dyr + (j % 3) * K::DY_SLOT + half * K::DY_STAGE) +
                  (size_t)(og * NN) * KI * kFragElems;
    float tv[RPT];
    gen_read(j + 1, tv);
    __builtin_amdgcn_sched_barrier(0);
    Frag<BF> fa[KI][PH], fb[KI][NN];
#pragma unroll
    for (int kk = 0; kk < KI; ++kk) {
#pragma unroll
      for (int e = 0; e < PH; ++e) fa[kk][e] = load_frag<BF>(ab + (e * KI + kk) * kFragElems, lane);
#pragma unroll
      for (int ni = 0; ni < NN; ++ni) fb[kk][ni] = load_frag<BF>(bb + (ni * KI + kk) * kFragElems, lane);
      __builtin_amdgcn_sched_barrier(0);  // k-block order of the reads (LDS returns in order)
    }
    gen_write(j + 1, tv);
#pragma unroll
    for (int kk = 0; kk < KI; ++kk)
#pragma unroll
      for (int e = 0; e < PH; ++e)
#pragma unroll
        for (int ni = 0; ni < NN; ++ni) mma(acc[e][ni], fa[kk][e], fb[kk][ni]);
#pragma unroll
    for (int q = 0; q < KI * PH * NN; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // up to four VALU
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // up to one LDS read
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // up to one LDS write
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // prologue: tanh tiles of pairs 0..2, dy of pairs 0..1, basis of pair 0.
  // Waves 0-3 (the older wave of each SIMD, issued first) copy t(j+3) and
  // dy(j+2) after their MFMAs of step j, while waves 4-7 still run theirs;
  // both slots were last read in step j-1, before step j's barrier.  Past
  // the end the copies fetch in-range data that is never read.
  const bool copier = wave < 4;
  pin_sgpr(colsum_part);  // used after the loop
  pin_sgpr(out);
  if (copier) {
    dma_t(0);
    dma_t(1);
    dma_dy(0);
    dma_t(2);
    dma_dy(1);
    wait_vmcnt<2 * HOPS>();  // t(0) landed
  }
  block_barrier();
  {
    float tv0[RPT];
    gen_read(0, tv0);
    gen_write(0, tv0);
  }
  for (int j = 0; j < npair; ++j) {
    // dy(j) and t(j+1) have landed once only the copies of the last issue
    // (t(j+2), dy(j+1)) may be in flight
    if (copier) wait_vmcnt<HOPS>();
    wait_lgkmcnt<0>();  // this thread's basis writes for pair j are done
    block_barrier();
    step(j);  // also generates pair j+1 (unused after the last pair)
    if (copier) {
      dma_t(j + 3);
      dma_dy(j + 2);
    }
  }
  wait_vmcnt<0>();  // the prefetches past the end land before the LDS is reused

  // d = 0 column, sum_b dy[b, o]: thread (rgp, oi) adds every RS-th of the
  // NBB per-64-row partials of output oi (fixed order); the RS results are
  // combined in order when staged
  constexpr int NOW = NO * 32, RS = 512 / NOW;
  float* cpart = reinterpret_cast<float*>(smem + K::BIG_BYTES);
  if (blockIdx.z == 0) {
    const int oi = tid % NOW, rgp = tid / NOW;
    if (rgp < RS) {
      const int o = min(obk * NOW + oi, p.O32 - 1);
      const float* cp = colsum_part + o;
      // batches of 16 independent loads, each batch summed as a fixed tree
      float a = 0.0f;
      int k = rgp;
      for (; k + 15 * RS < p.NBB; k += 16 * RS) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = cp[(size_t)(k + u * RS) * p.O32];
#pragma unroll
        for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
          for (int u = 0; u < w; ++u) v[u] += v[u + w];
        a += v[0];
      }
      for (; k < p.NBB; k += RS) a += cp[(size_t)k * p.O32];
      cpart[rgp * NOW + oi] = a;
    }
  }

  // with H = 2 the groups exchange: group 0 keeps fragments [0, NF/2),
  // group 1 the rest; with H = 1 every wave keeps all NF
  wait_lgkmcnt<0>();
  block_barrier();
  float* xch = reinterpret_cast<float*>(smem);
  auto xat = [&](int giver, int fj, int v) __attribute__((always_inline)) {
    return xch + (((giver * 4 + wq) * (NF / 2) + fj) * 16 + v) * 64 + lane;
  };
  auto exchange = [&](auto KEEP) __attribute__((always_inline)) {
    constexpr int keep0 = decltype(KEEP)::value, give0 = NF / 2 - keep0;
#pragma unroll
    for (int fj = 0; fj < NF / 2; ++fj)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        *xat(half, fj, v) = acc[(give0 + fj) / NN][(give0 + fj) % NN][v];
    wait_lgkmcnt<0>();
    block_barrier();
#pragma unroll
    for (int fj = 0; fj < NF / 2; ++fj)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        acc[(keep0 + fj) / NN][(keep0 + fj) % NN][v] += *xat(half ^ 1, fj, v);
  };
  // staging of output group c: [32 inputs][NN*32 outputs][D degrees]
  float* stg = reinterpret_cast<float*>(smem);
  constexpr int OW = NN * 32;
  constexpr int NK = H == 2 ? NF / 2 : NF;  // fragments a wave stages
  auto stage_own = [&](auto KEEP) __attribute__((always_inline)) {
    constexpr int keep0 = decltype(KEEP)::value;
#pragma unroll
    for (int fj = 0; fj < NK; ++fj) {
      const int e = (keep0 + fj) / NN, ni = (keep0 + fj) % NN;
      const int d = dh * PH + e + 1;
      if (d > p.deg) continue;
      const int ol = ni * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) stg[(acc_row(v, g) * OW + ol) * p.D + d] = acc[e][ni][v];
    }
  };
  float* outz = out + (size_t)blockIdx.z * p.I * p.O * p.D;
  const int ivalid = min(32, p.I - ib * 32);
  if constexpr (H == 2) {
    if (half == 0) exchange(std::integral_constant<int, 0>{});
    else exchange(std::integral_constant<int, NF / 2>{});
  }
#pragma unroll 1
  for (int c = 0; c < OG; ++c) {
    const int o0 = (obk * NO + c * NN) * 32;
    const int ovalid = min(OW, p.O - o0);
    block_barrier();  // previous readers of the LDS are done
    if (og == c) {
      if (half == 0) stage_own(std::integral_constant<int, 0>{});
      else stage_own(std::integral_constant<int, NK>{});
    }
    for (int q = tid; q < 32 * OW; q += 512) {
      const int il = q / OW, ol = q - il * OW;
      float cs = 0.0f;
      if (blockIdx.z == 0 && ol < ovalid) {
#pragma unroll
        for (int r = 0; r < RS; ++r) cs += cpart[r * NOW + c * OW + ol];
      }
      stg[q * p.D] = cs;
    }
    wait_lgkmcnt<0>();
    block_barrier();
    if constexpr (XF) {
      // the staged rows in the family's basis, in the arithmetic of
      // k_coeff_from_cheb (the same bits as that separate pass); M from its
      // LDS copy
      const float* xm = reinterpret_cast<const float*>(smem + K::LDS_BYTES);
      // up to degree 8 the lower triangle of M (45 values) stays in registers
      // for all of the thread's rows; above, each use reads it from LDS
      constexpr bool MREG = P <= 8;
      float mr[MREG ? (P + 1) * (P + 2) / 2 : 1];
      if constexpr (MREG) {
#pragma unroll
        for (int n = 0, i = 0; n <= P; ++n)
#pragma unroll
          for (int k = 0; k <= n; ++k, ++i) mr[i] = xm[n * kMaxD + k];
      }
      for (int q = tid; q < 32 * OW; q += 512) {
        float* r = stg + q * p.D;
        float gv[P + 1];
#pragma unroll
        for (int k = 0; k <= P; ++k) gv[k] = k < p.D ? r[k] : 0.0f;
#pragma unroll
        for (int n = 0; n <= P; ++n) {
          float acc = 0.0f;
#pragma unroll
          for (int k = 0; k <= n; ++k)
            acc = fmaf(gv[k], MREG ? mr[n * (n + 1) / 2 + k] : xm[n * kMaxD + k], acc);
          if (n < p.D) r[n] = acc;
        }
      }
      wait_lgkmcnt<0>();
      block_barrier();
    }
    if (ovalid > 0) {
      // ivalid runs of ovalid * D contiguous floats (one per input row), as
      // float4 when every run starts 16-byte aligned
      const int run = ovalid * p.D;
      float* dst0 = outz + ((size_t)ib * 32 * p.O + o0) * p.D;
      const size_t pitch = (size_t)p.O * p.D;  // floats between input rows
      if (run % 4 == 0 && pitch % 4 == 0 && (reinterpret_cast<uintptr_t>(dst0) & 15) == 0) {
        const int run4 = run / 4;
        for (int q = tid; q < ivalid * run4; q += 512) {
          const int il = q / run4, k4 = q - il * run4;
          const f32x4_t v = *reinterpret_cast<const f32x4_t*>(stg + il * OW * p.D + 4 * k4);
          f32x4_t* d = reinterpret_cast<f32x4_t*>(dst0 + il * pitch) + k4;
          dc_write4(d, v, om);
        }
      } else {
        for (int q = tid; q < ivalid * run; q += 512) {
          const int il = q / run, k = q - il * run;
          const float v = stg[il * OW * p.D + k];
          float* d = dst0 + il * pitch + k;
          dc_write(d, v, om);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side configuration and launchers
// ---------------------------------------------------------------------------

// Raises a kernel's dynamic-LDS limit before its first launch on each device
// (the attribute is per device).  `done` holds one bit per device.
static void ensure_lds_limit(const void* fn, int bytes, std::atomic<uint32_t>& done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 32) dev = 0;
  const uint32_t bit = 1u << dev;
  if (done.load(std::memory_order_acquire) & bit) return;
  (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  done.fetch_or(bit, std::memory_order_acq_rel);
}

// Number of workgroups that fills the chip once: 256 CUs, one 4-wave block each.
static constexpr int kChipBlocks = 256;

// The pipelined forward addresses its copies as a block base plus a per-lane
// 32-bit offset: up to 4 output fragments of coefficients, 256 tanh rows.
static bool fwd_pipe_offsets_fit(const Plan& p) {
  return (uint64_t)4 * p.KB * kFragElems * p.esz < (1ull << 32) &&
         (uint64_t)256 * p.I_sg * sizeof(float) < (1ull << 32);
}

// The one-launch small-batch forward needs a block per CU or more: 8-output
// streams, so at least 2048 outputs.
constexpr int kFwdColsMinBlocks = 256;

FwdChoice choose_fwd(const Plan& p) {
  FwdChoice c;
  if (p.B <= (p.P == 2 ? 2 : 16) && p.esz == 2 && p.O32 / 8 >= kFwdColsMinBlocks) {
    // enough 8-output streams to spread the coefficient stream over the chip
    // without a split reduction: one launch
    c.tile = kFwdCols;
    c.bm = p.B <= 1 ? 1 : p.B <= 2 ? 2 : p.B <= 4 ? 4 : p.B <= 8 ? 8 : 16;
    c.bnf = 8;
    c.tiles_m = 1;
    c.tiles_n = p.O32 / 8;
    c.splits = 1;
    c.sg_per_split = p.I_sg / p.SGI;
    return c;
  }
  if (p.B <= 64) {
    // coefficient streaming: one 4-wave block per 4 x SPW super-groups of a column block
    const int spw = 16 / p.SGK;
    const int nsg = p.I_sg / p.SGI;
    c.tile = p.B <= 32 ? kFwdStream32 : kFwdStream64;
    c.bm = p.B <= 32 ? 32 : 64;
    c.bnf = 1;
    c.tiles_m = 1;
    c.tiles_n = p.NBf;
    c.splits = (int)ceil_div(nsg, 4 * spw);  // blocks per column block
    c.sg_per_split = 4 * spw;
    return c;
  }
  if (p.B <= 32) {
    c.tile = kFwdSmall32; c.bm = 32; c.bnf = 4;
  } else if (p.B <= 64 || (p.B <= 512 && ceil_div(p.B, 256) * ceil_div(p.NBf, 4) < 64)) {
    // at most 2 output fragments: 2 x 2 waves, none idle (config 2's 784 -> 64
    // forward 13.4 -> 10.6 us with the tanh in the kernel)
    if (p.NBf <= 2) {
      c.tile = kFwdSmall64N2; c.bm = 64; c.bnf = 2;
    } else {
      c.tile = kFwdSmall64; c.bm = 64; c.bnf = 4;
    }
  } else {
    // at most 64 outputs: a 64-column tile (the pipelined kernel's BNF = 2)
    c.tile = kFwdBig; c.bm = 256; c.bnf = p.NBf <= 2 ? 2 : 4;
  }
  c.tiles_m = (int)ceil_div(p.B, c.bm);
  c.tiles_n = (int)ceil_div(p.NBf, c.bnf);
  const int nsg = p.I_sg / p.SGI;
  const int64_t tiles = (int64_t)c.tiles_m * c.tiles_n;
  const int target = (c.tile == kFwdBig) ? kChipBlocks : 2 * kChipBlocks;
  int splits = 1;
  if (tiles < target) splits = (int)ceil_div(target, tiles);
  // at least 4 super-groups per split for the large tile; the small-batch
  // tiles are latency-bound (a block's super-groups run one after another),
  // so they split down to one super-group each (config 2: 131 -> 119 us/step)
  const int min_sg = c.tile == kFwdBig ? 4 : 1;
  const int max_splits = (int)ceil_div(nsg, min_sg);
  if (splits > max_splits) splits = max_splits;
  if (splits > 64) splits = 64;
  if (splits < 1) splits = 1;
  c.sg_per_split = (int)ceil_div(nsg, splits);
  c.splits = (int)ceil_div(nsg, c.sg_per_split);
  if (c.splits < 1) c.splits = 1;
  return c;
}

template <int P, bool BF>
static void fwd_dispatch(const float* x, float* t, const void* packed, float* y, void* ws,
                         const Plan& p, const FwdChoice& c, hipStream_t s, int nib,
                         bool out_tanh, bool reduce, bool xt) {
  typedef typename Elem<BF>::type E;
  const E* Cf = reinterpret_cast<const E*>(packed);
  char* pk = const_cast<char*>(reinterpret_cast<const char*>(packed));
  const float* bias = reinterpret_cast<const float*>(pk + packed_biasf_offset(p));
  // nib > 0: the forward sums the per-input-block bias partials itself and
  // fills the bias slot (bias_out) for later forwards on this packed buffer
  const float* bpart = reinterpret_cast<const float*>(pk + packed_bias_offset(p));
  float* bias_out = nib > 0 ? reinterpret_cast<float*>(pk + packed_biasf_offset(p)) : nullptr;
  float* part = reinterpret_cast<float*>(ws);
  const bool split = c.splits > 1 || fwd_streaming(c);
  const int nib_k = split ? 0 : nib;  // unsplit kernels add the bias, split ones leave it to the reduce
  if (c.tile == kFwdCols) {
    if constexpr (BF) {
      const dim3 g((unsigned)c.tiles_n);
      const uint16_t* cf = reinterpret_cast<const uint16_t*>(Cf);
#define CKAN_COLS(R)                                                                       \
  hipLaunchKernelGGL((k_fwd_cols<P, R>), g, dim3(1024), 0, s, x, t, cf, bias, y, p, bpart, \
                     nib_k, bias_out)
      // degree 2 (four inputs per vector in registers) up to 2 rows
      if (c.bm == 1) CKAN_COLS(1);
      else if (c.bm == 2) CKAN_COLS(2);
      else if constexpr (P > 2) {
        if (c.bm == 4) CKAN_COLS(4);
        else if (c.bm == 8) CKAN_COLS(8);
        else CKAN_COLS(16);
      }
#undef CKAN_COLS
    }
    return;
  }
  if (fwd_streaming(c)) {
    dim3 g1(c.tiles_n * c.splits);
    if (c.tile == kFwdStream32)
      hipLaunchKernelGGL((k_fwd_stream<P, BF, 1, false>), g1, dim3(256), 0, s, x, t, Cf, part, p, c.splits, (int)is_al16(x));
    else  // 33..64 rows: tanh once by launch_tanh, not once per column block
      hipLaunchKernelGGL((k_fwd_stream<P, BF, 2, true>), g1, dim3(256), 0, s, x, t, Cf, part, p, c.splits, (int)is_al16(x));
  } else {
    dim3 grid(c.tiles_m, c.tiles_n, c.splits);
    switch (c.tile) {
      // xt: the kernel maps x itself and stores the tanh cache t
      case kFwdSmall32:
        if (xt)
          hipLaunchKernelGGL((k_fwd<P, BF, 1, 1, 1, 4, true>), grid, dim3(256), 0, s, x, Cf, bias, y,
                             part, p, c.sg_per_split, bpart, nib_k, bias_out, t);
        else
          hipLaunchKernelGGL((k_fwd<P, BF, 1, 1, 1, 4>), grid, dim3(256), 0, s, t, Cf, bias, y, part,
                             p, c.sg_per_split, bpart, nib_k, bias_out, nullptr);
        break;
      case kFwdSmall64N2:
        if (xt)
          hipLaunchKernelGGL((k_fwd<P, BF, 1, 1, 2, 2, true>), grid, dim3(256), 0, s, x, Cf, bias, y,
                             part, p, c.sg_per_split, bpart, nib_k, bias_out, t);
        else
          hipLaunchKernelGGL((k_fwd<P, BF, 1, 1, 2, 2>), grid, dim3(256), 0, s, t, Cf, bias, y, part,
                             p, c.sg_per_split, bpart, nib_k, bias_out, nullptr);
        break;
      case kFwdSmall64:
        if (xt)
          hipLaunchKernelGGL((k_fwd<P, BF, 2, 1, 1, 4, true>), grid, dim3(256), 0, s, x, Cf, bias, y,
                             part, p, c.sg_per_split, bpart, nib_k, bias_out, t);
        else
          hipLaunchKernelGGL((k_fwd<P, BF, 2, 1, 1, 4>), grid, dim3(256), 0, s, t, Cf, bias, y, part,
                             p, c.sg_per_split, bpart, nib_k, bias_out, nullptr);
        break;
      default:
        if constexpr (FwdPipe<P, BF>::kOk) {
          if (!fwd_pipe_offsets_fit(p)) {  // per-lane copy offsets are 32-bit
            hipLaunchKernelGGL((k_fwd<P, BF, 2, 4, 4, 1>), grid, dim3(256), 0, s, t, Cf, bias, y,
                               part, p, c.sg_per_split, bpart, nib_k, bias_out, nullptr);
            break;
          }
          // one LDS-limit flag per instantiation
          auto launch = [&](auto OTc, auto BNFc, std::atomic<uint32_t>& flag) {
            constexpr bool OTv = decltype(OTc)::value;
            constexpr int BNFv = decltype(BNFc)::value;
            typedef FwdPipe<P, BF, BNFv> KV;
            const void* fn = reinterpret_cast<const void*>(&k_fwd_pipe<P, BF, OTv, BNFv>);
            ensure_lds_limit(fn, KV::LDS_BYTES, flag);
            hipLaunchKernelGGL((k_fwd_pipe<P, BF, OTv, BNFv>), grid, dim3(KV::THREADS),
                               (size_t)KV::LDS_BYTES, s, t, Cf, bias, y, part, p, c.sg_per_split,
                               bpart, nib_k, nib_k > 0 ? bias_out : nullptr);
          };
          typedef std::integral_constant<bool, true> OT1;
          typedef std::integral_constant<bool, false> OT0;
          static std::atomic<uint32_t> lds_set[4];
          if (c.bnf == 2) {
            if (out_tanh) launch(OT1{}, std::integral_constant<int, 2>{}, lds_set[0]);
            else launch(OT0{}, std::integral_constant<int, 2>{}, lds_set[1]);
          } else {
            if (out_tanh) launch(OT1{}, std::integral_constant<int, 4>{}, lds_set[2]);
            else launch(OT0{}, std::integral_constant<int, 4>{}, lds_set[3]);
          }
        } else {
          hipLaunchKernelGGL((k_fwd<P, BF, 2, 4, 4, 1>), grid, dim3(256), 0, s, t, Cf, bias, y,
                             part, p, c.sg_per_split, bpart, nib_k, bias_out, nullptr);
        }
        break;
    }
  }
  if (split && reduce) {
    const int64_t n = p.B * (int64_t)p.O;
    int64_t gsz = ((n > p.O32 ? n : p.O32) + 255) / 256;
    if (gsz > 65536) gsz = 65536;
    hipLaunchKernelGGL(k_fwd_reduce, dim3((unsigned)gsz), dim3(256), 0, s, part, c.splits, bias, y,
                       p, bpart, nib, bias_out, (int)out_tanh);
  }
}

// The forward can store tanh(y) in place of y: the pipelined kernel, unsplit,
// stores y itself; a split forward's reduce stores every y.
template <int P, bool BF> static bool out_tanh_ok(const Plan& p, const FwdChoice& c) {
  if (c.tile != kFwdCols && (c.splits > 1 || fwd_streaming(c))) return true;
  if constexpr (FwdPipe<P, BF>::kOk)
    return c.tile == kFwdBig && c.splits == 1 && fwd_pipe_offsets_fit(p);
  else
    return false;
}
bool fwd_out_tanh_ok(const Plan& p) {
  const FwdChoice c = choose_fwd(p);
  const bool bf = p.esz == 2;
  switch (p.P) {
    case 2: return bf ? out_tanh_ok<2, true>(p, c) : out_tanh_ok<2, false>(p, c);
    case 4: return bf ? out_tanh_ok<4, true>(p, c) : out_tanh_ok<4, false>(p, c);
    case 8: return bf ? out_tanh_ok<8, true>(p, c) : out_tanh_ok<8, false>(p, c);
    default: return bf ? out_tanh_ok<16, true>(p, c) : out_tanh_ok<16, false>(p, c);
  }
}

// The forward can sum the bias partials itself: every unsplit kernel does it
// once per column; a split forward's reduce does it per output element, so
// only for small outputs.
bool fwd_sums_bias(const Plan& p, const FwdChoice& c) {
  if (p.NIB <= 1) return false;
  const bool split = c.splits > 1 || fwd_streaming(c);
  if (split) return (uint64_t)p.B * p.O * p.NIB <= ((uint64_t)1 << 22);
  return true;
}

bool fwd_maps_x_ok(const Plan& p, const FwdChoice& c, const float* x) {
  return (c.tile == kFwdSmall32 || c.tile == kFwdSmall64 || c.tile == kFwdSmall64N2) &&
         p.I == p.I_sg && p.I % 4 == 0 &&
         is_al16(x);
}

void launch_fwd_gemm(const float* x, float* t, const void* packed, float* y, void* ws,
                     const Plan& p, const FwdChoice& c, hipStream_t s, bool sum_bias,
                     bool out_tanh, bool reduce, bool xt) {
  const bool bf = p.esz == 2;
  const int nib = sum_bias && fwd_sums_bias(p, c) ? p.NIB : 0;
#define CKAN_FW(PP, BB) fwd_dispatch<PP, BB>(x, t, packed, y, ws, p, c, s, nib, out_tanh, reduce, xt)
  switch (p.P) {
    case 2: bf ? CKAN_FW(2, true) : CKAN_FW(2, false); break;
    case 4: bf ? CKAN_FW(4, true) : CKAN_FW(4, false); break;
    case 8: bf ? CKAN_FW(8, true) : CKAN_FW(8, false); break;
    default: bf ? CKAN_FW(16, true) : CKAN_FW(16, false); break;
  }
#undef CKAN_FW
}

// dX stage depth: 4 k-blocks for bf16; fp32 halves it to bound LDS.
template <bool BF> struct DxKI { static constexpr int v = BF ? 4 : 2; };

// k_dx16's limits: 32-bit per-lane offsets into the tanh cache and a tile
// count that fits an int
static bool dx16_ok(const Plan& p) {
  return (uint64_t)p.B * p.I_sg * sizeof(float) < (1ull << 32) &&
         ceil_div(p.B32, Dx16::ROWS) * ceil_div(p.I, 16) < (1ll << 30);
}

// k_dx_ws's limits: at least four stages per tile (the tanh copies of a tile
// are waited two stages after their issue), 32-bit per-lane offsets into the
// tanh cache, a tile count that fits an int
static bool dx_ws_ok(const Plan& p) {
  return p.KBx / DxWs<8>::KI >= DxWs<8>::MIN_STAGES &&
         (uint64_t)p.B * p.I_sg * sizeof(float) < (1ull << 32) &&
         ceil_div(p.B32, 256) * p.NIB < (1ll << 30);
}

template <int P, bool BF>
static void dx_dispatch(const void* dYx, const void* packed, const float* t, float* dx,
                        const Plan& p, hipStream_t s) {
  typedef typename Elem<BF>::type E;
  constexpr int NM = BwdTile<P>::NM;
  const E* Cb = reinterpret_cast<const E*>(packed) + packed_cf_elems(p);
  if constexpr (P == 16 && BF) {
    if (dx16_ok(p)) {
      const int nib16 = (int)ceil_div(p.I, 16);
      const int ntiles = (int)(ceil_div(p.B32, Dx16::ROWS) * nib16);
      static std::atomic<uint32_t> lds_set{0};
      ensure_lds_limit(reinterpret_cast<const void*>(&k_dx16), Dx16::LDS_BYTES, lds_set);
      hipLaunchKernelGGL(k_dx16, dim3(ntiles < kChipBlocks ? ntiles : kChipBlocks), dim3(Dx16::THR),
                         Dx16::LDS_BYTES, s, reinterpret_cast<const uint16_t*>(dYx),
                         reinterpret_cast<const uint16_t*>(Cb), t, dx, p, nib16, ntiles);
      return;
    }
  }
  if constexpr (BF && (P == 4 || P == 8)) {
    if (dx_ws_ok(p)) {
      typedef DxWs<P> K;
      const int n_rb = (int)ceil_div(p.B32, 256);
      const int ntiles = n_rb * p.NIB;
      static std::atomic<uint32_t> lds_set{0};
      ensure_lds_limit(reinterpret_cast<const void*>(&k_dx_ws<P>), K::LDS_BYTES, lds_set);
      hipLaunchKernelGGL((k_dx_ws<P>), dim3(ntiles < kChipBlocks ? ntiles : kChipBlocks),
                         dim3(K::THR), K::LDS_BYTES, s, reinterpret_cast<const uint16_t*>(dYx),
                         reinterpret_cast<const uint16_t*>(Cb), t, dx, p, n_rb, ntiles);
      return;
    }
  }
  if constexpr (DxDh<P, BF>::kOk) {
    typedef DxDh<P, BF> K;
    const int n_rb = (int)ceil_div(p.B32 / 32, K::RG * K::NM);
    static std::atomic<uint32_t> lds_set{0};
    ensure_lds_limit(reinterpret_cast<const void*>(&k_dx_dh<P, BF>), K::LDS_BYTES, lds_set);
    hipLaunchKernelGGL((k_dx_dh<P, BF>), dim3(n_rb * p.NIB), dim3(K::THR), K::LDS_BYTES, s,
                       reinterpret_cast<const E*>(dYx), Cb, t, dx, p, n_rb);
    return;
  }
  if constexpr (DxPipe<P, BF>::kOk) {
    typedef DxPipe<P, BF> K;
    const int n_rb = (int)ceil_div(p.B32 / 32, K::WGM * NM);
    const int blocks = n_rb * p.NIB;
    const size_t lds = (size_t)K::NBUF * K::STAGE_BYTES;
    static std::atomic<uint32_t> lds_set{0};
    ensure_lds_limit(reinterpret_cast<const void*>(&k_dx_pipe<P, BF>), (int)lds, lds_set);
    hipLaunchKernelGGL((k_dx_pipe<P, BF>), dim3(blocks), dim3(256), lds, s,
                       reinterpret_cast<const E*>(dYx), Cb, t, dx, p, n_rb);
    return;
  }
  dim3 grid((unsigned)ceil_div(p.B32 / 32, 4 * NM), p.NIB);
  hipLaunchKernelGGL((k_dx<P, BF, NM, DxKI<BF>::v>), grid, dim3(256), 0, s,
                     reinterpret_cast<const E*>(dYx), Cb, t, dx, p);
}

void launch_dx_gemm(const void* dYx, const void* packed, const float* t, float* dx,
                    const Plan& p, hipStream_t s) {
  const bool bf = p.esz == 2;
  switch (p.P) {
    case 2: bf ? dx_dispatch<2, true>(dYx, packed, t, dx, p, s) : dx_dispatch<2, false>(dYx, packed, t, dx, p, s); break;
    case 4: bf ? dx_dispatch<4, true>(dYx, packed, t, dx, p, s) : dx_dispatch<4, false>(dYx, packed, t, dx, p, s); break;
    case 8: bf ? dx_dispatch<8, true>(dYx, packed, t, dx, p, s) : dx_dispatch<8, false>(dYx, packed, t, dx, p, s); break;
    default: bf ? dx_dispatch<16, true>(dYx, packed, t, dx, p, s) : dx_dispatch<16, false>(dYx, packed, t, dx, p, s); break;
  }
}

// dC stage depth in k-blocks: 4 for bf16, 2 for fp32 (LDS bound).
template <bool BF> struct DcKI { static constexpr int v = BF ? 4 : 2; };

// Stage groups of the pipelined dC kernel for this shape (see DcPipe).
static int dc_h(const Plan& p) { return (p.P == 16 && p.NBf >= 4) ? 1 : 2; }

template <int P, bool BF> static bool dc_ok_t(int h) {
  return h == 1 ? DcPipe<P, BF, 1>::kOk : DcPipe<P, BF, 2>::kOk;
}
static bool dc_pipe_ok(const Plan& p) {
  const bool bf = p.esz == 2;
  const int h = dc_h(p);
  switch (p.P) {
    case 2: return bf ? dc_ok_t<2, true>(h) : dc_ok_t<2, false>(h);
    case 4: return bf ? dc_ok_t<4, true>(h) : dc_ok_t<4, false>(h);
    case 8: return bf ? dc_ok_t<8, true>(h) : dc_ok_t<8, false>(h);
    default: return bf ? dc_ok_t<16, true>(h) : dc_ok_t<16, false>(h);
  }
}

// output fragments per dC block and k-blocks per stage of the pipelined kernel
template <int P, bool BF> static void dc_shape_t(int h, int& no, int& ki) {
  no = h == 1 ? DcPipe<P, BF, 1>::NO : DcPipe<P, BF, 2>::NO;
  ki = h == 1 ? DcPipe<P, BF, 1>::KI : DcPipe<P, BF, 2>::KI;
}
static void dc_pipe_shape(const Plan& p, int& no, int& ki) {
  const bool bf = p.esz == 2;
  const int h = dc_h(p);
  switch (p.P) {
    case 2: bf ? dc_shape_t<2, true>(h, no, ki) : dc_shape_t<2, false>(h, no, ki); break;
    case 4: bf ? dc_shape_t<4, true>(h, no, ki) : dc_shape_t<4, false>(h, no, ki); break;
    case 8: bf ? dc_shape_t<8, true>(h, no, ki) : dc_shape_t<8, false>(h, no, ki); break;
    default: bf ? dc_shape_t<16, true>(h, no, ki) : dc_shape_t<16, false>(h, no, ki); break;
  }
}

BwdLayout bwd_layout(const Plan& p, bool need_dx_arg, bool need_dc_arg) {
  BwdLayout L;
  L.dc_small = need_dc_arg && dc_small_ok(p);
  L.dx_small = need_dx_arg && dx_small_ok(p);
  // the re-laid operands and partials
  const bool need_dc = need_dc_arg && !L.dc_small, need_dx = need_dx_arg && !L.dx_small;
  size_t off = 0;
  L.dyx_off = off;
  if (need_dx) off += align256((size_t)dx_row_frags(p) * p.KBx * kFragElems * p.esz);
  L.dyc_off = off;
  if (need_dc) off += align256((size_t)p.NBf * p.KBc * kFragElems * p.esz);
  L.colsum_off = off;  // NBB partial rows + the reduced row
  if (need_dc) off += align256((size_t)(p.NBB + 1) * p.O32 * sizeof(float));
  L.part_off = off;
  L.dc_splits = 1;
  L.dc_st_per_split = 0;
  L.dc_pipe = need_dc && dc_pipe_ok(p);
  if (need_dc && L.dc_pipe) {
    int no, ki;
    dc_pipe_shape(p, no, ki);
    const int64_t tiles = (int64_t)p.NIB * ceil_div(p.NBf, no);
    const int nst = (int)(p.KBc / ki);
    int splits = 1;
    if (tiles < kChipBlocks) splits = (int)ceil_div(kChipBlocks, tiles);
    // at least one pair of stages per split (latency-bound small problems
    // gain from the parallelism: config 2 119 -> 114 us/step)
    const int max_splits = nst / 2 > 1 ? nst / 2 : 1;
    if (splits > max_splits) splits = max_splits;
    if (splits > 64) splits = 64;
    if (splits < 1) splits = 1;
    // even stage counts per split (nst is even: Bc is a multiple of 64 rows)
    L.dc_st_per_split = (int)round_up(ceil_div(nst, splits), 2);
    L.dc_splits = (int)ceil_div(nst, L.dc_st_per_split);
    if (L.dc_splits > 1) off += align256((size_t)L.dc_splits * p.I * p.O * p.D * sizeof(float));
  } else if (need_dc) {
    const int nm = bwd_nm(p.P);
    const int64_t tiles = ceil_div(p.NBf, 4 * nm) * (int64_t)p.NIB;
    const int nst = (int)(p.KBc / (p.esz == 2 ? DcKI<true>::v : DcKI<false>::v));
    int splits = 1;
    if (tiles < kChipBlocks) splits = (int)ceil_div(kChipBlocks, tiles);
    if (splits > nst) splits = nst;
    if (splits > 64) splits = 64;
    if (splits < 1) splits = 1;
    L.dc_st_per_split = (int)ceil_div(nst, splits);
    L.dc_splits = (int)ceil_div(nst, L.dc_st_per_split);
    if (L.dc_splits < 1) L.dc_splits = 1;
    off += align256((size_t)L.dc_splits * p.P * p.I32 * p.O32 * sizeof(float));
  }
  L.total = off;
  return L;
}

template <int P, bool BF, int H>
static bool dc_pipe_launch(const void* dYc, const float* t, const float* colsum, float* part,
                           float* dC, DcOut om, const Plan& p, const BwdLayout& L,
                           hipStream_t s, const BasisXform* xf) {
  typedef typename Elem<BF>::type E;
  if constexpr (DcPipe<P, BF, H>::kOk) {
    typedef DcPipe<P, BF, H> K;
    const bool split = L.dc_splits > 1;
    dim3 grid(p.NIB, (unsigned)ceil_div(p.NBf, K::NO), L.dc_splits);
    if constexpr (dc_xf_fits<P, BF, H>()) {
      if (xf && !split) {  // the unsplit launch writes the whole gradient: it maps it
        static std::atomic<uint32_t> lds_xf{0};
        const int lds = K::LDS_BYTES + kDcXfBytes<P>;
        ensure_lds_limit(reinterpret_cast<const void*>(&k_dc_pipe<P, BF, H, true>), lds, lds_xf);
        hipLaunchKernelGGL((k_dc_pipe<P, BF, H, true>), grid, dim3(512), (size_t)lds, s,
                           reinterpret_cast<const E*>(dYc), t, colsum, dC, p, L.dc_st_per_split,
                           om, DcXf<true>{*xf});
        return true;
      }
    }
    static std::atomic<uint32_t> lds_set{0};
    ensure_lds_limit(reinterpret_cast<const void*>(&k_dc_pipe<P, BF, H>), K::LDS_BYTES, lds_set);
    hipLaunchKernelGGL((k_dc_pipe<P, BF, H>), grid, dim3(512), K::LDS_BYTES, s,
                       reinterpret_cast<const E*>(dYc), t, colsum, split ? part : dC, p,
                       L.dc_st_per_split, split ? DcOut{kDcStore} : om, DcXf<false>{});
    return true;
  }
  return false;
}

template <int P, bool BF>
static void dc_dispatch(const void* dYc, const float* t, const float* colsum, float* part,
                        float* dC, DcOut om, const Plan& p, const BwdLayout& L,
                        hipStream_t s, const BasisXform* xf) {
  typedef typename Elem<BF>::type E;
  if (L.dc_pipe) {
    bool done = false;
    if constexpr (P == 16) {  // dc_h(p) is 1 only for degree 16
      if (dc_h(p) == 1) done = dc_pipe_launch<P, BF, 1>(dYc, t, colsum, part, dC, om, p, L, s, xf);
    }
    if (!done) done = dc_pipe_launch<P, BF, 2>(dYc, t, colsum, part, dC, om, p, L, s, xf);
    if (done) return;
  }
  constexpr int NM = BwdTile<P>::NM;
  dim3 grid((unsigned)ceil_div(p.NBf, 4 * NM), p.NIB, L.dc_splits);
  hipLaunchKernelGGL((k_dc<P, BF, NM, DcKI<BF>::v>), grid, dim3(256), 0, s,
                     reinterpret_cast<const E*>(dYc), t, part, p, L.dc_st_per_split);
}

bool dc_gemm_maps_basis(const Plan& p, const BwdLayout& L) {
  if (!L.dc_pipe || L.dc_splits > 1) return false;
  const bool bf = p.esz == 2;
  // the instantiation dc_dispatch launches, and whether it has LDS left for M
  switch (p.P) {
    case 2: return bf ? dc_xf_fits<2, true, 2>() : dc_xf_fits<2, false, 2>();
    case 4: return bf ? dc_xf_fits<4, true, 2>() : dc_xf_fits<4, false, 2>();
    case 8: return bf ? dc_xf_fits<8, true, 2>() : dc_xf_fits<8, false, 2>();
    default: {  // H = 1 where dc_h says so and that kernel fits, else H = 2
      const bool h1 = dc_h(p) == 1 && (bf ? DcPipe<16, true, 1>::kOk : DcPipe<16, false, 1>::kOk);
      if (h1) return bf ? dc_xf_fits<16, true, 1>() : dc_xf_fits<16, false, 1>();
      return bf ? dc_xf_fits<16, true, 2>() : dc_xf_fits<16, false, 2>();
    }
  }
}

void launch_dc_gemm(const void* dYc, const float* t, const float* colsum, float* part, float* dC,
                    DcOut om, const Plan& p, const BwdLayout& L, hipStream_t s,
                    const BasisXform* xf) {
  const bool bf = p.esz == 2;
#define CKAN_DC(PP, BB) dc_dispatch<PP, BB>(dYc, t, colsum, part, dC, om, p, L, s, xf)
  switch (p.P) {
    case 2: bf ? CKAN_DC(2, true) : CKAN_DC(2, false); break;
    case 4: bf ? CKAN_DC(4, true) : CKAN_DC(4, false); break;
    case 8: bf ? CKAN_DC(8, true) : CKAN_DC(8, false); break;
    default: bf ? CKAN_DC(16, true) : CKAN_DC(16, false); break;
  }
#undef CKAN_DC
}

bool fwd_tail_ce_ok(const Plan& pa, const FwdChoice& ca, int Ob, int Db) {
  return (ca.splits > 1 && !fwd_streaming(ca) && ca.tile != kFwdCols) && pa.O <= 64 && Ob >= 1 &&
         Ob <= kTailO && Db >= 1 && Db <= 17 && pa.O * Ob * Db <= kTailC && pa.B <= 4096;
}

void launch_fwd_tail_ce(const void* packed_a, void* ws, const Plan& pa, const FwdChoice& ca,
                        bool sum_bias, float* tb, const float* Cb, int Ob, int Db, float* yb,
                        const int64_t* labels, float* dyb, float* loss_part, hipStream_t s,
                        float* dxa) {
  char* pk = const_cast<char*>(reinterpret_cast<const char*>(packed_a));
  const float* bias = reinterpret_cast<const float*>(pk + packed_biasf_offset(pa));
  const float* bpart = reinterpret_cast<const float*>(pk + packed_bias_offset(pa));
  const int nib = sum_bias && fwd_sums_bias(pa, ca) ? pa.NIB : 0;
  float* bias_out = nib > 0 ? reinterpret_cast<float*>(pk + packed_biasf_offset(pa)) : nullptr;
  const unsigned grid = (unsigned)ceil_div(pa.B, kTailRows);
  const size_t lds = (size_t)pa.O * Ob * Db * sizeof(float);
  hipLaunchKernelGGL(k_fwd_tail_ce, dim3(grid), dim3(64 * kTailRows), lds, s,
                     reinterpret_cast<const float*>(ws), ca.splits, bias, pa, bpart, nib, bias_out,
                     tb, Cb, Ob, Db, yb, labels, dyb, loss_part, dxa, padded_degree(Db - 1));
}

}  // namespace ckan
