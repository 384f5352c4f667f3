// Shared definitions of the gfx950 ChebyKAN kernels: the layout plan, MFMA
// fragment helpers and the Chebyshev recurrences.
//
// Notation: B rows, I inputs, O outputs, deg the degree, D = deg + 1.
// The T_0 = 1 term of every contraction is handled apart from the MFMA work
// (as a per-output bias in the forward, a column sum of dy in dC, and it has
// no derivative), so the contractions run over T_1..T_P, where P is deg
// padded to 2, 4, 8 or 16 with zero coefficients.
//
// MFMA operand layout ("fragment-major").  One k-block is 16 reduction
// indices; for v_mfma_f32_32x32x16_bf16 a wave's operand fragment is 64 lanes
// x 8 values, lane l holding row/column (l % 32) and the 8 reduction slots of
// half g = l / 32.  The fp32 path runs the same k-block as 8
// v_mfma_f32_32x32x2_f32, value j of both halves feeding instruction j.
// Which reduction index sits in slot (g, j) is free as long as both operands
// agree, so every packed operand is stored as [frag row-block][k-block][lane][8],
// one contiguous 1 KiB (bf16) / 2 KiB (fp32) run per fragment: a wave loads a
// fragment with one fully coalesced 16 B (or 32 B) access per lane, and the
// LDS copy of a fragment is read back without bank conflicts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ckan {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4_t;

constexpr int kFragElems = 512;  // 64 lanes x 8 values
constexpr int kNumCUs = 256;      // MI355X: 8 XCDs x 32 compute units

__host__ __device__ constexpr int padded_degree(int deg) {
  return deg <= 2 ? 2 : deg <= 4 ? 4 : deg <= 8 ? 8 : deg <= 16 ? 16 : -1;
}

// Forward reduction grouping for padded degree P.  A "group" gives each lane
// half IPG/2 inputs x P degrees = 8*KBG values (KBG k-blocks); a
// "super-group" (SG) is 4 groups, SGI inputs, SGK k-blocks, so one lane reads
// 2*IPG consecutive tanh values per SG with vector loads.
template <int P> struct FwdGroup {
  static constexpr int IPG = 2 * (P < 8 ? 8 / P : 1);
  static constexpr int KBG = P > 8 ? P / 8 : 1;
  static constexpr int SGI = 4 * IPG;
  static constexpr int SGK = 4 * KBG;
  static constexpr int LANE_T = 2 * IPG;  // tanh values a lane reads per SG
};

__host__ __device__ inline int fwd_sgi(int P) { return 4 * 2 * (P < 8 ? 8 / P : 1); }
__host__ __device__ inline int fwd_sgk(int P) { return 4 * (P > 8 ? P / 8 : 1); }

inline int64_t round_up(int64_t a, int64_t b) { return (a + b - 1) / b * b; }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Batch rows per k-block stage of the dC reduction (4 k-blocks of 16 rows).
constexpr int kDcStageRows = 64;
// Output columns per k-block stage of the dX reduction.
constexpr int kDxStageCols = 64;
// Rows covered by one prep_dy wave (colsum partial granularity).
constexpr int kPrepRows = 64;

struct Plan {
  int64_t B;       // rows
  int I, O, deg, D, P;
  int SGI, SGK;    // forward super-group inputs / k-blocks
  int I_sg;        // I padded to SGI (tanh-cache row pitch, forward K inputs)
  int KB;          // forward k-blocks = I_sg * P / 16
  int O32, NBf;    // O padded to 32; forward N fragments
  int I32, NIB;    // I padded to 32; input blocks of 32
  int O64, KBx;    // O padded to 64; dX reduction k-blocks
  int64_t B32;     // rows padded to 32
  int64_t Bc, KBc; // rows padded to kDcStageRows; dC reduction k-blocks
  int NBB;         // prep_dy row blocks (colsum partials)
  int esz;         // bytes per packed operand element (2 bf16, 4 fp32)
  int imap;        // input map: 0 t = tanh(x), 1 t = ima * x + imb
  float ima, imb;
};

// The basis argument t of an input x, and dt/dx as a function of t.
__device__ __forceinline__ float input_map(float x, int imap, float a, float b) {
  return imap ? fmaf(a, x, b) : tanhf(x);
}
__device__ __forceinline__ float input_slope(float t, const Plan& p) {
  return p.imap ? p.ima : 1.0f - t * t;
}

// How the dC kernels write the finished gradient g into the destination d:
// store it, add it, or (for a caller that wants only the updated parameter,
// with d the parameter itself) apply the SGD step d -= lr * (g + wd * d) or
// an Adam step (moments m, v at the offset of d from base; the step's
// -lr / (1 - b1^t) and sqrt(1 - b2^t) read from sc[0], sc[1] on the device).
enum DcMode : int { kDcStore = 0, kDcAccumulate = 1, kDcSgd = 2, kDcAdam = 3 };
struct DcOut {
  int mode;
  float lr, wd;
  float w1, beta2, one_m_beta2, eps;  // Adam: w1 = 1 - beta1
  const float* base;
  float* m;
  float* v;
  const float* sc;
};

// A loss mean for a kernel that also takes it (the last launch of an executor
// step's loss, folded into the next launch): out = scale * sum_k part[k],
// k < n; also into out2 when given.  part == nullptr: none.
struct LossMean {
  const float* part;
  int64_t n;
  float scale;
  float* out;
  float* out2;
};

// The sum of LossMean by one block (256 threads or more; the first 256 do
// the work) in a fixed order: strided per-thread sums, then a tree
// (k_sum_scalar's order, so the same bits).
__device__ __forceinline__ void loss_mean_block(const LossMean& lm) {
  __shared__ float red[256];
  if (threadIdx.x < 256) {
    float s = 0.0f;
    for (int64_t k = threadIdx.x; k < lm.n; k += 256) s += lm.part[k];
    red[threadIdx.x] = s;
  }
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    *lm.out = red[0] * lm.scale;
    if (lm.out2) *lm.out2 = red[0] * lm.scale;
  }
}

// The SGD update of one parameter: the arithmetic of every SGD path here.
__device__ __forceinline__ float sgd_update(float p, float g, float lr, float wd) {
  float gv = g;
  if (wd != 0.0f) gv = gv + wd * p;
  return p - lr * gv;
}

// The Adam update of one parameter pv with gradient g and moments *m, *v
// (torch's single-tensor order of operations): the arithmetic of the
// executor's Adam paths.
__device__ __forceinline__ float adam_update(float pv, float g, float* m, float* v, float w1,
                                             float beta2, float one_m_beta2, float eps, float wd,
                                             float neg_step, float bc2_sqrt) {
  float gv = g;
  if (wd != 0.0f) gv = gv + wd * pv;
  float mv = *m;
  mv = (w1 < 0.5f) ? mv + w1 * (gv - mv) : gv - (gv - mv) * (1.0f - w1);
  float vv = *v * beta2;
  vv = vv + one_m_beta2 * gv * gv;
  const float denom = sqrtf(vv) / bc2_sqrt + eps;
  *m = mv;
  *v = vv;
  return pv + neg_step * (mv / denom);
}

// Writes g into d as the mode says, with old the value d holds (read ahead
// by the caller), and returns the value stored.
__device__ __forceinline__ float dc_apply_from(float* d, float old, float g, const DcOut& o) {
  float v;
  if (o.mode == kDcStore) {
    v = g;
  } else if (o.mode == kDcAccumulate) {
    v = old + g;
  } else if (o.mode == kDcSgd) {
    v = sgd_update(old, g, o.lr, o.wd);
  } else {
    const size_t q = (size_t)(d - o.base);
    v = adam_update(old, g, o.m + q, o.v + q, o.w1, o.beta2, o.one_m_beta2, o.eps, o.wd, o.sc[0],
                    o.sc[1]);
  }
  *d = v;
  return v;
}

__device__ __forceinline__ void dc_write(float* d, float g, const DcOut& o) {
  if (o.mode == kDcStore) {
    *d = g;
  } else if (o.mode == kDcAccumulate) {
    *d = *d + g;
  } else if (o.mode == kDcSgd) {
    *d = sgd_update(*d, g, o.lr, o.wd);
  } else {
    const size_t q = (size_t)(d - o.base);
    *d = adam_update(*d, g, o.m + q, o.v + q, o.w1, o.beta2, o.one_m_beta2, o.eps, o.wd, o.sc[0],
                     o.sc[1]);
  }
}

__device__ __forceinline__ void dc_write4(f32x4_t* d, f32x4_t g, const DcOut& o) {
  if (o.mode == kDcStore) {
    __builtin_nontemporal_store(g, d);
  } else if (o.mode == kDcAdam) {
    float* e = reinterpret_cast<float*>(d);
    dc_write(e, g.x, o);
    dc_write(e + 1, g.y, o);
    dc_write(e + 2, g.z, o);
    dc_write(e + 3, g.w, o);
  } else {
    f32x4_t v = *d;
    if (o.mode == kDcAccumulate) {
      v = v + g;
    } else {
      v.x = sgd_update(v.x, g.x, o.lr, o.wd);
      v.y = sgd_update(v.y, g.y, o.lr, o.wd);
      v.z = sgd_update(v.z, g.z, o.lr, o.wd);
      v.w = sgd_update(v.w, g.w, o.lr, o.wd);
    }
    *d = v;
  }
}

inline Plan make_plan(int64_t B, int I, int O, int deg, bool bf16) {
  Plan p;
  p.B = B; p.I = I; p.O = O; p.deg = deg; p.D = deg + 1;
  p.P = padded_degree(deg);
  p.SGI = fwd_sgi(p.P);
  p.SGK = fwd_sgk(p.P);
  p.I_sg = (int)round_up(I, p.SGI);
  p.KB = p.I_sg * p.P / 16;
  p.O32 = (int)round_up(O, 32);
  p.NBf = p.O32 / 32;
  p.I32 = (int)round_up(I, 32);
  p.NIB = p.I32 / 32;
  p.O64 = (int)round_up(O, kDxStageCols);
  p.KBx = p.O64 / 16;
  p.B32 = round_up(B, 32);
  p.Bc = round_up(B, kDcStageRows);
  p.KBc = p.Bc / 16;
  p.NBB = (int)ceil_div(B, kPrepRows);
  p.esz = bf16 ? 2 : 4;
  p.imap = 0;
  p.ima = p.imb = 0.0f;
  return p;
}

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

template <bool BF> struct Elem;
template <> struct Elem<true> { typedef uint16_t type; };
template <> struct Elem<false> { typedef float type; };

// One lane's share of an MFMA operand fragment for one k-block.
template <bool BF> struct Frag;
template <> struct Frag<true> { bf16x8_t v; };
template <> struct Frag<false> { f32x4_t lo, hi; };

__device__ __forceinline__ Frag<true> make_frag_bf(const float* v) {
  Frag<true> f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f.v[j] = (__bf16)v[j];  // v_cvt_pk_bf16_f32, RNE
  return f;
}

template <bool BF> __device__ __forceinline__ Frag<BF> make_frag(const float* v);
template <> __device__ __forceinline__ Frag<true> make_frag<true>(const float* v) {
  return make_frag_bf(v);
}
template <> __device__ __forceinline__ Frag<false> make_frag<false>(const float* v) {
  Frag<false> f;
  f.lo = f32x4_t{v[0], v[1], v[2], v[3]};
  f.hi = f32x4_t{v[4], v[5], v[6], v[7]};
  return f;
}

// The bf16 forward coefficients (Cf) are stored by 8-output streams: for a
// 32-output fragment column nb, stream (nb, sub) holds columns 8 sub .. 8 sub
// + 7 of every k-block kb in order, each k-block as its first half (k 0-7)
// then its second (k 8-15), 16 bytes per column.  Lane L of fragment (nb, kb)
// (column L % 32, half L / 32) finds its 8 values at this element offset.  A
// reader of a few columns (the small-batch forward) then streams contiguous
// bytes; the GEMMs copy each lane's 16 bytes from here instead of from
// fragment-contiguous storage.  fp32 fragments stay fragment-contiguous.
__host__ __device__ inline size_t cf_bf16_elem(int KB, int nb, int kb, int L) {
  const int ol = L & 31, g = L >> 5;
  return ((((size_t)nb * 4 + (ol >> 3)) * KB + kb) * 2 + g) * 64 + (size_t)(ol & 7) * 8;
}
// Element offset of lane L's 8 values of forward fragment (nb, kb).
template <bool BF> __host__ __device__ inline size_t cf_elem(int KB, int nb, int kb, int L) {
  if constexpr (BF) return cf_bf16_elem(KB, nb, kb, L);
  else return ((size_t)nb * KB + kb) * kFragElems + (size_t)L * 8;
}

// Load this lane's 8 values of a fragment stored at `base` (fragment start).
template <bool BF> __device__ __forceinline__ Frag<BF> load_frag(const typename Elem<BF>::type* base, int lane);
template <> __device__ __forceinline__ Frag<true> load_frag<true>(const uint16_t* base, int lane) {
  Frag<true> f;
  f.v = *reinterpret_cast<const bf16x8_t*>(base + lane * 8);
  return f;
}
template <> __device__ __forceinline__ Frag<false> load_frag<false>(const float* base, int lane) {
  Frag<false> f;
  const f32x4_t* p = reinterpret_cast<const f32x4_t*>(base + lane * 8);
  f.lo = p[0];
  f.hi = p[1];
  return f;
}

// Non-temporal fragment load, for operands a launch streams once (the
// coefficient stream of the small-batch forwards): marked for early eviction
// they leave the caches to the data that is reused (config 5 at B = 1:
// 14.1 -> 13.2 us cold).  Outputs nothing in the same step reads again (y,
// dx, dC) are stored non-temporally for the same reason.
template <bool BF> __device__ __forceinline__ Frag<BF> load_frag_nt(const typename Elem<BF>::type* base, int lane);
template <> __device__ __forceinline__ Frag<true> load_frag_nt<true>(const uint16_t* base, int lane) {
  Frag<true> f;
  f.v = __builtin_nontemporal_load(reinterpret_cast<const bf16x8_t*>(base + lane * 8));
  return f;
}
template <> __device__ __forceinline__ Frag<false> load_frag_nt<false>(const float* base, int lane) {
  Frag<false> f;
  const f32x4_t* p = reinterpret_cast<const f32x4_t*>(base + lane * 8);
  f.lo = __builtin_nontemporal_load(p);
  f.hi = __builtin_nontemporal_load(p + 1);
  return f;
}

template <bool BF> __device__ __forceinline__ Frag<BF> zero_frag();
template <> __device__ __forceinline__ Frag<true> zero_frag<true>() {
  Frag<true> f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f.v[j] = (__bf16)0.0f;
  return f;
}
template <> __device__ __forceinline__ Frag<false> zero_frag<false>() {
  Frag<false> f;
  f.lo = f32x4_t{0.f, 0.f, 0.f, 0.f};
  f.hi = f.lo;
  return f;
}

// Store 8 values as this lane's share of a fragment at `base`.
template <bool BF> __device__ __forceinline__ void store_frag(typename Elem<BF>::type* base, int lane, const float* v);
template <> __device__ __forceinline__ void store_frag<true>(uint16_t* base, int lane, const float* v) {
  Frag<true> f = make_frag_bf(v);
  *reinterpret_cast<bf16x8_t*>(base + lane * 8) = f.v;
}
template <> __device__ __forceinline__ void store_frag<false>(float* base, int lane, const float* v) {
  f32x4_t* p = reinterpret_cast<f32x4_t*>(base + lane * 8);
  p[0] = f32x4_t{v[0], v[1], v[2], v[3]};
  p[1] = f32x4_t{v[4], v[5], v[6], v[7]};
}

// acc[32x32] += A_frag(k-block) * B_frag(k-block)
__device__ __forceinline__ void mma(f32x16_t& acc, const Frag<true>& a, const Frag<true>& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x16_t& acc, const Frag<false>& a, const Frag<false>& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.lo[0], b.lo[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.lo[1], b.lo[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.lo[2], b.lo[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.lo[3], b.lo[3], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.hi[0], b.hi[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.hi[1], b.hi[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.hi[2], b.hi[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.hi[3], b.hi[3], acc, 0, 0, 0);
}

// ---- pipeline primitives ----------------------------------------------------
// Wait until at most N vector-memory operations of this wave are in flight
// (gfx9 s_waitcnt encoding: vmcnt[3:0] | vmcnt[5:4] << 14; expcnt and lgkmcnt
// left at their maxima so only vmcnt is waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Wait until at most N LDS/scalar-memory operations are in flight.
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt is a 4-bit field");
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (N << 8));
}
// Workgroup execution barrier without the memory fence of __syncthreads():
// in-flight prefetches stay in flight.  The empty asm keeps the compiler
// from moving LDS accesses across it.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// One 16-byte-per-lane global -> LDS copy (global_load_lds_dwordx4): lane l's
// 16 bytes from `src` land at lds_base + 16 * l.  `lds_base` must be
// wave-uniform.
__device__ __forceinline__ void dma16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}
// The same copy in saddr form, for pipelined loops: lane l's 16 bytes at
// sbase + voff land at LDS byte lds + 16 * l, with sbase and lds wave-uniform
// (SGPRs) and voff a per-lane 32-bit offset.  Two measured reasons for the
// inline assembly:
//  * the compiler counts an LDS-DMA instruction as an LGKM event of another
//    kind than ds_read and then waits with lgkmcnt(0) at every LDS read of a
//    loop that contains one, which serialises each prefetched fragment read;
//    the hardware counts these copies only in vmcnt (an lgkmcnt(0) right
//    after one returns at once), so the copies are hidden from the compiler
//    and the loops wait for them with explicit vmcnt waits;
//  * vector-ALU address work for a copy (64-bit adds, readfirstlane of the
//    LDS address) issues slowly while another wave of the SIMD streams MFMAs
//    (copy rate fell from ~58 to ~7 B/clk per CU); here issuing is SALU only.
// Callers keep voff + sbase inside the source allocation and pass sbase and
// lds wave-uniform; readfirstlane only moves them to SGPRs where the compiler
// cannot prove that (it folds away for values it knows are uniform).
//
// A vector memory instruction that reads an SGPR written by a VALU
// instruction (v_readfirstlane here) needs 5 wait states in between on this
// GPU generation, or it reads the SGPR's previous contents.  The compiler's
// hazard pass does not look inside inline assembly, so dma16s supplies the 5
// itself (s_mov counts as one, s_nop N as N + 1).
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds) {
  const uint64_t a = (uint64_t)(uintptr_t)sbase;
  const uint64_t s = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t l = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 3\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(s), "s"(l) : "memory", "m0");
}
// dma16s for a base and LDS address that the kernel computes with scalar
// instructions only (kernel arguments, loop counters, readfirstlane results
// made well before the loop): no VALU writes them, so the copy waits only the
// one state M0 needs.  tests/test_isa_hazards.py checks the compiled kernels
// for any vector memory read of an SGPR fewer than 5 states after a VALU
// write.
__device__ __forceinline__ void dma16s_salu(const void* sbase, uint32_t voff, uint32_t lds) {
  const uint64_t a = (uint64_t)(uintptr_t)sbase;
  const uint64_t s = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t l = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(s), "s"(l) : "memory", "m0");
}

// Word 3 of a raw buffer descriptor on gfx9 parts (32-bit data format, no
// swizzle); the descriptor's size field bounds-checks each access, and
// stores past it are dropped.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy bits of a buffer access marked non-temporal (gfx940+ "nt").
constexpr int kBufferNonTemporal = 2;
// A raw buffer descriptor for `bytes` bytes from `base`.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufferWord3);
}
// Non-temporal store of one float at byte offset voff + soff of a buffer
// (the builtin takes the data as an unsigned int: the bits, not the value).
__device__ __forceinline__ void buffer_store_f32_nt(float v, __amdgpu_buffer_rsrc_t rs, int voff, int soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rs, voff, soff, kBufferNonTemporal);
}

// Makes a wave-uniform value (a kernel argument) live in SGPRs from here on.
// Without it the compiler may issue the scalar load of an argument that is
// only used after a pipelined loop right before that loop; a scalar load in
// flight turns every LDS wait inside the loop into lgkmcnt(0), since scalar
// loads may complete out of order.
template <typename T>
__device__ __forceinline__ void pin_sgpr(T v) {
  asm volatile("" ::"s"(v));
}

// The bias sum_i C[i, o, 0] from nparts per-input-block partials
// part[k * pitch + o], in k_col_reduce's order: four running sums over
// k = 0, 1, 2, 3 (mod 4), then ((s0 + s1) + s2) + s3.  Every kernel that sums
// the partials itself uses this, so its bias has the bits of the reduction
// launch it replaces.
__device__ __forceinline__ float bias_from_parts(const float* __restrict__ part, int nparts,
                                                 int pitch, int o) {
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
  int k = 0;
  for (; k + 4 <= nparts; k += 4) {
    s0 += part[(size_t)k * pitch + o];
    s1 += part[(size_t)(k + 1) * pitch + o];
    s2 += part[(size_t)(k + 2) * pitch + o];
    s3 += part[(size_t)(k + 3) * pitch + o];
  }
  if (k < nparts) s0 += part[(size_t)k * pitch + o];
  if (k + 1 < nparts) s1 += part[(size_t)(k + 1) * pitch + o];
  if (k + 2 < nparts) s2 += part[(size_t)(k + 2) * pitch + o];
  return ((s0 + s1) + s2) + s3;
}

// Row of accumulator value v (0..15) for lane half g in a 32x32 MFMA result;
// the column is lane % 32.
__device__ __forceinline__ int acc_row(int v, int g) { return 8 * (v >> 2) + 4 * g + (v & 3); }

// T_1..T_P of t by the three-term recurrence T_{n+1} = 2 t T_n - T_{n-1}.
template <int P>
__device__ __forceinline__ void cheb_T(float t, float* out) {
  const float t2 = t + t;
  float a = 1.0f, b = t;
  out[0] = t;
#pragma unroll
  for (int d = 1; d < P; ++d) {
    const float c = fmaf(t2, b, -a);
    out[d] = c;
    a = b;
    b = c;
  }
}

}  // namespace ckan
