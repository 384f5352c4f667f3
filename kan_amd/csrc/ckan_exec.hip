// Resident multi-layer executor: a KANSequential of ChebyKAN layers trained in
// place on one GPU (include/chebykan.h, ckan_exec_*).  All device memory is
// allocated once at creation; a training step is a fixed sequence of launches
// (pack, forward per layer, fused loss + gradient, backward per layer,
// optimizer) on one stream, optionally captured once into a HIP graph and
// replayed.  The Adam step count lives on the device, so replays stay exact.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "chebykan.h"
#include "ckan_kernels.hpp"

using namespace ckan;

namespace {

constexpr int kLossBlocks = 256;  // fixed partial count: deterministic loss sums

// MSE (torch.nn.MSELoss, reduction='mean'): loss = sum (y - t)^2 / N,
// dy = 2 (y - t) / N.  Grid-stride over N elements with a fixed grid; each
// block writes one partial sum.
__global__ void __launch_bounds__(256)
k_mse(const float* __restrict__ y, const float* __restrict__ tgt, float* __restrict__ dy,
      int64_t n, float scale_grad, float* __restrict__ part, int vec) {
  __shared__ float red[256];
  float s = 0.0f;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (vec) {
    // float4 strides, four of them loaded before any is used (one element
    // per round trip made config 4's 4 M-element loss latency-bound: 31 us)
    constexpr int U = 4;
    const int64_t n4 = n / 4;
    const f32x4_t* y4 = reinterpret_cast<const f32x4_t*>(y);
    const f32x4_t* t4 = reinterpret_cast<const f32x4_t*>(tgt);
    f32x4_t* d4 = reinterpret_cast<f32x4_t*>(dy);
    for (int64_t q0 = t0; q0 < n4; q0 += U * stride) {
      f32x4_t a[U], b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t q = q0 + u * stride;
        a[u] = q < n4 ? __builtin_nontemporal_load(y4 + q) : f32x4_t{0.f, 0.f, 0.f, 0.f};
        b[u] = q < n4 ? __builtin_nontemporal_load(t4 + q) : f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t q = q0 + u * stride;
        const f32x4_t d = a[u] - b[u];
#pragma unroll
        for (int j = 0; j < 4; ++j) s = fmaf(d[j], d[j], s);
        if (q < n4) d4[q] = scale_grad * d;
      }
    }
  } else {
    for (int64_t q = t0; q < n; q += stride) {
      const float d = y[q] - tgt[q];
      s = fmaf(d, d, s);
      dy[q] = scale_grad * d;
    }
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

// Softmax cross-entropy (torch.nn.CrossEntropyLoss, reduction='mean') on
// logits y [B, O] and int64 labels: one wave per row; the row loss
// logsumexp(y) - y[label] goes to row_loss[b], dy = (softmax(y) - onehot) / B.
__global__ void __launch_bounds__(256)
k_ce(const float* __restrict__ y, const int64_t* __restrict__ labels, float* __restrict__ dy,
     int64_t B, int O, float* __restrict__ row_loss) {
  const int lane = threadIdx.x & 63;
  const int64_t b = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= B) return;
  const float* yr = y + b * O;
  float m = -INFINITY;
  for (int o = lane; o < O; o += 64) m = fmaxf(m, yr[o]);
#pragma unroll
  for (int w = 32; w > 0; w >>= 1) m = fmaxf(m, __shfl_xor(m, w));
  float s = 0.0f;
  for (int o = lane; o < O; o += 64) s += expf(yr[o] - m);
#pragma unroll
  for (int w = 32; w > 0; w >>= 1) s += __shfl_xor(s, w);
  const int64_t lab = labels[b];
  const float inv_b = 1.0f / (float)B;
  for (int o = lane; o < O; o += 64) {
    const float pr = expf(yr[o] - m) / s;
    dy[b * O + o] = (pr - (o == lab ? 1.0f : 0.0f)) * inv_b;
  }
  if (lane == 0) {
    const float yl = (lab >= 0 && lab < O) ? yr[lab] : 0.0f;
    row_loss[b] = (logf(s) + m) - yl;
  }
}

// Softmax cross-entropy and its mean in one launch, for up to 1024 rows of
// at most 16 classes (config 2's 10): thread b owns row b.  The row's max and
// exp-sum are formed in k_ce's order (its lane butterfly, with the lanes past
// O adding exact zeros), and the row losses are summed in k_sum_scalar's
// order, so dy and the loss have the bits of the two-launch path.
constexpr int kCeSmallRows = 1024, kCeSmallO = 16;
__global__ void __launch_bounds__(1024)
k_ce_small(const float* __restrict__ y, const int64_t* __restrict__ labels, float* __restrict__ dy,
           int B, int O, float* __restrict__ out, float* __restrict__ out2) {
  __shared__ float rl[kCeSmallRows];
  __shared__ float red[256];
  const int b = threadIdx.x;
  if (b < B) {
    const float* yr = y + (int64_t)b * O;
    float yv[kCeSmallO], e[kCeSmallO];
#pragma unroll
    for (int o = 0; o < kCeSmallO; ++o) yv[o] = o < O ? yr[o] : 0.0f;
    float m = -INFINITY;
#pragma unroll
    for (int o = 0; o < kCeSmallO; ++o)
      if (o < O) m = fmaxf(m, yv[o]);
#pragma unroll
    for (int o = 0; o < kCeSmallO; ++o) e[o] = o < O ? expf(yv[o] - m) : 0.0f;
#pragma unroll
    for (int w = kCeSmallO / 2; w > 0; w >>= 1)
#pragma unroll
      for (int o = 0; o < w; ++o) e[o] = e[o] + e[o + w];
    const float s = e[0];
    const int64_t lab = labels[b];
    const float inv_b = 1.0f / (float)B;
#pragma unroll
    for (int o = 0; o < kCeSmallO; ++o)
      if (o < O) dy[(int64_t)b * O + o] = (expf(yv[o] - m) / s - (o == lab ? 1.0f : 0.0f)) * inv_b;
    const float yl = (lab >= 0 && lab < O) ? yr[lab] : 0.0f;
    rl[b] = (logf(s) + m) - yl;
  }
  __syncthreads();
  if (b < 256) {
    float acc = 0.0f;
    for (int k = b; k < B; k += 256) acc += rl[k];
    red[b] = acc;
  }
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (b < w) red[b] += red[b + w];
    __syncthreads();
  }
  if (b == 0) {
    const float scale = (float)(1.0 / (double)B);
    *out = red[0] * scale;
    if (out2) *out2 = red[0] * scale;
  }
}

// loss = scale * sum_k part[k], k < n, in a fixed order (one block); also
// into out2 when given (the caller's per-step loss slot).
__global__ void __launch_bounds__(256)
k_sum_scalar(const float* __restrict__ part, int64_t n, float scale, float* __restrict__ out,
             float* __restrict__ out2) {
  loss_mean_block(LossMean{part, n, scale, out, out2});
}

// Adam scalars for the next step from the device step counter (one thread):
// step += 1; sc[0] = -lr / (1 - b1^step); sc[1] = sqrt(1 - b2^step), in double
// as torch computes them, then rounded to fp32.
__global__ void k_adam_scalars(int64_t* __restrict__ step, double lr, double b1, double b2,
                               float* __restrict__ sc) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const int64_t s = *step + 1;
    *step = s;
    sc[0] = (float)(-(lr / (1.0 - pow(b1, (double)s))));
    sc[1] = (float)sqrt(1.0 - pow(b2, (double)s));
  }
}

__global__ void __launch_bounds__(256)
k_copy_f32(const float* __restrict__ src, float* __restrict__ dst, int64_t n) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * blockDim.x)
    dst[q] = src[q];
}

// ---------------------------------------------------------------------------
// Small stacks: one training step in one workgroup.  For a network whose whole
// step is a few hundred thousand multiply-adds (config 1, the README loop,
// is 1.8 thousand), the multi-kernel step costs ~10 launches of a few us
// each while the arithmetic takes well under a microsecond.  k_tiny_step runs
// the same step in one launch: tanh and the Chebyshev recurrence in fp32, the
// contractions as fixed-order fp32 sums (with the bf16 compute mode's operand
// rounding: basis values, coefficients and dy of the d >= 1 terms rounded to
// bf16, the T_0 terms kept in fp32, as the MFMA path does), the loss and its
// gradient, then per layer from the last: dx (with the coefficients before
// their update), dC and the SGD / Adam update.  All reductions are in a fixed
// order, so steps are bitwise reproducible.
// ---------------------------------------------------------------------------
constexpr int kTinyMaxLayers = 8;
constexpr int kTinyMaxD = 17;
constexpr int64_t kTinyMaxMacs = (int64_t)1 << 18;  // multiply-adds per step
constexpr int kTinyStepsPerLaunch = 1024;  // fit's steps per launch (bounds a launch's duration)

struct TinyLayerArg {
  float* C;
  float* m;
  float* v;
  float* t;   // tanh of the layer input [B, I]
  float* y;   // layer output [B, O]
  float* dy;  // gradient wrt y [B, O]
  int I, O, D;
  // float offsets of the same arrays in the launch's LDS (TinyArgs::lds)
  int sC, sm, sv, st, sy, sdy;
};

struct TinyArgs {
  TinyLayerArg L[kTinyMaxLayers];
  int nl;
  int loss;
  int opt;
  int bf16;
  int64_t B;
  float lr, wd, w1, beta2, one_m_beta2, eps;
  double lr_d, b1_d, b2_d;
  // the whole state (coefficients, moments, activations) fits in LDS: the
  // launch copies the coefficients and moments in, runs its steps there and
  // copies them back, so a step's phases pass no data through memory
  int lds, lds_floats;
};
constexpr int kTinyLdsFloats = 12 * 1024;  // 48 KiB of dynamic LDS

// Layer l with its arrays in LDS when the launch keeps the state there.
__device__ __forceinline__ TinyLayerArg tiny_layer(const TinyArgs& a, float* st, int l) {
  TinyLayerArg ly = a.L[l];
  if (a.lds) {
    ly.C = st + ly.sC;
    ly.m = st + ly.sm;
    ly.v = st + ly.sv;
    ly.t = st + ly.st;
    ly.y = st + ly.sy;
    ly.dy = st + ly.sdy;
  }
  return ly;
}

__device__ __forceinline__ float tiny_round(float v, int bf) { return bf ? (float)(__bf16)v : v; }

// Sum of red[0..n) (n a power of two, every thread of the block calls it) by a
// fixed tree; the result is returned to every thread.
__device__ float tiny_block_sum(float* red, float v) {
  const int tid = threadIdx.x;
  red[tid] = v;
  __syncthreads();
  for (int w = blockDim.x >> 1; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

// nsteps steps on the same x / target (the executor's fit), one after the
// other in this one workgroup: step k's loss also goes to losses[k] when given.
// A barrier ends each layer's update, so the next step reads the new
// coefficients.
__global__ void __launch_bounds__(1024)
k_tiny_step(TinyArgs a, const float* __restrict__ x, const void* __restrict__ target,
            int64_t* __restrict__ step, float* __restrict__ loss, float* __restrict__ losses,
            int nsteps) {
  __shared__ float red[1024];
  __shared__ float scs[kTinyStepsPerLaunch][2];
  extern __shared__ float st_lds[];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t B = a.B;
  const int bf = a.bf16;
  auto move_state = [&](bool in) {  // coefficients and moments, global <-> LDS
    for (int l = 0; l < a.nl; ++l) {
      const TinyLayerArg g = a.L[l];
      const int64_t n = (int64_t)g.I * g.O * g.D;
      const bool adam = a.opt == CKAN_OPT_ADAM;
      for (int64_t q = tid; q < n; q += nt) {
        if (in) {
          st_lds[g.sC + q] = g.C[q];
          if (adam) {
            st_lds[g.sm + q] = g.m[q];
            st_lds[g.sv + q] = g.v[q];
          }
        } else {
          g.C[q] = st_lds[g.sC + q];
          if (adam) {
            g.m[q] = st_lds[g.sm + q];
            g.v[q] = st_lds[g.sv + q];
          }
        }
      }
    }
    __syncthreads();
  };
  if (a.lds) move_state(true);
  if (a.opt == CKAN_OPT_ADAM) {
    // every step's Adam scalars up front, one step per thread (as
    // k_adam_scalars, in double from the device step count): a pow per step
    // on one thread would hold every step's barrier
    const int64_t s0 = *step;
    for (int k = tid; k < nsteps; k += nt) {
      const double s1 = (double)(s0 + k + 1);
      scs[k][0] = (float)(-(a.lr_d / (1.0 - pow(a.b1_d, s1))));
      scs[k][1] = (float)sqrt(1.0 - pow(a.b2_d, s1));
    }
    __syncthreads();  // every thread has read the count
    if (tid == 0) *step = s0 + nsteps;
  }
  for (int ks = 0; ks < nsteps; ++ks) {
  const float* sc = scs[ks];

  // ---- forward: t = tanh(in); y = sum_i C[i,o,0] + sum_{i,d>=1} T_d(t) C[i,o,d]
  const float* in = x;
  for (int l = 0; l < a.nl; ++l) {
    const TinyLayerArg ly = tiny_layer(a, st_lds, l);
    const int I = ly.I, O = ly.O, D = ly.D;
    for (int64_t q = tid; q < B * I; q += nt) ly.t[q] = tanhf(in[q]);
    __syncthreads();
    for (int64_t q = tid; q < B * O; q += nt) {
      const int64_t b = q / O;
      const int o = (int)(q - b * O);
      const float* tb = ly.t + b * I;
      float acc = 0.0f, bias = 0.0f;
      for (int i = 0; i < I; ++i) {
        const float* c = ly.C + ((size_t)i * O + o) * D;
        const float tv = tb[i], t2 = tv + tv;
        bias += c[0];
        float tm = 1.0f, tc = tv;
        for (int d = 1; d < D; ++d) {
          acc = fmaf(tiny_round(tc, bf), tiny_round(c[d], bf), acc);
          const float tn = fmaf(t2, tc, -tm);
          tm = tc;
          tc = tn;
        }
      }
      ly.y[q] = acc + bias;
    }
    __syncthreads();
    in = ly.y;
  }

  // ---- loss and its gradient (mean reduction)
  const TinyLayerArg last = tiny_layer(a, st_lds, a.nl - 1);
  const int O = last.O;
  float part = 0.0f;
  if (a.loss == CKAN_LOSS_MSE) {
    const int64_t n = B * O;
    const float gs = (float)(2.0 / (double)n);
    const float* tgt = reinterpret_cast<const float*>(target);
    for (int64_t q = tid; q < n; q += nt) {
      const float d = last.y[q] - tgt[q];
      part = fmaf(d, d, part);
      last.dy[q] = gs * d;
    }
    part = tiny_block_sum(red, part) * (float)(1.0 / (double)n);
  } else {
    const int64_t* lab = reinterpret_cast<const int64_t*>(target);
    const float inv_b = 1.0f / (float)B;
    for (int64_t b = tid; b < B; b += nt) {
      const float* yr = last.y + b * O;
      float m = -INFINITY;
      for (int o = 0; o < O; ++o) m = fmaxf(m, yr[o]);
      float s = 0.0f;
      for (int o = 0; o < O; ++o) s += expf(yr[o] - m);
      const int64_t lb = lab[b];
      for (int o = 0; o < O; ++o)
        last.dy[b * O + o] = (expf(yr[o] - m) / s - (o == lb ? 1.0f : 0.0f)) * inv_b;
      part += (logf(s) + m) - ((lb >= 0 && lb < O) ? yr[lb] : 0.0f);
    }
    part = tiny_block_sum(red, part) * (float)(1.0 / (double)B);
  }
  if (tid == 0) {
    *loss = part;
    if (losses) losses[ks] = part;
  }
  __syncthreads();

  // ---- backward and the optimizer, last layer first
  for (int l = a.nl - 1; l >= 0; --l) {
    const TinyLayerArg ly = tiny_layer(a, st_lds, l);
    const int I = ly.I, Ol = ly.O, D = ly.D;
    if (l > 0) {
      // dx[b,i] = (1 - t^2) sum_d U_{d-1}(t) sum_o dy[b,o] d C[i,o,d]
      float* dx = tiny_layer(a, st_lds, l - 1).dy;
      for (int64_t q = tid; q < B * I; q += nt) {
        const int64_t b = q / I;
        const int i = (int)(q - b * I);
        const float tv = ly.t[q], t2 = tv + tv;
        float dt[kTinyMaxD];
#pragma unroll
        for (int d = 0; d < kTinyMaxD; ++d) dt[d] = 0.0f;
        for (int o = 0; o < Ol; ++o) {
          const float g = tiny_round(ly.dy[b * Ol + o], bf);
          const float* c = ly.C + ((size_t)i * Ol + o) * D;
#pragma unroll
          for (int d = 1; d < kTinyMaxD; ++d)
            if (d < D) dt[d] = fmaf(g, tiny_round(c[d] * (float)d, bf), dt[d]);
        }
        float sum = 0.0f, up = 0.0f, u = 1.0f;  // U_{-1}, U_0
#pragma unroll
        for (int d = 1; d < kTinyMaxD; ++d) {
          if (d < D) sum = fmaf(dt[d], u, sum);
          const float un = fmaf(t2, u, -up);
          up = u;
          u = un;
        }
        dx[q] = sum * (1.0f - tv * tv);
      }
      __syncthreads();  // dx used the coefficients before their update
    }
    // dC[i,o,0] = sum_b dy[b,o]; dC[i,o,d] = sum_b T_d(t[b,i]) dy[b,o], one wave per
    // (i, o): lane k sums rows k, k + 64, ..., then a fixed butterfly over the
    // lanes; lane d < D then applies the update of coefficient d
    const int lane = tid & 63, wv = tid >> 6, nwv = nt >> 6;
    for (int64_t q = wv; q < (int64_t)I * Ol; q += nwv) {
      const int i = (int)(q / Ol), o = (int)(q - (int64_t)i * Ol);
      float g[kTinyMaxD];
#pragma unroll
      for (int d = 0; d < kTinyMaxD; ++d) g[d] = 0.0f;
      for (int64_t b = lane; b < B; b += 64) {
        const float dyv = ly.dy[b * Ol + o], dyr = tiny_round(dyv, bf);
        const float tv = ly.t[b * I + i], t2 = tv + tv;
        g[0] += dyv;
        float tm = 1.0f, tc = tv;
#pragma unroll
        for (int d = 1; d < kTinyMaxD; ++d) {
          if (d < D) g[d] = fmaf(tiny_round(tc, bf), dyr, g[d]);
          const float tn = fmaf(t2, tc, -tm);
          tm = tc;
          tc = tn;
        }
      }
#pragma unroll
      for (int w = 32; w > 0; w >>= 1)
#pragma unroll
        for (int d = 0; d < kTinyMaxD; ++d) g[d] += __shfl_xor(g[d], w);
      float gd = 0.0f;  // this lane's coefficient gradient (lane < D)
#pragma unroll
      for (int d = 0; d < kTinyMaxD; ++d) gd = lane == d ? g[d] : gd;
      if (lane < D) {
        const size_t k = (size_t)q * D + lane;
        float* c = ly.C + k;
        if (a.opt == CKAN_OPT_SGD) {
          *c = sgd_update(*c, gd, a.lr, a.wd);
        } else {
          *c = adam_update(*c, gd, ly.m + k, ly.v + k, a.w1, a.beta2, a.one_m_beta2, a.eps,
                           a.wd, sc[0], sc[1]);
        }
      }
    }
    __syncthreads();
  }
  }  // steps
  if (a.lds) move_state(false);
}

int grid_of(int64_t n) {
  int64_t g = (n + 255) / 256;
  return (int)(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

}  // namespace

struct ckan_exec {
  struct Layer {
    ckan_desc desc;
    int64_t ncoef;
    float* C = nullptr;     // fp32 master [I, O, D]
    float* m = nullptr;     // Adam moments
    float* v = nullptr;
    void* packed = nullptr;
    float* t = nullptr;     // tanh cache
    float* y = nullptr;     // activation out [B, O]
    float* dy = nullptr;    // gradient wrt y  [B, O]
    size_t packed_bytes = 0;
    // the training step's forward stores tanh(y) straight into the next
    // layer's tanh cache (y itself is not needed by the step)
    bool tanh_out = false;
    // this layer's pack and the next layer's run as one launch (the next
    // layer's input comes from this one's tanh output)
    bool pack_pair = false;
    // with pack_pair on the last two layers of a cross-entropy stack: the
    // second layer's forward and the loss gradient run in one tail launch
    bool tail_ce = false;
    // A Jacobi / Hermite layer (P_n(scale t) in place of T_n(t)).  Up to
    // kMfmaMaxDegree its pack multiplies C by the change of basis M into
    // Chebyshev coefficients C' = C M; its dC kernels then produce dC', and one
    // more launch forms dC = dC' M^T and applies the optimizer step to C.
    // Above it the vector-ALU backward differentiates in the family's basis
    // and applies the step itself, as for a Chebyshev layer.
    bool family = false;
    ckan_basis_spec spec{};
    BasisXform xf{};
  };
  ckan_exec_config cfg;
  std::vector<int32_t> widths, degrees;
  std::vector<Layer> layers;
  void* fws = nullptr;
  size_t fws_bytes = 0;
  void* bws = nullptr;
  size_t bws_bytes = 0;
  float* loss_part = nullptr;  // max(kLossBlocks, B) partials
  float* gcheb = nullptr;      // dC' of the family layers on the MFMA path
  float* loss = nullptr;
  int64_t* step = nullptr;     // Adam step count (device)
  float* adam_sc = nullptr;    // Adam scalars (device)
  bool tiny = false;           // the whole step runs as one k_tiny_step launch
  // A two-layer cross-entropy stack whose packed operands are kept current by
  // the step's dC launch (self_pack_pair_fits): the step runs no pack, and
  // every other change of C (creation, ckan_exec_set_coeffs) packs at once.
  // Layer 0's dX operand is not kept (the first layer has no dX).
  bool self_pack = false;
  // graph mode
  hipStream_t es = nullptr;
  hipEvent_t ev_in = nullptr, ev_out = nullptr;
  hipGraphExec_t graph = nullptr;         // captured on the executor-owned input buffers
  hipGraphExec_t graph_direct = nullptr;  // captured on the caller's x / target (gd_x, gd_t)
  const void* gd_x = nullptr;
  const void* gd_t = nullptr;
  const void* last_x = nullptr;           // the previous step's input pointers
  const void* last_t = nullptr;
  float* x_own = nullptr;
  void* tgt_own = nullptr;
  size_t tgt_bytes = 0;
  std::vector<void*> allocs;
};

namespace {

int efail(int code, const char* msg) {
  set_last_error(msg);
  return code;
}

int dev_alloc(ckan_exec* ex, void** p, size_t bytes) {
  if (bytes == 0) bytes = 256;
  if (hipMalloc(p, bytes) != hipSuccess) return efail(CKAN_ERR_HIP, "executor: hipMalloc failed");
  ex->allocs.push_back(*p);
  return CKAN_OK;
}

void free_all(ckan_exec* ex) {
  if (ex->graph) hipGraphExecDestroy(ex->graph);
  if (ex->graph_direct) hipGraphExecDestroy(ex->graph_direct);
  if (ex->ev_in) hipEventDestroy(ex->ev_in);
  if (ex->ev_out) hipEventDestroy(ex->ev_out);
  if (ex->es) hipStreamDestroy(ex->es);
  for (void* p : ex->allocs) hipFree(p);
  ex->allocs.clear();
}

// Whether the stack is small enough for the one-launch step.
bool tiny_eligible(const ckan_exec* ex) {
  const auto& c = ex->cfg;
  if (c.flags & CKAN_EXEC_NO_FUSED_SMALL) return false;
  if (c.n_layers > kTinyMaxLayers) return false;
  for (const auto& ly : ex->layers)  // the one-launch step: Chebyshev series of tanh(x) only
    if (ly.family || ly.desc.input_map != CKAN_INPUT_TANH) return false;
  int64_t macs = 0;
  for (int l = 0; l < c.n_layers; ++l) {
    const int64_t io = (int64_t)ex->widths[l] * ex->widths[l + 1];
    if (ex->degrees[l] + 1 > kTinyMaxD) return false;
    macs += c.batch * io * (ex->degrees[l] + 1) * (l > 0 ? 3 : 2);
  }
  return macs <= kTinyMaxMacs;
}

int run_tiny(ckan_exec* ex, const float* x, const void* target, float* losses, hipStream_t s,
             int nsteps = 1) {
  const auto& c = ex->cfg;
  TinyArgs a{};
  a.nl = c.n_layers;
  int64_t off = 0;
  const bool adam = c.optimizer == CKAN_OPT_ADAM;
  for (int l = 0; l < a.nl; ++l) {
    const auto& ly = ex->layers[l];
    TinyLayerArg& t = a.L[l];
    t = TinyLayerArg{ly.C, ly.m, ly.v, ly.t, ly.y, ly.dy, ly.desc.in_dim, ly.desc.out_dim,
                     ly.desc.degree + 1};
    const int64_t nc = (int64_t)t.I * t.O * t.D, bi = c.batch * t.I, bo = c.batch * t.O;
    t.sC = (int)off; off += nc;
    t.sm = (int)off; off += adam ? nc : 0;
    t.sv = (int)off; off += adam ? nc : 0;
    t.st = (int)off; off += bi;
    t.sy = (int)off; off += bo;
    t.sdy = (int)off; off += bo;
  }
  a.lds = off <= kTinyLdsFloats;
  a.lds_floats = a.lds ? (int)off : 0;
  a.loss = c.loss;
  a.opt = c.optimizer;
  a.bf16 = c.compute == CKAN_COMPUTE_BF16;
  a.B = c.batch;
  a.lr = c.lr;
  a.wd = c.weight_decay;
  a.w1 = (float)(1.0 - (double)c.beta1);
  a.beta2 = c.beta2;
  a.one_m_beta2 = (float)(1.0 - (double)c.beta2);
  a.eps = c.eps;
  a.lr_d = (double)c.lr;
  a.b1_d = (double)c.beta1;
  a.b2_d = (double)c.beta2;
  // threads: the widest elementwise phase (B x width), as a power of two
  // from 64 to 1024: idle waves only lengthen every barrier of the step
  int64_t widest = 1;
  for (int l = 0; l < a.nl; ++l) {
    const int64_t w = c.batch * (a.L[l].I > a.L[l].O ? a.L[l].I : a.L[l].O);
    if (w > widest) widest = w;
  }
  int threads = 64;
  while (threads < 1024 && threads < widest) threads *= 2;
  hipLaunchKernelGGL(k_tiny_step, dim3(1), dim3(threads), (size_t)a.lds_floats * sizeof(float), s,
                     a, x, target, ex->step, ex->loss, losses, nsteps);
  return hipGetLastError() == hipSuccess ? CKAN_OK : efail(CKAN_ERR_HIP, "executor: step launch failed");
}

// The optimizer write mode of layer ly's dC.
DcOut step_mode(const ckan_exec* ex, ckan_exec::Layer& ly) {
  const auto& c = ex->cfg;
  if (c.optimizer == CKAN_OPT_SGD) return DcOut{kDcSgd, c.lr, c.weight_decay};
  return DcOut{kDcAdam, 0.0f, c.weight_decay, (float)(1.0 - (double)c.beta1), c.beta2,
               (float)(1.0 - (double)c.beta2), c.eps, ly.C, ly.m, ly.v, ex->adam_sc};
}

// The step of a self_pack stack, three launches: layer 0's forward (its GEMM
// maps x itself) leaving split partials; the fused tail (layer 1's forward,
// the loss gradient and layer 1's dX into layer 0's dy); both layers' dC with
// the optimizer step, writing the packed operands the next step reads, and
// the loss mean.
int run_step_self_packed(ckan_exec* ex, const float* x, const void* target, hipStream_t s,
                         float* loss_copy) {
  auto& a = ex->layers[0];
  auto& b = ex->layers[1];
  const auto& c = ex->cfg;
  int rc;
  if ((rc = forward_tail_ce_packed(&a.desc, a.packed, x, a.t, &b.desc, b.C, b.t, b.y,
                                   reinterpret_cast<const int64_t*>(target), b.dy, ex->loss_part,
                                   a.dy, ex->fws, ex->fws_bytes, s)))
    return rc;
  if (c.optimizer != CKAN_OPT_SGD) {
    hipLaunchKernelGGL(k_adam_scalars, dim3(1), dim3(64), 0, s, ex->step, (double)c.lr,
                       (double)c.beta1, (double)c.beta2, ex->adam_sc);
    if (hipGetLastError() != hipSuccess) return efail(CKAN_ERR_HIP, "executor: adam launch failed");
  }
  const LossMean lm{ex->loss_part, c.batch, (float)(1.0 / (double)c.batch), ex->loss, loss_copy};
  return backward_self_packed(&a.desc, a.t, a.dy, a.C, step_mode(ex, a), a.packed, &b.desc, b.t,
                              b.dy, b.C, step_mode(ex, b), b.packed, lm, s);
}

// The step body on stream s with inputs x / target; the loss also goes to
// loss_copy when given.
int run_step(ckan_exec* ex, const float* x, const void* target, hipStream_t s,
             float* loss_copy = nullptr) {
  if (ex->tiny) return run_tiny(ex, x, target, loss_copy, s);
  if (ex->self_pack) return run_step_self_packed(ex, x, target, s, loss_copy);
  const int L = (int)ex->layers.size();
  int rc;
  for (int l = 0; l < L; ++l) {
    auto& ly = ex->layers[l];
    // pack and forward in one call: tanh in the pack launch (or, after a layer
    // with tanh_out, already in ly.t), bias summed by the forward
    const bool t_ready = l > 0 && ex->layers[l - 1].tanh_out;
    if (ly.tail_ce) {  // the last two layers, their packs, forwards and the loss gradient
      auto& nx = ex->layers[l + 1];
      if ((rc = pack2_forward_tail_ce(&ly.desc, ly.C, ly.packed, l == 0 ? x : ex->layers[l - 1].y,
                                      ly.t, t_ready, &nx.desc, nx.C, nx.packed, nx.t, nx.y,
                                      reinterpret_cast<const int64_t*>(target), nx.dy,
                                      ex->loss_part, ex->fws, ex->fws_bytes, s)))
        return rc;
      ++l;
      continue;
    }
    if (ly.pack_pair) {  // layers l and l + 1: both packs in one launch
      auto& nx = ex->layers[l + 1];
      float* outb = nx.tanh_out ? ex->layers[l + 2].t : nx.y;
      if ((rc = pack2_forward_ex(&ly.desc, ly.C, ly.packed, l == 0 ? x : ex->layers[l - 1].y, ly.t,
                                 t_ready, &nx.desc, nx.C, nx.packed, nx.t, outb, nx.tanh_out,
                                 ex->fws, ex->fws_bytes, s)))
        return rc;
      ++l;
      continue;
    }
    const float* in = l == 0 ? x : ex->layers[l - 1].y;
    float* out = ly.tanh_out ? ex->layers[l + 1].t : ly.y;
    if ((rc = pack_forward_ex(&ly.desc, ly.C, ly.packed, t_ready ? nullptr : in, out, ly.t,
                              ex->fws, ex->fws_bytes, s, t_ready, ly.tanh_out,
                              ly.family ? &ly.spec : nullptr)))
      return rc;
  }
  auto& last = ex->layers[L - 1];
  const int64_t B = ex->cfg.batch;
  const int O = last.desc.out_dim;
  // with the fused tail the rows' losses are in loss_part; the last layer's
  // backward takes their mean along
  const bool tail = L >= 2 && ex->layers[L - 2].tail_ce;
  const LossMean lm_tail{ex->loss_part, B, (float)(1.0 / (double)B), ex->loss, loss_copy};
  if (tail) {
    // no loss launch: the tail wrote dy and the rows' losses
  } else if (ex->cfg.loss == CKAN_LOSS_MSE) {
    const int64_t n = B * O;
    const int vec = n % 4 == 0 && (reinterpret_cast<uintptr_t>(target) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(last.y) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(last.dy) & 15) == 0;
    hipLaunchKernelGGL(k_mse, dim3(kLossBlocks), dim3(256), 0, s, last.y,
                       reinterpret_cast<const float*>(target), last.dy, n,
                       (float)(2.0 / (double)n), ex->loss_part, vec);
    hipLaunchKernelGGL(k_sum_scalar, dim3(1), dim3(256), 0, s, ex->loss_part,
                       (int64_t)kLossBlocks, (float)(1.0 / (double)n), ex->loss, loss_copy);
  } else if (B <= kCeSmallRows && O <= kCeSmallO) {
    // one thread per row, at least the 256 of the fixed-order sum
    const int threads = B <= 256 ? 256 : B <= 512 ? 512 : kCeSmallRows;
    hipLaunchKernelGGL(k_ce_small, dim3(1), dim3(threads), 0, s, last.y,
                       reinterpret_cast<const int64_t*>(target), last.dy, (int)B, O, ex->loss,
                       loss_copy);
  } else {
    hipLaunchKernelGGL(k_ce, dim3((unsigned)((B + 3) / 4)), dim3(256), 0, s, last.y,
                       reinterpret_cast<const int64_t*>(target), last.dy, B, O, ex->loss_part);
    hipLaunchKernelGGL(k_sum_scalar, dim3(1), dim3(256), 0, s, ex->loss_part, B,
                       (float)(1.0 / (double)B), ex->loss, loss_copy);
  }
  if (hipGetLastError() != hipSuccess) return efail(CKAN_ERR_HIP, "executor: loss launch failed");
  const auto& c = ex->cfg;
  // The optimizer step is applied by the dC kernels themselves, into C:
  // nothing reads a layer's C after its dC (the dX pass reads the packed copy).
  const bool sgd = c.optimizer == CKAN_OPT_SGD;
  if (!sgd) {
    hipLaunchKernelGGL(k_adam_scalars, dim3(1), dim3(64), 0, s, ex->step, (double)c.lr,
                       (double)c.beta1, (double)c.beta2, ex->adam_sc);
    if (hipGetLastError() != hipSuccess) return efail(CKAN_ERR_HIP, "executor: adam launch failed");
  }
  for (int l = L - 1; l >= 0; --l) {
    auto& ly = ex->layers[l];
    float* dx = l > 0 ? ex->layers[l - 1].dy : nullptr;
    const DcOut om = step_mode(ex, ly);
    const LossMean* lm = tail && l == L - 1 ? &lm_tail : nullptr;
    if (ly.family && !layer_on_valu(&ly.desc)) {
      // dC' into gcheb, then dC = dC' M^T and the optimizer step into C
      if ((rc = backward_impl(&ly.desc, ly.t, ly.packed, ly.dy, dx, ex->gcheb, DcOut{kDcStore},
                              ex->bws, ex->bws_bytes, s, lm)))
        return rc;
      const Plan p = make_plan(c.batch, ly.desc.in_dim, ly.desc.out_dim, ly.desc.degree,
                               c.compute == CKAN_COMPUTE_BF16);
      launch_coeff_from_cheb(ex->gcheb, ly.C, p, om, ly.xf, s);
      if (hipGetLastError() != hipSuccess)
        return efail(CKAN_ERR_HIP, "executor: basis gradient launch failed");
      continue;
    }
    if ((rc = backward_impl(&ly.desc, ly.t, ly.packed, ly.dy, dx, ly.C, om, ex->bws,
                            ex->bws_bytes, s, lm)))
      return rc;
  }
  return CKAN_OK;
}

}  // namespace

extern "C" {

int ckan_exec_create(const ckan_exec_config* cfg, ckan_exec** out, void* stream) {
  return ckan_exec_create_basis(cfg, nullptr, nullptr, out, stream);
}

int ckan_exec_create_basis(const ckan_exec_config* cfg, const ckan_basis_spec* bases,
                           const float* affine, ckan_exec** out, void* stream) {
  if (!cfg || !out) return efail(CKAN_ERR_INVALID_ARG, "executor: cfg/out is NULL");
  *out = nullptr;
  if (cfg->n_layers < 1 || !cfg->widths || !cfg->degrees)
    return efail(CKAN_ERR_INVALID_ARG, "executor: need n_layers >= 1 and widths/degrees");
  if (cfg->batch < 1) return efail(CKAN_ERR_INVALID_ARG, "executor: batch must be >= 1");
  if (cfg->loss != CKAN_LOSS_MSE && cfg->loss != CKAN_LOSS_CE)
    return efail(CKAN_ERR_INVALID_ARG, "executor: unknown loss");
  if (cfg->optimizer != CKAN_OPT_SGD && cfg->optimizer != CKAN_OPT_ADAM)
    return efail(CKAN_ERR_INVALID_ARG, "executor: unknown optimizer");
  if (cfg->optimizer == CKAN_OPT_ADAM &&
      !(cfg->beta1 >= 0.f && cfg->beta1 < 1.f && cfg->beta2 >= 0.f && cfg->beta2 < 1.f))
    return efail(CKAN_ERR_INVALID_ARG, "executor: betas must lie in [0, 1)");
  ckan_exec* ex = new ckan_exec();
  ex->cfg = *cfg;
  ex->widths.assign(cfg->widths, cfg->widths + cfg->n_layers + 1);
  ex->degrees.assign(cfg->degrees, cfg->degrees + cfg->n_layers);
  ex->cfg.widths = ex->widths.data();
  ex->cfg.degrees = ex->degrees.data();
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int rc = CKAN_OK;
  ex->layers.resize(cfg->n_layers);
  int64_t gcheb_elems = 0;
  for (int l = 0; l < cfg->n_layers && rc == CKAN_OK; ++l) {
    auto& ly = ex->layers[l];
    ly.desc = ckan_desc{cfg->batch, ex->widths[l], ex->widths[l + 1], ex->degrees[l],
                        cfg->compute, CKAN_DTYPE_F32, CKAN_INPUT_TANH};
    if (affine && (affine[2 * l] != 0.0f || affine[2 * l + 1] != 0.0f)) {
      ly.desc.input_map = CKAN_INPUT_AFFINE;
      ly.desc.in_scale = affine[2 * l];
      ly.desc.in_shift = affine[2 * l + 1];
    }
    ly.packed_bytes = ckan_packed_bytes(&ly.desc);
    if (ly.packed_bytes == 0) {
      rc = efail(CKAN_ERR_INVALID_ARG, "executor: invalid layer shape, degree or input map");
      break;
    }
    if (bases) {
      ly.spec = bases[l];
      if (ly.spec.degree != ly.desc.degree) {
        char msg[96];
        snprintf(msg, sizeof msg, "executor: layer %d basis degree %d != layer degree %d", l,
                 ly.spec.degree, ly.desc.degree);
        rc = efail(CKAN_ERR_INVALID_ARG, msg);
        break;
      }
      // a Chebyshev spec of scale 1 is the plain layer
      ly.family = !(ly.spec.family == CKAN_BASIS_CHEBYSHEV && ly.spec.scale == 1.0);
      if (ly.family && (rc = basis_check(&ly.spec, ly.desc.degree, &ly.xf))) break;
    }
    ly.ncoef = (int64_t)ly.desc.in_dim * ly.desc.out_dim * (ly.desc.degree + 1);
    if (ly.family && !layer_on_valu(&ly.desc) && ly.ncoef > gcheb_elems) gcheb_elems = ly.ncoef;
    const int64_t ny = cfg->batch * ly.desc.out_dim;
    if ((rc = dev_alloc(ex, (void**)&ly.C, ly.ncoef * 4)) ||
        (rc = dev_alloc(ex, &ly.packed, ly.packed_bytes)) ||
        (rc = dev_alloc(ex, (void**)&ly.t, ckan_tcache_elems(&ly.desc) * 4)) ||
        (rc = dev_alloc(ex, (void**)&ly.y, ny * 4)) ||
        (rc = dev_alloc(ex, (void**)&ly.dy, ny * 4)))
      break;
    launch_zero_f32(ly.C, ly.ncoef, s);
    if (cfg->optimizer == CKAN_OPT_ADAM) {
      if ((rc = dev_alloc(ex, (void**)&ly.m, ly.ncoef * 4)) ||
          (rc = dev_alloc(ex, (void**)&ly.v, ly.ncoef * 4)))
        break;
      launch_zero_f32(ly.m, ly.ncoef, s);
      launch_zero_f32(ly.v, ly.ncoef, s);
    }
    const size_t f = ckan_fwd_workspace_bytes(&ly.desc);
    const size_t b = ckan_bwd_workspace_bytes(&ly.desc, l > 0, 1);
    if (f > ex->fws_bytes) ex->fws_bytes = f;
    if (b > ex->bws_bytes) ex->bws_bytes = b;
  }
  for (int l = 0; rc == CKAN_OK && l + 1 < cfg->n_layers; ++l)
    ex->layers[l].tanh_out = layer_out_tanh_ok(&ex->layers[l].desc) &&
                             ex->layers[l + 1].desc.input_map == CKAN_INPUT_TANH &&
                             layer_reads_tcache(&ex->layers[l + 1].desc);
  for (int l = 0; rc == CKAN_OK && l + 1 < cfg->n_layers; ++l) {
    auto& ly = ex->layers[l];
    // the paired launch packs Chebyshev coefficients and maps x by tanh
    ly.pack_pair = ly.tanh_out && !ly.family && !ex->layers[l + 1].family &&
                   ly.desc.input_map == CKAN_INPUT_TANH &&
                   pack_pair_fits(&ly.desc, &ex->layers[l + 1].desc);
    ly.tail_ce = ly.pack_pair && l + 2 == cfg->n_layers && cfg->loss == CKAN_LOSS_CE &&
                 pack2_tail_ce_fits(&ly.desc, &ex->layers[l + 1].desc);
    if (ly.pack_pair) ++l;  // the next layer's pack is taken
  }
  if (rc == CKAN_OK) {
    ex->fws_bytes = align256(ex->fws_bytes);
    ex->bws_bytes = align256(ex->bws_bytes);
    const int64_t nloss = cfg->batch > kLossBlocks ? cfg->batch : kLossBlocks;
    if (!(rc = dev_alloc(ex, &ex->fws, ex->fws_bytes)) &&
        !(rc = dev_alloc(ex, &ex->bws, ex->bws_bytes)) &&
        !(rc = dev_alloc(ex, (void**)&ex->loss_part, nloss * 4)) &&
        !(rc = dev_alloc(ex, (void**)&ex->loss, 256)) &&
        !(rc = dev_alloc(ex, (void**)&ex->step, 256)) &&
        !(rc = dev_alloc(ex, (void**)&ex->adam_sc, 256)) &&
        !(rc = gcheb_elems ? dev_alloc(ex, (void**)&ex->gcheb, gcheb_elems * 4) : CKAN_OK)) {
      if (ex->fws_bytes) launch_zero(ex->fws, ex->fws_bytes, s);
      launch_zero(ex->step, 256, s);
    }
  }
  if (rc == CKAN_OK) ex->tiny = tiny_eligible(ex);
  if (rc == CKAN_OK && !ex->tiny && cfg->n_layers == 2 && ex->layers[0].tail_ce &&
      !(cfg->flags & CKAN_EXEC_PACK_EACH_STEP) &&
      self_pack_pair_fits(&ex->layers[0].desc, &ex->layers[1].desc)) {
    ex->self_pack = true;
    for (int l = 0; l < 2 && rc == CKAN_OK; ++l)
      rc = self_pack_layer(&ex->layers[l].desc, ex->layers[l].C, ex->layers[l].packed, s);
  }
  if (rc == CKAN_OK && cfg->use_graph) {
    const int O = ex->widths[cfg->n_layers];
    ex->tgt_bytes = cfg->loss == CKAN_LOSS_MSE ? (size_t)cfg->batch * O * 4 : (size_t)cfg->batch * 8;
    if (!(rc = dev_alloc(ex, (void**)&ex->x_own, (size_t)cfg->batch * ex->widths[0] * 4)) &&
        !(rc = dev_alloc(ex, &ex->tgt_own, ex->tgt_bytes))) {
      if (hipStreamCreateWithFlags(&ex->es, hipStreamNonBlocking) != hipSuccess ||
          hipEventCreateWithFlags(&ex->ev_in, hipEventDisableTiming) != hipSuccess ||
          hipEventCreateWithFlags(&ex->ev_out, hipEventDisableTiming) != hipSuccess)
        rc = efail(CKAN_ERR_HIP, "executor: stream/event creation failed");
    }
  }
  if (rc == CKAN_OK && hipGetLastError() != hipSuccess)
    rc = efail(CKAN_ERR_HIP, "executor: initialisation launch failed");
  if (rc != CKAN_OK) {
    free_all(ex);
    delete ex;
    return rc;
  }
  *out = ex;
  return CKAN_OK;
}

int ckan_exec_destroy(ckan_exec* ex) {
  if (!ex) return CKAN_OK;
  if (ex->es) hipStreamSynchronize(ex->es);
  hipDeviceSynchronize();
  free_all(ex);
  delete ex;
  return CKAN_OK;
}

static int check_layer(ckan_exec* ex, int32_t layer) {
  if (!ex) return efail(CKAN_ERR_INVALID_ARG, "executor is NULL");
  if (layer < 0 || layer >= (int32_t)ex->layers.size())
    return efail(CKAN_ERR_INVALID_ARG, "executor: layer index out of range");
  return CKAN_OK;
}

int ckan_exec_set_coeffs(ckan_exec* ex, int32_t layer, const float* src, void* stream) {
  int rc = check_layer(ex, layer);
  if (rc) return rc;
  if (!src) return efail(CKAN_ERR_INVALID_ARG, "executor: src is NULL");
  auto& ly = ex->layers[layer];
  hipLaunchKernelGGL(k_copy_f32, dim3(grid_of(ly.ncoef)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), src, ly.C, ly.ncoef);
  if (hipGetLastError() != hipSuccess) return efail(CKAN_ERR_HIP, "executor: copy failed");
  // the packed operands follow C (the step itself does not pack)
  return ex->self_pack ? self_pack_layer(&ly.desc, ly.C, ly.packed, stream) : CKAN_OK;
}

int ckan_exec_get_coeffs(ckan_exec* ex, int32_t layer, float* dst, void* stream) {
  int rc = check_layer(ex, layer);
  if (rc) return rc;
  if (!dst) return efail(CKAN_ERR_INVALID_ARG, "executor: dst is NULL");
  auto& ly = ex->layers[layer];
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (ex->es) {  // order after any graph replay on the executor stream
    hipEventRecord(ex->ev_out, ex->es);
    hipStreamWaitEvent(s, ex->ev_out, 0);
  }
  hipLaunchKernelGGL(k_copy_f32, dim3(grid_of(ly.ncoef)), dim3(256), 0, s, ly.C, dst, ly.ncoef);
  return hipGetLastError() == hipSuccess ? CKAN_OK : efail(CKAN_ERR_HIP, "executor: copy failed");
}

int ckan_exec_get_adam_state(ckan_exec* ex, int32_t layer, float* m, float* v, int64_t* step,
                             void* stream) {
  int rc = check_layer(ex, layer);
  if (rc) return rc;
  if (ex->cfg.optimizer != CKAN_OPT_ADAM)
    return efail(CKAN_ERR_UNSUPPORTED, "executor: optimizer has no Adam state");
  if (!m || !v || !step) return efail(CKAN_ERR_INVALID_ARG, "executor: m/v/step is NULL");
  auto& ly = ex->layers[layer];
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (ex->es) {
    hipEventRecord(ex->ev_out, ex->es);
    hipStreamWaitEvent(s, ex->ev_out, 0);
  }
  hipLaunchKernelGGL(k_copy_f32, dim3(grid_of(ly.ncoef)), dim3(256), 0, s, ly.m, m, ly.ncoef);
  hipLaunchKernelGGL(k_copy_f32, dim3(grid_of(ly.ncoef)), dim3(256), 0, s, ly.v, v, ly.ncoef);
  if (hipMemcpyAsync(step, ex->step, sizeof(int64_t), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return efail(CKAN_ERR_HIP, "executor: state copy failed");
  return CKAN_OK;
}

int ckan_exec_set_adam_state(ckan_exec* ex, int32_t layer, const float* m, const float* v,
                             int64_t step, void* stream) {
  int rc = check_layer(ex, layer);
  if (rc) return rc;
  if (ex->cfg.optimizer != CKAN_OPT_ADAM)
    return efail(CKAN_ERR_UNSUPPORTED, "executor: optimizer has no Adam state");
  if (!m || !v || step < 0) return efail(CKAN_ERR_INVALID_ARG, "executor: bad m/v/step");
  auto& ly = ex->layers[layer];
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_copy_f32, dim3(grid_of(ly.ncoef)), dim3(256), 0, s, m, ly.m, ly.ncoef);
  hipLaunchKernelGGL(k_copy_f32, dim3(grid_of(ly.ncoef)), dim3(256), 0, s, v, ly.v, ly.ncoef);
  int64_t st = step;
  if (hipMemcpyAsync(ex->step, &st, sizeof(int64_t), hipMemcpyHostToDevice, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return efail(CKAN_ERR_HIP, "executor: state copy failed");
  return CKAN_OK;
}

int ckan_exec_step(ckan_exec* ex, const float* x, const void* target, float* loss_out,
                   void* stream) {
  if (!ex) return efail(CKAN_ERR_INVALID_ARG, "executor is NULL");
  if (!x || !target) return efail(CKAN_ERR_INVALID_ARG, "executor: x/target is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int rc;
  // small device copies use a kernel: a DMA-engine copy adds tens of us of latency
  auto copy = [&](void* dst, const void* src, size_t bytes, hipStream_t st) {
    const int64_t n = (int64_t)(bytes / 4);
    hipLaunchKernelGGL(k_copy_f32, dim3(grid_of(n)), dim3(256), 0, st,
                       reinterpret_cast<const float*>(src), reinterpret_cast<float*>(dst), n);
    return hipGetLastError() == hipSuccess;
  };
  if (!ex->cfg.use_graph) {
    return run_step(ex, x, target, s, loss_out);  // writes loss_out itself
  }
  // graph mode.  The graph is captured once on the executor's own stream and
  // replayed on `stream`.  A step whose x and target pointers are those of
  // the step before replays a graph captured on those buffers (the usual
  // training loop reuses them; the graph reads whatever they hold when it
  // runs); otherwise the inputs are first copied into executor-owned buffers
  // and a graph captured on those is replayed (two small copy kernels more).
  auto capture = [&](const float* cx, const void* ct, hipGraphExec_t* out) -> int {
    if (hipEventRecord(ex->ev_in, s) != hipSuccess || hipStreamWaitEvent(ex->es, ex->ev_in, 0) != hipSuccess)
      return efail(CKAN_ERR_HIP, "executor: stream ordering failed");
    hipGraph_t g = nullptr;
    if (hipStreamBeginCapture(ex->es, hipStreamCaptureModeThreadLocal) != hipSuccess)
      return efail(CKAN_ERR_HIP, "executor: graph capture failed to start");
    const int rc2 = run_step(ex, cx, ct, ex->es);
    const hipError_t ec = hipStreamEndCapture(ex->es, &g);
    if (rc2) {
      if (g) hipGraphDestroy(g);
      return rc2;
    }
    if (ec != hipSuccess || hipGraphInstantiate(out, g, nullptr, nullptr, 0) != hipSuccess) {
      if (g) hipGraphDestroy(g);
      return efail(CKAN_ERR_HIP, "executor: graph capture failed");
    }
    hipGraphDestroy(g);
    return CKAN_OK;
  };
  const bool repeat = x == ex->last_x && target == ex->last_t;
  ex->last_x = x;
  ex->last_t = target;
  if (repeat) {
    if (ex->graph_direct && (ex->gd_x != x || ex->gd_t != target)) {
      // a graph on other buffers: let its replays finish before it goes
      if (hipStreamSynchronize(s) != hipSuccess) return efail(CKAN_ERR_HIP, "executor: sync failed");
      hipGraphExecDestroy(ex->graph_direct);
      ex->graph_direct = nullptr;
    }
    if (!ex->graph_direct) {
      if ((rc = capture(x, target, &ex->graph_direct))) return rc;
      ex->gd_x = x;
      ex->gd_t = target;
    }
    if (hipGraphLaunch(ex->graph_direct, s) != hipSuccess)
      return efail(CKAN_ERR_HIP, "executor: graph launch failed");
  } else {
    const size_t xb = (size_t)ex->cfg.batch * ex->widths[0] * 4;
    if (!copy(ex->x_own, x, xb, s) || !copy(ex->tgt_own, target, ex->tgt_bytes, s))
      return efail(CKAN_ERR_HIP, "executor: input staging failed");
    if (!ex->graph && (rc = capture(ex->x_own, ex->tgt_own, &ex->graph))) return rc;
    if (hipGraphLaunch(ex->graph, s) != hipSuccess)
      return efail(CKAN_ERR_HIP, "executor: graph launch failed");
  }
  if (loss_out && !copy(loss_out, ex->loss, 4, s))
    return efail(CKAN_ERR_HIP, "executor: loss copy failed");
  return CKAN_OK;
}

int ckan_exec_steps(ckan_exec* ex, const float* x, const void* target, int64_t nsteps,
                    float* losses, void* stream) {
  if (!ex) return efail(CKAN_ERR_INVALID_ARG, "executor is NULL");
  if (!x || !target) return efail(CKAN_ERR_INVALID_ARG, "executor: x/target is NULL");
  if (nsteps < 0) return efail(CKAN_ERR_INVALID_ARG, "executor: nsteps must be >= 0");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (ex->es) {  // order after any graph replay on the executor stream
    hipEventRecord(ex->ev_out, ex->es);
    hipStreamWaitEvent(s, ex->ev_out, 0);
  }
  int rc;
  if (ex->tiny) {  // the steps in one launch per chunk: no launch gap between steps
    for (int64_t k = 0; k < nsteps; k += kTinyStepsPerLaunch) {
      const int n = (int)(nsteps - k < kTinyStepsPerLaunch ? nsteps - k : kTinyStepsPerLaunch);
      if ((rc = run_tiny(ex, x, target, losses ? losses + k : nullptr, s, n))) return rc;
    }
    return CKAN_OK;
  }
  for (int64_t k = 0; k < nsteps; ++k) {
    float* lk = losses ? losses + k : nullptr;
    if ((rc = run_step(ex, x, target, s, lk))) return rc;
  }
  return CKAN_OK;
}

int ckan_exec_forward(ckan_exec* ex, const float* x, float* y, void* stream) {
  if (!ex) return efail(CKAN_ERR_INVALID_ARG, "executor is NULL");
  if (!x || !y) return efail(CKAN_ERR_INVALID_ARG, "executor: x/y is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (ex->es) {
    hipEventRecord(ex->ev_out, ex->es);
    hipStreamWaitEvent(s, ex->ev_out, 0);
  }
  const int L = (int)ex->layers.size();
  int rc;
  for (int l = 0; l < L; ++l) {
    auto& ly = ex->layers[l];
    const float* in = l == 0 ? x : ex->layers[l - 1].y;
    float* out = l == L - 1 ? y : ly.y;
    if ((rc = ckan_pack_forward(&ly.desc, ly.family ? &ly.spec : nullptr, ly.C, ly.packed, in,
                                out, ly.t, ex->fws, ex->fws_bytes, s)))
      return rc;
  }
  return CKAN_OK;
}

}  // extern "C"
