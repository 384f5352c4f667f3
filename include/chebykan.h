/*
 * chebykan.h -- C-ABI of the MI355X (gfx950) ChebyKAN layer hot path.
 *
 * The reference (0xEodum/KAN) is pure Python on torch; this boundary replaces
 * the torch op sequences its ChebyKAN layer executes.  Each entry point names
 * the reference code it stands in for.  No torch or C++ types cross it: plain
 * device pointers, sizes and a hipStream_t passed as void*.
 *
 * Conventions
 *   - All pointers are device pointers unless stated; all launches are
 *     stream-ordered on `stream` (a hipStream_t) and never synchronise the host.
 *   - x, y, dy, dx and t are row-major fp32.  Coefficients C are [in, out, D]
 *     row-major (D = degree + 1), fp32 or bf16, the layout of the reference's
 *     `cheby_coeffs` parameter (kan/layers/chebykan.py:48-51).
 *   - Every call returns a ckan_status; on failure ckan_last_error() returns a
 *     thread-local message.  Argument checks happen on the host before any
 *     launch, so an invalid call launches nothing.
 *   - Workspaces are caller-allocated scratch (split-K partials, re-laid
 *     operands); no call needs them zeroed.  Calls that share one workspace
 *     must not overlap in time.
 */
#ifndef CHEBYKAN_H
#define CHEBYKAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum ckan_status {
  CKAN_OK = 0,
  CKAN_ERR_INVALID_ARG = 1,   /* bad shape, null pointer, size mismatch  */
  CKAN_ERR_UNSUPPORTED = 2,   /* valid request this build does not serve */
  CKAN_ERR_WORKSPACE = 3,     /* workspace smaller than required          */
  CKAN_ERR_HIP = 4            /* a HIP runtime call or launch failed      */
} ckan_status;

typedef enum ckan_compute {
  CKAN_COMPUTE_FP32 = 0,      /* fp32 MFMA (v_mfma_f32_32x32x2_f32)                 */
  CKAN_COMPUTE_BF16 = 1       /* bf16 MFMA, fp32 accumulate (v_mfma_f32_32x32x16_bf16) */
} ckan_compute;

typedef enum ckan_dtype {
  CKAN_DTYPE_F32 = 0,
  CKAN_DTYPE_BF16 = 1
} ckan_dtype;

/* How the layer maps an input x to the argument t of its basis. */
typedef enum ckan_input_map {
  CKAN_INPUT_TANH = 0,    /* t = tanh(x), the reference's default
                             (kan/basis/chebyshev.py:68-78)                */
  CKAN_INPUT_AFFINE = 1   /* t = in_scale * x + in_shift: the Hermite
                             layer's map of a finite domain onto [-3, 3]
                             (kan/basis/hermite.py:102-112), expressed on
                             [-1, 1] with the basis scale 3               */
} ckan_input_map;

/* Problem descriptor: one ChebyKANLayer(in_dim, out_dim, degree) applied to a
 * batch of `batch` rows (kan/layers/chebykan.py:21-22,64).
 * Degrees 0..16 run on the MFMA kernels in the compute precision.  Degrees
 * 17..1024 (the reference layer takes any degree, kan/layers/chebykan.py:21-51)
 * run on vector-ALU kernels in fp32 whatever `compute` asks, with either input
 * map; their packed buffer is C widened to fp32 in its own [in, out, D]
 * layout followed by the basis recurrence block, and they need no workspace
 * (the size queries return 0). */
typedef struct ckan_desc {
  int64_t batch;        /* B: rows of x after x.view(-1, in_dim)          */
  int32_t in_dim;       /* I                                               */
  int32_t out_dim;      /* O                                               */
  int32_t degree;       /* deg (0..1024); D = deg + 1 coefficients per (i, o) */
  int32_t compute;      /* ckan_compute                                    */
  int32_t coeff_dtype;  /* ckan_dtype of C passed to ckan_pack_coeffs      */
  int32_t input_map;    /* ckan_input_map (0: tanh)                        */
  float in_scale;       /* CKAN_INPUT_AFFINE: t = in_scale * x + in_shift  */
  float in_shift;       /* (both 0 with CKAN_INPUT_TANH)                   */
} ckan_desc;

/* ---- sizes (host only, no device work) ---------------------------------- */

/* Bytes of the packed-coefficient buffer written by ckan_pack_coeffs. */
size_t ckan_packed_bytes(const ckan_desc* desc);
/* Elements (fp32) of the tanh cache written by ckan_forward and read by
 * ckan_backward: tanh(x) as [B, in_pad] with zero padding columns. */
size_t ckan_tcache_elems(const ckan_desc* desc);
/* Bytes of forward / backward workspace. */
size_t ckan_fwd_workspace_bytes(const ckan_desc* desc);
size_t ckan_bwd_workspace_bytes(const ckan_desc* desc, int need_dx, int need_dcoeffs);

/* Zero-fill a workspace on `stream` with a fill kernel (no hipMemset).  No
 * entry point requires it; kept for callers that want defined contents. */
int ckan_workspace_init(void* ws, size_t ws_bytes, void* stream);

/* ---- layer operators ---------------------------------------------------- */

/* Re-lays C [in, out, D] out into the MFMA operand layouts used by the
 * forward and input-gradient contractions, in the compute precision, and the
 * per-output bias sum_i C[i, o, 0] (the T_0 = 1 term).
 * Replaces: the coefficient permute/reshape/clone inside
 * torch.einsum('bid,iod->bo') (kan/basis/chebyshev.py:101). */
int ckan_pack_coeffs(const ckan_desc* desc, const void* coeffs, void* packed, void* stream);

/* y[b, o] = sum_{i, d} T_d(tanh x[b, i]) C[i, o, d]; also writes t = tanh(x)
 * into t_cache (ckan_tcache_elems floats) for the backward.
 * Replaces: ChebyshevBasis.forward (kan/basis/chebyshev.py:80-101): tanh
 * (:78), closed-form basis (:130-145) and the einsum (:101). */
int ckan_forward(const ckan_desc* desc, const float* x, const void* packed, float* y,
                 float* t_cache, void* ws, size_t ws_bytes, void* stream);

/* ckan_pack_coeffs (or, with a non-NULL basis spec, ckan_pack_coeffs_basis,
 * below) followed by ckan_forward, in fewer launches: the tanh of x is
 * computed by the pack launch itself where the layout allows, and the
 * per-output bias sum is reduced by the forward GEMM where it can.  Same
 * arguments, results and packed-buffer contents as the two calls.
 * Replaces: the layer forward as the reference runs it on every call, the
 * einsum's coefficient re-layout included (kan/layers/chebykan.py:64-67,
 * kan/basis/chebyshev.py:78,92-101). */
struct ckan_basis_spec;
int ckan_pack_forward(const ckan_desc* desc, const struct ckan_basis_spec* spec,
                      const void* coeffs, void* packed, const float* x, float* y, float* t_cache,
                      void* ws, size_t ws_bytes, void* stream);

/* ckan_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * split-K partials of the small-batch paths go to a fixed device array of
 * CKAN_NOALLOC_SCRATCH_BYTES, one per GPU, held until the process ends; the
 * call allocates nothing (no hipMalloc / hipFree).  Shapes whose
 * ckan_fwd_workspace_bytes exceeds that size return CKAN_ERR_WORKSPACE and
 * launch nothing.  Every call on one GPU shares that GPU's array, so calls that
 * overlap in time on one GPU (e.g. on two streams) race; calls in one stream
 * order are safe.  Results are identical to ckan_forward's. */
#define CKAN_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int ckan_forward_noalloc(const ckan_desc* desc, const float* x, const void* packed, float* y,
                         float* t_cache, void* stream);

/* Gradients of the forward for upstream gradient dy [B, out]:
 *   dx[b, i]    = (1 - t^2) sum_{o, d} dy[b, o] C[i, o, d] d U_{d-1}(t)   (dx may be NULL)
 *   dC[i, o, d] = sum_b T_d(t[b, i]) dy[b, o]                            (dcoeffs may be NULL)
 * With accumulate != 0, dC is added to the existing contents of dcoeffs
 * (torch AccumulateGrad semantics); otherwise it is overwritten.  packed may
 * be NULL when dx is NULL, except above degree 16, where it also carries the
 * basis recurrence that dC needs.
 * Replaces: torch autograd through kan/basis/chebyshev.py:78,101,136-145
 * (BmmBackward0 x2, CosBackward0, MulBackward0, AcosBackward0, TanhBackward0).
 * Divergence: for |x| >= 9.0108, where fp32 tanh(x) == +-1, the reference
 * yields NaN in dx (acos'(+-1) = -inf); this returns the finite analytic value. */
int ckan_backward(const ckan_desc* desc, const float* t_cache, const void* packed,
                  const float* dy, float* dx, float* dcoeffs, int accumulate,
                  void* ws, size_t ws_bytes, void* stream);

/* ---- fp64 path ------------------------------------------------------------
 * The reference layer computes in fp64 when its parameter is fp64
 * (kan/layers/chebykan.py:48-51 after .double(); kan/basis/chebyshev.py:78-101
 * then runs in fp64).  These entry points run that case in fp64 end to end
 * (fp64 FMA on the vector ALU).  x, coeffs [in, out, D], y, t_cache [B, in],
 * dy, dx and dcoeffs are fp64; desc->compute and desc->coeff_dtype must be 0.
 * No packing and no workspace: coeffs are read in their own layout.
 * Same formulas, NULL rules and accumulate semantics as ckan_forward /
 * ckan_backward, and the same finite value at tanh saturation (|x| >= 19.06
 * in fp64). */
int ckan_forward_f64(const ckan_desc* desc, const double* x, const double* coeffs, double* y,
                     double* t_cache, void* stream);
int ckan_backward_f64(const ckan_desc* desc, const double* t_cache, const double* coeffs,
                      const double* dy, double* dx, double* dcoeffs, int accumulate, void* stream);

/* The fp64 path for a layer of another polynomial family (ckan_basis_spec,
 * below): the Jacobi and Hermite layers after .double(), whose reference
 * computes their bases in fp64 (kan/basis/jacobi.py:96-117,159-188,
 * kan/basis/hermite.py:118-139,158-233).  The basis P_n(s tanh x) is evaluated
 * by the family's three-term recurrence in fp64 (no change of basis, whose
 * matrix entries reach 1e10 for Hermite), from a recurrence block that
 * ckan_write_recurrence_f64 writes into a caller-owned device buffer of
 * ckan_recurrence_bytes_f64(spec) bytes (8-byte aligned) once per spec;
 * the forward and backward then read it (spec->degree must equal
 * desc->degree: the library cannot check the buffer's contents).  dcoeffs is
 * the family coefficients' gradient.  The tanh input map only. */
size_t ckan_recurrence_bytes_f64(const struct ckan_basis_spec* spec);
int ckan_write_recurrence_f64(const struct ckan_basis_spec* spec, double* rec, void* stream);
int ckan_forward_f64_basis(const ckan_desc* desc, const double* rec, const double* x,
                           const double* coeffs, double* y, double* t_cache, void* stream);
int ckan_backward_f64_basis(const ckan_desc* desc, const double* rec, const double* t_cache,
                            const double* coeffs, const double* dy, double* dx, double* dcoeffs,
                            int accumulate, void* stream);

/* ---- other polynomial bases through the same kernels ---------------------
 * A layer whose basis is a three-term-recurrence family P_0..P_deg evaluated
 * at s * tanh(x) is the ChebyKAN layer with coefficients C' = C M, where
 *   P_n(s u) = sum_k M[n, k] T_k(u)      (M lower triangular, exact),
 * and its coefficient gradient is dC = dC' M^T; the input gradient is the
 * ChebyKAN layer's with C'.  So ckan_pack_coeffs_basis + ckan_forward +
 * ckan_backward (into dC') + ckan_coeff_grad_from_chebyshev run such a layer
 * (ckan_backward_basis: the last two in one call).
 * Above degree 16 (the vector-ALU kernels) the packed buffer carries the
 * family's recurrence instead of C M: the kernels evaluate P_n(s u) by the
 * recurrence and differentiate it, ckan_backward's dC is already the family
 * coefficients' gradient and ckan_coeff_grad_from_chebyshev is the identity
 * (a copy, an accumulation, or nothing in place), so the same four calls
 * serve every degree.
 * Families and the reference code each replaces:
 *   JACOBI     P_n^(alpha,beta), alpha, beta > -1, s = 1: JacobiBasis
 *              (kan/basis/jacobi.py:84-117,147-188), JacobiKANLayer
 *              (kan/layers/jacobikan.py:26-77)
 *   HERMITE    physicists' H_n; HermiteKANLayer's default input map is
 *              s = 3 (kan/basis/hermite.py:85-116,158-193)
 *   HERMITE_E  probabilists' He_n, s = 3 (kan/basis/hermite.py:195-233)
 *   CHEBYSHEV  T_n (M = identity)
 */
typedef enum ckan_basis_family {
  CKAN_BASIS_CHEBYSHEV = 0,
  CKAN_BASIS_JACOBI = 1,
  CKAN_BASIS_HERMITE = 2,
  CKAN_BASIS_HERMITE_E = 3
} ckan_basis_family;

typedef struct ckan_basis_spec {
  int32_t family;   /* ckan_basis_family                                      */
  int32_t degree;   /* 0..1024 (0..16 for ckan_basis_to_chebyshev and the
                       derivative entry points); equal to desc->degree where a
                       desc is passed too */
  double alpha;     /* Jacobi parameters (> -1); ignored by the other families */
  double beta;
  double scale;     /* s: the basis is evaluated at s * tanh(x) (finite)       */
} ckan_basis_spec;

/* Host only: M as (degree+1)^2 doubles, M[n * (degree+1) + k]. */
int ckan_basis_to_chebyshev(const ckan_basis_spec* spec, double* M);
/* ckan_pack_coeffs of C' = C M, for C in the family's basis (fp32 or bf16 per
 * desc->coeff_dtype).  M is built on the host and passed by value.  Above
 * degree 16: C widened to fp32 and the family's recurrence block. */
int ckan_pack_coeffs_basis(const ckan_desc* desc, const ckan_basis_spec* spec, const void* coeffs,
                           void* packed, void* stream);
/* dcoeffs[i, o, n] (+)= sum_k dcheb[i, o, k] M[n, k] (fp32 [in, out, D]);
 * dcheb may equal dcoeffs when accumulate == 0 (in place).  Above degree 16,
 * dcoeffs (+)= dcheb (ckan_backward's output is already in the family basis). */
int ckan_coeff_grad_from_chebyshev(const ckan_desc* desc, const ckan_basis_spec* spec,
                                   const float* dcheb, float* dcoeffs, int accumulate, void* stream);
/* ckan_backward (accumulate = 0) followed by ckan_coeff_grad_from_chebyshev
 * in place, in one call: dcoeffs receives the family coefficients' gradient
 * (stored), dx the input gradient, the workspace as for ckan_backward.  Where
 * one pipelined dC launch writes the whole gradient, it applies M^T to each
 * row before its stores (no second pass over dC); otherwise the map runs as
 * its own launch.  The results are the same bits either way.
 * Replaces: torch autograd through kan/basis/jacobi.py:95-116 and
 * kan/basis/hermite.py:118-139 (the einsum's backward in the family basis). */
int ckan_backward_basis(const ckan_desc* desc, const ckan_basis_spec* spec, const float* t_cache,
                        const void* packed, const float* dy, float* dx, float* dcoeffs, void* ws,
                        size_t ws_bytes, void* stream);
/* out[q, n] = P_n(t[q]), n = 0..degree (<= 1024), by the family's recurrence
 * (the reference's basis_functions of an already-normalised input; s unused). */
int ckan_family_basis(const ckan_basis_spec* spec, const float* t, int64_t n, float* out,
                      void* stream);
/* dt[q] = sum_n g[q, n] P_n'(t[q]): backward of ckan_family_basis. */
int ckan_family_basis_backward(const ckan_basis_spec* spec, const float* t, const float* g,
                               int64_t n, float* dt, void* stream);

/* ---- derivatives with respect to the input --------------------------------
 * Each univariate function of a layer, f(x) = sum_n C[i, o, n] P_n(s tanh x)
 * (spec NULL: the ChebyKAN layer's T_n(tanh x)), has an order-k derivative in
 * x that is again a Chebyshev series in t = tanh x, of degree degree + k:
 *   d^k f / dx^k = sum_j Ck[i, o, j] T_j(t),   Ck = C R,   R = M L^k,
 * with M the family's change of basis and L : p -> (1 - t^2) p'(t) (exact in
 * the T basis).  Under the affine input map of desc (t = a x + b, the Hermite
 * layer's finite domain) L : p -> a p'(t) instead, the series one degree
 * lower (Ck keeps degree + 1 + k columns, the last 2k zero).  Requires fp32
 * coefficients and degree + k <= 16 for a family basis or the affine map,
 * degree + k <= 256 for the Chebyshev one under tanh (above 16 the device
 * applies L row by row in place of the matrix R).
 * Replaces KANLayer.compute_derivatives / jacobian (kan/layers/base.py:102-141)
 * and ChebyshevBasis.derivative (kan/basis/chebyshev.py:174-267).  Divergence:
 * the reference's derivative coefficients are wrong for n >= 3, omit the
 * tanh chain factor and its jacobian adds the other inputs' derivatives at 0;
 * these return the exact derivatives with respect to x. */
/* R (fp64, row-major [degree + 1][degree + 1 + order]) of the tanh map; host only. */
int ckan_derivative_matrix(const ckan_basis_spec* spec, int32_t degree, int32_t order, double* R);
/* out [in, out, degree + 1 + order] = coeffs [in, out, degree + 1] R; a
 * ChebyKAN forward of degree desc->degree + order with `out` then gives
 * sum_i d^k f_{i,o} / dx^k (x_i), the layer's compute_derivatives(x, k). */
int ckan_derivative_coeffs(const ckan_desc* desc, const ckan_basis_spec* spec, int32_t order,
                           const float* coeffs, float* out, void* stream);
/* dcoeffs [in, out, degree + 1] = dout_grad [in, out, degree + 1 + order] R^T
 * (the gradient of ckan_derivative_coeffs). */
int ckan_derivative_coeffs_backward(const ckan_desc* desc, const ckan_basis_spec* spec,
                                    int32_t order, const float* dout_grad, float* dcoeffs,
                                    void* stream);
/* jac [batch, out, in]: jac[b, o, i] = d y[b, o] / d x[b, i] for x [batch, in]
 * and fp32 coeffs; the workspace holds the order-1 coefficients re-laid out. */
size_t ckan_jacobian_workspace_bytes(const ckan_desc* desc);
int ckan_jacobian(const ckan_desc* desc, const ckan_basis_spec* spec, const float* x,
                  const float* coeffs, float* jac, void* ws, size_t ws_bytes, void* stream);

/* out[n, d] = T_d(t[n]) for d = 0..degree (fp32).  Replaces
 * ChebyshevBasis.basis_functions (kan/basis/chebyshev.py:103-172). */
int ckan_basis(const float* t, int64_t n, int32_t degree, float* out, void* stream);
/* d_t[n] = sum_d g[n, d] d U_{d-1}(t[n]): backward of ckan_basis. */
int ckan_basis_backward(const float* t, const float* g, int64_t n, int32_t degree,
                        float* dt, void* stream);

/* ---- optimizers (in place, fp32) ---------------------------------------- */

/* p -= lr * (g + weight_decay * p).  Replaces torch.optim.SGD.step without
 * momentum (torch/optim/sgd.py, used by configs 2 and 4). */
int ckan_sgd_step(float* p, const float* g, int64_t n, float lr, float weight_decay,
                  void* stream);

/* Adam in torch's single-tensor order (torch/optim/adam.py; README.md:59,66):
 *   g' = g + wd p;  m = lerp(m, g', 1 - b1);  v = b2 v + (1 - b2) g'^2;
 *   p -= (lr / (1 - b1^step)) * m / (sqrt(v) / sqrt(1 - b2^step) + eps).
 * `step` is the step count after increment (1 on the first call). */
int ckan_adam_step(float* p, const float* g, float* m, float* v, int64_t n, int64_t step,
                   double lr, double beta1, double beta2, double eps, double weight_decay,
                   void* stream);

/* ---- resident multi-layer executor ---------------------------------------- */
/* A stack of ChebyKAN layers (KANSequential, kan/layers/base.py:144-166)
 * trained in place on one GPU: the executor owns fp32 master coefficients,
 * their packed operands, activations, tanh caches, gradients, optimizer state
 * and workspaces, allocated once at creation.  One ckan_exec_step runs
 * forward, the loss and its gradient, backward and the optimizer update for
 * every layer, the work of one iteration of the reference's training loop
 * (README.md:61-69) over a KANSequential. */

typedef struct ckan_exec ckan_exec;  /* opaque */

typedef enum ckan_loss {
  CKAN_LOSS_MSE = 0,  /* torch.nn.MSELoss(): mean over all B x out elements   */
  CKAN_LOSS_CE = 1    /* torch.nn.CrossEntropyLoss(): mean over B; int64 labels */
} ckan_loss;

typedef enum ckan_optimizer {
  CKAN_OPT_SGD = 0,   /* torch.optim.SGD (no momentum)  */
  CKAN_OPT_ADAM = 1   /* torch.optim.Adam (no amsgrad)  */
} ckan_optimizer;

typedef struct ckan_exec_config {
  int32_t n_layers;        /* >= 1                                          */
  const int32_t* widths;   /* host array, n_layers + 1 entries              */
  const int32_t* degrees;  /* host array, n_layers entries                  */
  int64_t batch;           /* rows per step (fixed for the executor)        */
  int32_t compute;         /* ckan_compute                                  */
  int32_t loss;            /* ckan_loss                                     */
  int32_t optimizer;       /* ckan_optimizer                                */
  int32_t use_graph;       /* replay each step as a captured HIP graph      */
  float lr, beta1, beta2, eps, weight_decay;
  int32_t flags;           /* ckan_exec_flags, 0 for the defaults           */
} ckan_exec_config;

typedef enum ckan_exec_flags {
  /* A stack whose step is at most 2^18 multiply-adds (e.g. the README's
   * ChebyKANLayer(1, 1, 8) on 100 points) runs each step as one launch of a
   * single-workgroup kernel instead of the per-layer kernel sequence; this
   * flag keeps the kernel sequence for such stacks too. */
  CKAN_EXEC_NO_FUSED_SMALL = 1,
  /* A two-layer cross-entropy stack of small layers (e.g. 784 -> 64 -> 10)
   * keeps its packed operands current from the step's dC launch, which
   * writes them from the updated coefficients, so its steps run no pack
   * launch; this flag packs at every step instead (the same bits). */
  CKAN_EXEC_PACK_EACH_STEP = 2
} ckan_exec_flags;

/* Allocates every device buffer; coefficients start at zero (set them with
 * ckan_exec_set_coeffs).  `stream` orders the initialisation. */
int ckan_exec_create(const ckan_exec_config* cfg, ckan_exec** out, void* stream);
/* ckan_exec_create for a KANSequential whose layers may be JacobiKANLayer
 * (kan/layers/jacobikan.py:64-78) or HermiteKANLayer
 * (kan/layers/hermitekan.py:68-82).  `bases` holds n_layers basis specs (host
 * array; spec.degree must equal degrees[l]; a Chebyshev spec of scale 1 is the
 * plain ChebyKAN layer), NULL for a stack of ChebyKAN layers.  `affine` (host
 * array of 2 * n_layers floats, or NULL) gives layer l the input map
 * t = affine[2l] * x + affine[2l+1] (CKAN_INPUT_AFFINE: the Hermite layer's
 * finite domain) in place of tanh; (0, 0) keeps tanh.  A layer's
 * coefficients (ckan_exec_set/get_coeffs, Adam state) are those of its own
 * basis.  Family layers up to degree 16 train through the change of basis
 * into Chebyshev coefficients (gradient mapped back by the transpose before
 * the optimizer step); above it, on the vector-ALU recurrence. */
int ckan_exec_create_basis(const ckan_exec_config* cfg, const struct ckan_basis_spec* bases,
                           const float* affine, ckan_exec** out, void* stream);
int ckan_exec_destroy(ckan_exec* ex);
/* Device-to-device copy of one layer's fp32 master coefficients [in, out, D]. */
int ckan_exec_set_coeffs(ckan_exec* ex, int32_t layer, const float* src, void* stream);
int ckan_exec_get_coeffs(ckan_exec* ex, int32_t layer, float* dst, void* stream);
/* Adam moments of one layer (fp32, [in, out, D] each) and the step count,
 * for checkpoint/resume; SGD has none (returns CKAN_ERR_UNSUPPORTED). */
int ckan_exec_get_adam_state(ckan_exec* ex, int32_t layer, float* m, float* v,
                             int64_t* step, void* stream);
int ckan_exec_set_adam_state(ckan_exec* ex, int32_t layer, const float* m, const float* v,
                             int64_t step, void* stream);
/* One training step on x [batch, widths[0]] (fp32, device) and target:
 * fp32 [batch, widths[n]] for MSE or int64 [batch] class indices for CE.
 * Writes the step's loss (fp32 scalar, device) to loss_out when non-NULL.
 * CE labels must lie in [0, widths[n]): there is no ignore_index, every row
 * counts in the mean, and the kernels do not check the labels (an
 * out-of-range label reads nothing out of bounds but leaves the loss and its
 * gradient without that row's target term).  The Python wrapper rejects such
 * labels before the launch, as torch.nn.CrossEntropyLoss would. */
int ckan_exec_step(ckan_exec* ex, const float* x, const void* target, float* loss_out,
                   void* stream);
/* `nsteps` training steps on the same x and target (the reference loop's
 * full-batch epochs, README.md:61-69), issued from the library without a
 * return to the caller between steps; step k's loss goes to losses[k] (fp32,
 * device, nsteps entries) when losses is non-NULL.  Runs eagerly (no graph). */
int ckan_exec_steps(ckan_exec* ex, const float* x, const void* target, int64_t nsteps,
                    float* losses, void* stream);
/* Forward only: y [batch, widths[n]] (fp32, device). */
int ckan_exec_forward(ckan_exec* ex, const float* x, float* y, void* stream);

/* ---- diagnostics --------------------------------------------------------- */

const char* ckan_last_error(void);
const char* ckan_version(void);
/* Per-kernel HIP-event timing on the launch stream (off by default). */
int ckan_profile_enable(int on);
/* Writes "name count total_ms\n" lines (synchronises on the recorded events)
 * and clears the records.  Returns the number of bytes needed. */
size_t ckan_profile_report(char* buf, size_t len);

#ifdef __cplusplus
}
#endif

#endif /* CHEBYKAN_H */
