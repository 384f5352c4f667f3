// Launch interface between the C-ABI host code and the kernels, and the
// byte layout of the packed-coefficient buffer and the workspaces.
#pragma once

#include "ckan_common.hpp"

namespace ckan {

inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
// 16-byte aligned: the float4 load paths of x, dy and C require it.
inline bool is_al16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

// Sets the thread-local message returned by ckan_last_error().
void set_last_error(const char* msg);

// ---- packed coefficients: [Cf][Cb][bias partials][bias] -------------------
// Cf: forward B operand, C[i, o, d] for d >= 1 by (input, degree) k-blocks.
// Cb: dX B operand, d * C[i, o, d] (the factor of dT_d/dt = d U_{d-1}) by
// (input block, degree) and output k-blocks.
inline size_t packed_cf_elems(const Plan& p) { return (size_t)p.NBf * p.KB * kFragElems; }
inline size_t packed_cb_elems(const Plan& p) { return (size_t)p.NIB * p.P * p.KBx * kFragElems; }
inline size_t packed_bias_offset(const Plan& p) {
  return align256((packed_cf_elems(p) + packed_cb_elems(p)) * p.esz);
}
// final per-output bias sum_i C[i, o, 0], reduced from the partials
inline size_t packed_biasf_offset(const Plan& p) {
  return align256(packed_bias_offset(p) + (size_t)p.NIB * p.O32 * sizeof(float));
}
inline size_t packed_bytes(const Plan& p) {
  return align256(packed_biasf_offset(p) + (size_t)p.O32 * sizeof(float));
}

// ---- forward: tile configuration and split-K -------------------------------
// Tile shapes (waves along M x waves along N, fragments per wave M x N):
enum FwdTile {
  kFwdBig = 0, kFwdSmall32 = 1, kFwdSmall64 = 2, kFwdStream32 = 3, kFwdStream64 = 4,
  kFwdCols = 5,   // B <= 16, bf16: column-owning blocks, one launch (tanh in the kernel up to 8 rows)
  kFwdSmall64N2 = 6  // 64 rows x 2 output fragments, 2 x 2 waves (outputs <= 64: no idle wave column)
};
struct FwdChoice {
  int tile;           // FwdTile
  int bm, bnf;        // block rows, block N fragments
  int tiles_m, tiles_n;
  int splits, sg_per_split;
};
FwdChoice choose_fwd(const Plan& p);
inline bool fwd_streaming(const FwdChoice& c) { return c.tile == kFwdStream32 || c.tile == kFwdStream64; }
// The 32-row streaming forward and the column-owning forward up to
// kColsTanhRows rows compute tanh themselves (each value is needed by every
// column block, cheap at few rows); every other path reads the tanh cache
// written by launch_tanh first.  At the config-5 shape (2048 -> 2048, degree
// 8) the column-owning forward at 8 rows takes 15.6 us cold with its own tanh
// against 17.0 us with the cache and its launch; at 16 rows 19.4 against 17.9
// (the tanh per basis vector makes it vector-ALU-bound there).
constexpr int kColsTanhRows = 8;
inline bool fwd_reads_tcache(const FwdChoice& c) {
  return c.tile != kFwdStream32 && !(c.tile == kFwdCols && c.bm <= kColsTanhRows);
}
// split-K partials [splits][B32][O32] fp32, summed in order by k_fwd_reduce
inline size_t fwd_ws_bytes(const Plan& p, const FwdChoice& c) {
  if (c.splits <= 1 && !fwd_streaming(c)) return 0;
  return align256((size_t)c.splits * p.B32 * p.O32 * sizeof(float));
}

// ---- backward workspace: [dYx][dYc][colsum partials][dC split partials] ----
// dc_pipe: the pipelined dC kernel writes dC (dc_splits == 1) or split slices
// [split][I][O][D] summed by launch_dc_sum; otherwise partials
// [split][P][I32][O32] go through launch_dc_finalize.
struct BwdLayout {
  size_t dyx_off, dyc_off, colsum_off, part_off, total;
  int dc_splits, dc_st_per_split;
  bool dc_pipe;
  bool dc_small;  // dC by launch_dc_small (no dy re-layout, no partials)
  bool dx_small;  // dx by launch_dx_small (no dy re-layout)
};
BwdLayout bwd_layout(const Plan& p, bool need_dx, bool need_dc);

// ---- other polynomial bases expressed in the Chebyshev basis --------------
constexpr int kMaxD = 17;  // degree <= 16
// Change of basis P_n(s u) = sum_k m[n * kMaxD + k] T_k(u), zero-padded.
struct BasisXform { float m[kMaxD * kMaxD]; };
// Recurrence coefficients (double) of a ckan_basis_family; false if the
// family or its parameters are invalid.
bool family_recurrence(int family, int degree, double alpha, double beta, double* a, double* b,
                       double* c);
// The coefficients of degree n alone (a = b = c = 0 for n = 0); false as above.
__host__ __device__ bool recur_coef(int family, int n, double alpha, double beta, double* a,
                                    double* b, double* c);
// M[n * (degree + 1) + k] with P_n(scale u) = sum_k M[n, k] T_k(u) (exact, fp64).
void family_to_chebyshev(const double* a, const double* b, const double* c, int degree,
                         double scale, double* M);
// g[q, n] = sum_k dcheb[q, k] m[n][k] over the I*O rows q, written into dc
// by om (store, accumulate, or an SGD / Adam step on the parameter dc with
// om.base == dc); dcheb may be dc.
void launch_coeff_from_cheb(const float* dcheb, float* dc, const Plan& p, const DcOut& om,
                            const BasisXform& xf, hipStream_t s);
// out[q, n] = P_n(t[q]) (n <= deg <= kValuMaxDegree) and its backward; the
// recurrence coefficients are formed on the device (recur_coef).
void launch_basis_family(const float* t, int64_t n, int deg, int family, double alpha,
                         double beta, float* out, hipStream_t s);
void launch_basis_family_bwd(const float* t, const float* g, int64_t n, int deg, int family,
                             double alpha, double beta, float* dt, hipStream_t s);

// ---- derivatives of a layer's univariate functions w.r.t. its input ---------
// f(x) = sum_k c_k T_k(tanh x) has d/dx f = (1 - t^2) f'(t): again a Chebyshev
// series in t = tanh x, one degree higher.  R[n * (D + order) + k] (fp64,
// exact up to rounding) maps row n of M (the family's change of basis, D x D)
// through `order` such steps (R has degree + 1 rows of degree + 1 + order).
bool derivative_to_chebyshev(const double* M, int degree, int order, double* R);
// The same for the affine input map t = a x + b: d/dx f = a f'(t), the plain
// Chebyshev derivative (one degree lower), so R (same shape, D + order
// columns) holds a^order times row n of M differentiated `order` times, its
// last 2 * order columns zero.
bool affine_derivative_to_chebyshev(const double* M, int degree, int order, double a,
                                    double* R);
// out = in R over rows q of `rows`: in [rows][din], R [din][dout] (row-major,
// r[n * kMaxD + k]).  transposed_o > 0 writes out as [o][dout][i] for rows
// q = i * transposed_o + o (the Jacobian's layout), else [rows][dout].
void launch_coeff_xform(const float* in, float* out, int64_t rows, int din, int dout,
                        int transposed_o, const BasisXform& r, hipStream_t s);
// The derivative operator (adjoint: its transpose) applied row by row on the
// device, for Chebyshev series of any degree: in [rows][D] -> out [rows][D +
// order] (adjoint: [rows][D + order] -> [rows][D]); transposed_o > 0 writes
// [o][dout][i] as launch_coeff_xform does.
void launch_cheb_deriv_rows(const float* in, float* out, int64_t rows, int degree, int order,
                            bool adjoint, int transposed_o, hipStream_t s);
// jac[b, o, i] = sum_k C1t[o][k][i] T_k(t[b, i]), k < dout, t the input map
// (imap, ima, imb as in input_map) of x.
void launch_jacobian(const float* x, const float* c1t, float* jac, int64_t B, int I, int O,
                     int dout, int imap, float ima, float imb, hipStream_t s);

// ---- vector-ALU path (ckan_valu.hip): any degree, T = float or double ------
// Serves fp64 layers and fp32 layers above kMfmaMaxDegree, with C in its own
// [I, O, D] layout; t = input map of x, [B, I].  rec: the recurrence block
// (a[D], b[D], c[D], scale, kind) in the element type (fp32: the packed
// buffer's; fp64: written by launch_write_recur_f64); nullptr (and kind 0)
// selects the Chebyshev kernels' specialised recurrence.
constexpr int kMfmaMaxDegree = 16;   // the packed MFMA kernels' limit
constexpr int kValuMaxDegree = 1024;  // the vector-ALU path's limit
// Input derivatives: degree + order at most this (the series' coefficients
// grow like n^(2 order), past fp32's useful range well before 1024).
constexpr int kDerivMaxDegree = 256;
template <typename T>
void launch_forward_valu(const T* x, const T* C, T* y, T* t, int64_t B, int I, int O, int deg,
                         hipStream_t s, const T* rec = nullptr, int imap = 0, float ima = 0.0f,
                         float imb = 0.0f);
// dC written by mode om.mode (for T = double: store or accumulate only).
template <typename T>
void launch_backward_valu(const T* t, const T* C, const T* dy, T* dx, T* dC, DcOut om, int64_t B,
                          int I, int O, int deg, hipStream_t s, const T* rec = nullptr,
                          int imap = 0, float ima = 0.0f);
// The recurrence block (a[D], b[D], c[D], scale, kind) of a ckan_basis_family.
void launch_write_recur(float* rec, int family, double alpha, double beta, int degree, float scale,
                        hipStream_t s);
void launch_write_recur_f64(double* rec, int family, double alpha, double beta, int degree,
                            double scale, hipStream_t s);
// dst[q] = float(src[q]) (accumulate: dst[q] += float(src[q])) for q < n, src
// fp32 or bf16.
void launch_to_f32(const void* src, bool src_bf16, float* dst, int64_t n, hipStream_t s,
                   bool accumulate = false);
// Floats of the recurrence block of a layer of degree `degree`.
inline int64_t recur_floats(int degree) { return 3 * (int64_t)(degree + 1) + 2; }

// ---- launchers -------------------------------------------------------------
void launch_tanh(const float* x, float* t, const Plan& p, hipStream_t s);
// xf (optional, host struct passed by value to the kernel): pack C xf instead of C.
// reduce_bias = false leaves only the per-input-block bias partials (for a
// forward that sums them itself).  With x and t (pack_tanh_fusable(p, x)), the
// same launch also writes t = tanh(x) (the forward's tanh cache).
void launch_pack(const void* C, bool c_bf16, void* packed, const Plan& p, hipStream_t s,
                 const BasisXform* xf = nullptr, bool reduce_bias = true,
                 const float* x = nullptr, float* t = nullptr);
// x's tanh can ride in the pack launch: rows need no padding (I == I_sg),
// I % 4 == 0, x is 16-byte aligned (the flat float4 layout) and the pack's
// blocks cover the tanh stream in one pass each.
bool pack_tanh_fusable(const Plan& p, const float* x);
void launch_prep_dy(const float* dy, void* dYx, void* dYc, float* colsum_part, const Plan& p,
                    bool need_dx, bool need_dc, hipStream_t s);
// reduces the dy column-sum partials into row NBB and returns that row
float* launch_colsum_reduce(float* colsum_part, const Plan& p, hipStream_t s);
void launch_dc_finalize(const float* part, int S, const float* colsum, float* dC,
                        DcOut om, const Plan& p, hipStream_t s);
void launch_dc_sum(const float* part, int S, float* dC, DcOut om, const Plan& p, hipStream_t s);
// x is read only by the small-batch streaming kernel, which also writes t;
// the other paths read t written by launch_tanh.
// sum_bias: the packed buffer holds only the bias partials (launch_pack with
// reduce_bias = false) and the forward must reduce them; the pipelined kernel
// does so in its epilogue (and fills the bias slot) when fwd_sums_bias holds,
// the caller launches the reduction first otherwise.
// out_tanh: store tanh(y) in place of y (the next layer's tanh cache in a
// stack; needs fwd_out_tanh_ok).
// xt (needs fwd_maps_x_ok): the GEMM reads x, maps it itself and writes the
// tanh cache t (no launch_tanh before it).
void launch_fwd_gemm(const float* x, float* t, const void* packed, float* y, void* ws,
                     const Plan& p, const FwdChoice& c, hipStream_t s, bool sum_bias = false,
                     bool out_tanh = false, bool reduce = true, bool xt = false);
bool fwd_maps_x_ok(const Plan& p, const FwdChoice& c, const float* x);
// reduce = false above leaves a split forward's partials in ws for
// launch_fwd_tail_ce, which sums them (the last two layers of a stack
// trained with cross-entropy, when fwd_tail_ce_ok holds): layer a's split
// sum into b's tanh cache tb, layer b's forward from its fp32 coefficients
// Cb [Ib = a.O, Ob, Db] into yb, and the rows' cross-entropy gradient dyb and
// losses loss_part (their mean: k_sum_scalar).
// dxa (optional): also layer b's dX into dxa [B, a.O] (dL/dy_a; b's input
// map tanh), the bits of launch_dx_small on b's packed dX operand.
bool fwd_tail_ce_ok(const Plan& pa, const FwdChoice& ca, int Ob, int Db);
void launch_fwd_tail_ce(const void* packed_a, void* ws, const Plan& pa, const FwdChoice& ca,
                        bool sum_bias, float* tb, const float* Cb, int Ob, int Db, float* yb,
                        const int64_t* labels, float* dyb, float* loss_part, hipStream_t s,
                        float* dxa = nullptr);
bool fwd_sums_bias(const Plan& p, const FwdChoice& c);
// The forward path of p can store tanh(y) in place of y (the pipelined
// kernel, unsplit).
bool fwd_out_tanh_ok(const Plan& p);
// bias = sum of the per-input-block partials, into the packed buffer's bias slot
void launch_bias_reduce(void* packed, const Plan& p, hipStream_t s);
void launch_dx_gemm(const void* dYx, const void* packed, const float* t, float* dx,
                    const Plan& p, hipStream_t s);
// colsum: the per-64-row column-sum partials for the pipelined kernel (which
// reduces them itself), the reduced row otherwise.
// Small, latency-bound dC (few rows, few (input, output) pairs): fp32 on the
// vector ALU straight from dy and the tanh cache, one launch, written by om.
bool dc_small_ok(const Plan& p);
// Small, latency-bound dx (few outputs to reduce over): fp32 on the vector ALU
// from dy, the packed dX operand (degree-scaled C) and the tanh cache.
bool dx_small_ok(const Plan& p);
void launch_dx_small(const float* dy, const void* packed, const float* t, float* dx,
                     const Plan& p, hipStream_t s);
void launch_dc_small(const float* dy, const float* t, float* dC, DcOut om, const Plan& p,
                     hipStream_t s);
// launch_dx_small and launch_dc_small of one layer as one launch, for layers
// where that is one round of blocks (bwd_small_one_launch)
bool bwd_small_one_launch(const Plan& p);
void launch_bwd_small(const float* dy, const void* packed, const float* t, float* dx, float* dC,
                      DcOut om, const Plan& p, hipStream_t s,
                      LossMean lm = LossMean{});
// The small dC with an optimizer step (om: kDcSgd or kDcAdam on C) that also
// writes the layer's packed operands from the updated coefficients, bit for
// bit as launch_pack would write them from C after the step: the forward
// operand and bias partials (cf; the bias partials are those of a forward
// that sums them, reduce_bias = false) and the dX operand (cb).  Other
// entries of `packed` (padding, and the parts not requested) keep what the
// last pack wrote.  dc_pack_ok: dc_small_ok and P <= 8.
struct DcPackArgs {
  const float* dy;
  const float* t;
  float* C;
  DcOut om;
  Plan p;
  void* packed;
  bool cf, cb;
};
bool dc_pack_ok(const Plan& p);
// a and b (optional, same P and compute type) in one launch, with the loss
// mean lm (optional) by one more block.
void launch_dc_pack(const DcPackArgs& a, const DcPackArgs* b, hipStream_t s,
                    LossMean lm = LossMean{});
void launch_loss_mean(const LossMean& lm, hipStream_t s);
// xf: the gradient is wanted in another family's basis; the pipelined dC
// applies it before its stores where dc_gemm_maps_basis says so (one unsplit
// launch writes the whole gradient) and ignores it otherwise.
void launch_dc_gemm(const void* dYc, const float* t, const float* colsum, float* part, float* dC,
                    DcOut om, const Plan& p, const BwdLayout& L, hipStream_t s,
                    const BasisXform* xf = nullptr);
bool dc_gemm_maps_basis(const Plan& p, const BwdLayout& L);
void launch_sgd(float* p, const float* g, int64_t n, float lr, float wd, hipStream_t s);
// ckan_backward with the dC write mode given by om; with om.mode kDcSgd or
// kDcAdam, dcoeffs is the parameter and receives its optimizer step (batch
// >= 1 only).  lm (optional): a loss mean taken along, by one more block of
// the small one-launch backward where that path runs, else by one launch
// after the backward.
int backward_impl(const struct ckan_desc* desc, const float* t_cache, const void* packed,
                  const float* dy, float* dx, float* dcoeffs, DcOut om, void* ws,
                  size_t ws_bytes, void* stream, const LossMean* lm = nullptr);
// ckan_pack_forward (no basis spec) for a layer inside a stack: t_ready, the
// tanh cache already holds the layer's input map (x unused; the layer's
// forward must read the cache); out_tanh, store tanh(y) into `out` (the next
// layer's tanh cache) in place of y (needs fwd_out_tanh_ok).
// spec: the layer's basis (nullptr: Chebyshev), as in ckan_pack_forward.
int pack_forward_ex(const struct ckan_desc* desc, const void* coeffs, void* packed,
                    const float* x, float* out, float* t_cache, void* ws, size_t ws_bytes,
                    void* stream, bool t_ready, bool out_tanh,
                    const struct ckan_basis_spec* spec = nullptr);
// Whether the layer runs on the vector-ALU path (degree > kMfmaMaxDegree),
// whose backward differentiates in the layer's own basis.
bool layer_on_valu(const struct ckan_desc* desc);
// Validates a basis spec for a layer of degree `degree`; on the MFMA path
// (degree <= kMfmaMaxDegree) also forms its change of basis into *xf (when
// xf is given).  Sets the last error on failure.
int basis_check(const struct ckan_basis_spec* spec, int degree, BasisXform* xf);
// Whether the layer of desc can take t_ready / out_tanh in pack_forward_ex.
bool layer_reads_tcache(const struct ckan_desc* desc);
bool layer_out_tanh_ok(const struct ckan_desc* desc);
// Two consecutive layers a, b of a stack whose forward a stores tanh(y) into
// b's tanh cache tb: both packs in one launch (b's pack needs nothing of a),
// then a's forward, then b's (t_ready; out_tanh into outb when outb_tanh).
// pack_pair_fits: the pair allows it (fp32 coefficients, Chebyshev kernels on
// both, same padded degree and compute type, a's tanh output, b's cache read).
bool pack_pair_fits(const struct ckan_desc* a, const struct ckan_desc* b);
int pack2_forward_ex(const struct ckan_desc* da, const void* Ca, void* pka, const float* xa,
                     float* ta, bool ta_ready, const struct ckan_desc* db, const void* Cb,
                     void* pkb, float* tb, float* outb, bool outb_tanh, void* ws, size_t ws_bytes,
                     void* stream);
// pack2_forward_ex for the last two layers of a stack trained with
// cross-entropy (labels: int64 class per row): a's forward leaves its split
// partials, and one launch sums them into tb, runs b's forward into yb on the
// vector ALU and writes the rows' CE gradient dyb and losses loss_part (their
// mean is the caller's k_sum_scalar).  pack2_tail_ce_fits: the pair allows it
// (pack_pair_fits, fp32 compute, a split forward for a, a.O <= 64, b.O <= 16,
// b.degree <= 16, a.O * b.O * (b.degree + 1) <= 8192, B <= 4096).
bool pack2_tail_ce_fits(const struct ckan_desc* a, const struct ckan_desc* b);
int pack2_forward_tail_ce(const struct ckan_desc* da, const void* Ca, void* pka, const float* xa,
                          float* ta, bool ta_ready, const struct ckan_desc* db, const void* Cb,
                          void* pkb, float* tb, float* yb, const int64_t* labels, float* dyb,
                          float* loss_part, void* ws, size_t ws_bytes, void* stream);
// A two-layer stack trained with cross-entropy whose packed operands the
// step's dC launch keeps current, so that the step runs no pack:
// self_pack_pair_fits: pack2_tail_ce_fits, both layers on the small dC path
// with the packing epilogue (dc_pack_ok), b's dX on the small path, same P and
// compute type, a's bias summed from its partials by the tail.
// self_pack_layer: the pack that makes `packed` current after C changes other
// than by a step (creation, a copy into C); the packs of the per-step path
// without the tanh, so the same bytes.
// forward_tail_ce_packed: pack2_forward_tail_ce without the pack (a's GEMM
// maps x itself where fwd_maps_x_ok holds, else launch_tanh first); the tail
// also writes b's dX into dya (a's dy).
// backward_self_packed: one launch of both layers' dC with the optimizer step
// (oma, omb: kDcSgd or kDcAdam) that writes a's forward operand and bias
// partials and b's dX operand from the updated coefficients (a, the first
// layer, has no dX), and takes the loss mean lm along.
bool self_pack_pair_fits(const struct ckan_desc* a, const struct ckan_desc* b);
int self_pack_layer(const struct ckan_desc* desc, const void* C, void* packed, void* stream);
int forward_tail_ce_packed(const struct ckan_desc* da, const void* pka, const float* xa, float* ta,
                           const struct ckan_desc* db, const void* Cb, float* tb, float* yb,
                           const int64_t* labels, float* dyb, float* loss_part, float* dya,
                           void* ws, size_t ws_bytes, void* stream);
int backward_self_packed(const struct ckan_desc* da, const float* ta, const float* dya, float* Ca,
                         const DcOut& oma, void* pka, const struct ckan_desc* db, const float* tb,
                         const float* dyb, float* Cb, const DcOut& omb, void* pkb,
                         const LossMean& lm, void* stream);
// the Plan-level launch behind pack2_forward_ex (xa, ta: a's fused tanh, or null)
bool pack_pair_ok(const Plan& a, const Plan& b);
void launch_pack_pair(const float* Ca, void* pa, const Plan& qa, bool reduce_a, const float* xa,
                      float* ta, const float* Cb, void* pb, const Plan& qb, bool reduce_b,
                      hipStream_t s);
void launch_adam(float* p, const float* g, float* m, float* v, int64_t n, float w1, float beta2,
                 float one_m_beta2, float bc2_sqrt, float eps, float neg_step, float wd,
                 hipStream_t s);
void launch_basis(const float* t, int64_t n, int deg, float* out, hipStream_t s);
void launch_basis_bwd(const float* t, const float* g, int64_t n, int deg, float* dt,
                      hipStream_t s);
void launch_zero(void* ptr, size_t bytes, hipStream_t s);
void launch_zero_f32(float* ptr, int64_t n, hipStream_t s);

// dX / dC tile shapes (fragments per wave along M; 4 waves along M).
// NM * P = 16 fragments (256 accumulator registers per lane), capped at 4
// fragments along M so the P = 2 tile does not spill.
template <int P> struct BwdTile {
  static constexpr int NM = (16 / P) < 4 ? (16 / P) : 4;
  static constexpr int WGM = 4;
};
inline int bwd_nm(int P) { return (16 / P) < 4 ? (16 / P) : 4; }
// dX row fragments (32 rows each) padded to whole tiles of 4 waves x NM
// fragments; the padding fragments of dYx hold zeros.
// dY re-layout rows for dx, in 32-row fragments, zero-padded to whole row
// blocks of the dx kernel (256 rows; 128 for fp32 at degree 16)
inline int64_t dx_row_frags(const Plan& p) {
  return round_up(p.B32 / 32, p.P == 16 && p.esz == 2 ? 8 : 4 * bwd_nm(p.P));
}

}  // namespace ckan
