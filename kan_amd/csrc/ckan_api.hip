// C-ABI entry points (include/chebykan.h): argument checks on the host,
// workspace carving, kernel sequencing on the caller's stream, and optional
// per-kernel HIP-event timing.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "chebykan.h"
#include "ckan_kernels.hpp"

using namespace ckan;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(CKAN_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return CKAN_OK;
}

// ---- per-kernel event timing ------------------------------------------------
struct ProfRec {
  const char* name;
  hipEvent_t a, b;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<ProfRec> g_prof;

struct ProfScope {
  ProfRec rec{};
  bool on;
  hipStream_t s;
  ProfScope(const char* name, hipStream_t st) : s(st) {
    {
      std::lock_guard<std::mutex> lk(g_prof_mu);
      on = g_prof_on;
    }
    if (!on) return;
    rec.name = name;
    if (hipEventCreate(&rec.a) != hipSuccess || hipEventCreate(&rec.b) != hipSuccess) {
      on = false;
      return;
    }
    hipEventRecord(rec.a, s);
  }
  ~ProfScope() {
    if (!on) return;
    hipEventRecord(rec.b, s);
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof.push_back(rec);
  }
};

int validate_desc(const ckan_desc* d) {
  if (!d) return fail(CKAN_ERR_INVALID_ARG, "desc is NULL");
  if (d->batch < 0) return fail(CKAN_ERR_INVALID_ARG, "batch must be >= 0 (got %lld)", (long long)d->batch);
  if (d->in_dim < 1) return fail(CKAN_ERR_INVALID_ARG, "in_dim must be >= 1 (got %d)", d->in_dim);
  if (d->out_dim < 1) return fail(CKAN_ERR_INVALID_ARG, "out_dim must be >= 1 (got %d)", d->out_dim);
  if (d->degree < 0) return fail(CKAN_ERR_INVALID_ARG, "degree must be >= 0 (got %d)", d->degree);
  if (d->degree > kValuMaxDegree)
    return fail(CKAN_ERR_UNSUPPORTED, "degree %d > %d is not supported by this build", d->degree,
                kValuMaxDegree);
  if (d->compute != CKAN_COMPUTE_FP32 && d->compute != CKAN_COMPUTE_BF16)
    return fail(CKAN_ERR_INVALID_ARG, "unknown compute mode %d", d->compute);
  if (d->coeff_dtype != CKAN_DTYPE_F32 && d->coeff_dtype != CKAN_DTYPE_BF16)
    return fail(CKAN_ERR_INVALID_ARG, "unknown coefficient dtype %d", d->coeff_dtype);
  if (d->input_map == CKAN_INPUT_TANH) {
    if (d->in_scale != 0.0f || d->in_shift != 0.0f)
      return fail(CKAN_ERR_INVALID_ARG, "in_scale/in_shift must be 0 with the tanh input map");
  } else if (d->input_map == CKAN_INPUT_AFFINE) {
    if (!isfinite(d->in_scale) || !isfinite(d->in_shift) || d->in_scale == 0.0f)
      return fail(CKAN_ERR_INVALID_ARG, "affine input map needs a finite non-zero in_scale and finite in_shift");
  } else {
    return fail(CKAN_ERR_INVALID_ARG, "unknown input map %d", d->input_map);
  }
  // Index arithmetic inside the kernels uses 64-bit offsets; bound the
  // 32-bit grid dimensions.
  if (d->in_dim > (1 << 20) || d->out_dim > (1 << 20))
    return fail(CKAN_ERR_UNSUPPORTED, "in_dim/out_dim above 2^20 are not supported");
  if (d->batch > ((int64_t)1 << 34))
    return fail(CKAN_ERR_UNSUPPORTED, "batch above 2^34 rows is not supported");
  return CKAN_OK;
}

Plan plan_of(const ckan_desc* d) {
  Plan p = make_plan(d->batch, d->in_dim, d->out_dim, d->degree, d->compute == CKAN_COMPUTE_BF16);
  p.imap = d->input_map;
  p.ima = d->in_scale;
  p.imb = d->in_shift;
  return p;
}

// Layers above the MFMA kernels' degree limit run on the vector-ALU kernels
// in fp32 (whatever desc->compute asks).  Their packed buffer is C copied to
// fp32 in its own [I, O, D] layout, then (at the next 256-byte boundary) the
// basis recurrence block; the input-map cache has row pitch I.
inline bool valu_route(const ckan_desc* d) { return d->degree > kMfmaMaxDegree; }
inline int64_t valu_coeffs(const ckan_desc* d) {
  return (int64_t)d->in_dim * d->out_dim * (d->degree + 1);
}
inline size_t valu_rec_offset(const ckan_desc* d) {
  return align256((size_t)valu_coeffs(d) * sizeof(float));
}
inline float* valu_rec(const ckan_desc* d, void* packed) {
  return reinterpret_cast<float*>(static_cast<char*>(packed) + valu_rec_offset(d));
}
inline const float* valu_rec(const ckan_desc* d, const void* packed) {
  return reinterpret_cast<const float*>(static_cast<const char*>(packed) + valu_rec_offset(d));
}

// The vector-ALU dx launch puts 8 inputs per block on grid y (at most 65535).
int valu_backward_shape_ok(const ckan_desc* d) {
  if ((d->in_dim + 7) / 8 > 65535)
    return fail(CKAN_ERR_UNSUPPORTED, "in_dim %d above 524280 is not supported by the vector-ALU "
                "backward (degree above 16 or fp64)", d->in_dim);
  return CKAN_OK;
}

// Paths that implement only the tanh input map.
int require_tanh_map(const ckan_desc* d, const char* what) {
  if (d->input_map != CKAN_INPUT_TANH)
    return fail(CKAN_ERR_UNSUPPORTED, "%s: only the tanh input map is served", what);
  return CKAN_OK;
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

// ---- fixed scratch of the allocation-free forward ---------------------------
// Each GPU the library runs on holds one copy of this array until the process
// ends.  Host code never passes `scratch` itself to a kernel (on the host the
// name is only a stand-in for the device symbol): the device address is looked
// up once per device by hipGetSymbolAddress, with that device current, and
// kept in g_scratch_ptr.
static __device__ __align__(256) char scratch[CKAN_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`.
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(CKAN_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(CKAN_ERR_UNSUPPORTED, "device %d: at most %d devices are supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(CKAN_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return CKAN_OK;
}
}  // namespace

void ckan::set_last_error(const char* msg) { g_err = msg; }

namespace {
int backward_core(const ckan_desc* desc, const float* t_cache, const void* packed, const float* dy,
                  float* dx, float* dcoeffs, DcOut om, void* ws, size_t ws_bytes, void* stream,
                  const LossMean* lm, bool* lm_used, const BasisXform* xf = nullptr,
                  bool* xf_done = nullptr);
}

int ckan::backward_impl(const ckan_desc* desc, const float* t_cache, const void* packed,
                        const float* dy, float* dx, float* dcoeffs, DcOut om, void* ws,
                        size_t ws_bytes, void* stream, const LossMean* lm) {
  bool used = false;
  const int rc = backward_core(desc, t_cache, packed, dy, dx, dcoeffs, om, ws, ws_bytes, stream,
                               lm && lm->part ? lm : nullptr, &used);
  if (rc || !lm || !lm->part || used) return rc;
  launch_loss_mean(*lm, reinterpret_cast<hipStream_t>(stream));
  return check_launch("loss mean");
}

namespace {
int backward_core(const ckan_desc* desc, const float* t_cache, const void* packed, const float* dy,
                  float* dx, float* dcoeffs, DcOut om, void* ws, size_t ws_bytes, void* stream,
                  const LossMean* lm, bool* lm_used, const BasisXform* xf, bool* xf_done) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  const bool need_dx = dx != nullptr, need_dc = dcoeffs != nullptr;
  if (!need_dx && !need_dc) return CKAN_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (valu_route(desc)) {
    if ((rc = valu_backward_shape_ok(desc))) return rc;
    if (desc->batch == 0) {
      if (need_dc && om.mode >= kDcSgd)
        return fail(CKAN_ERR_UNSUPPORTED, "backward: an optimizer-applying call needs batch >= 1");
      if (need_dc && om.mode == kDcStore) {
        launch_zero_f32(dcoeffs, valu_coeffs(desc), s);
        return check_launch("zero dcoeffs");
      }
      return CKAN_OK;
    }
    // packed carries the basis recurrence: required for dC as well
    if (!t_cache || !dy || !packed) return fail(CKAN_ERR_INVALID_ARG, "t_cache/dy/packed is NULL");
    ProfScope ps("bwd_valu", s);
    launch_backward_valu<float>(t_cache, static_cast<const float*>(packed), dy, dx, dcoeffs, om,
                                desc->batch, desc->in_dim, desc->out_dim, desc->degree, s,
                                packed ? valu_rec(desc, packed) : nullptr, desc->input_map,
                                desc->in_scale);
    return check_launch("backward (vector ALU)");
  }
  const Plan p = plan_of(desc);
  if (p.B == 0) {
    // empty batch: dC = 0 (or unchanged when accumulating), dx is empty
    if (need_dc && om.mode >= kDcSgd)
      return fail(CKAN_ERR_UNSUPPORTED, "backward: an optimizer-applying call needs batch >= 1");
    if (need_dc && om.mode == kDcStore) {
      launch_zero_f32(dcoeffs, (int64_t)p.I * p.O * p.D, s);
      return check_launch("zero dcoeffs");
    }
    return CKAN_OK;
  }
  if (!t_cache || !dy || (need_dx && !packed))
    return fail(CKAN_ERR_INVALID_ARG, "t_cache/dy/packed is NULL");
  if (need_dx && !aligned16(packed)) return fail(CKAN_ERR_INVALID_ARG, "packed must be 16-byte aligned");
  const BwdLayout L = bwd_layout(p, need_dx, need_dc);
  if (ws_bytes < L.total)
    return fail(CKAN_ERR_WORKSPACE, "backward workspace too small: %zu < %zu bytes", ws_bytes, L.total);
  if (L.total > 0 && (!ws || !aligned16(ws)))
    return fail(CKAN_ERR_INVALID_ARG, "workspace is NULL or misaligned");
  char* w = reinterpret_cast<char*>(ws);
  void* dYx = w + L.dyx_off;
  void* dYc = w + L.dyc_off;
  float* colsum = reinterpret_cast<float*>(w + L.colsum_off);
  float* part = reinterpret_cast<float*>(w + L.part_off);
  // the small kernels read dy themselves
  const bool prep_x = need_dx && !L.dx_small, prep_c = need_dc && !L.dc_small;
  if (prep_x || prep_c) {
    ProfScope ps("prep_dy", s);
    launch_prep_dy(dy, dYx, dYc, colsum, p, prep_x, prep_c, s);
  }
  if ((rc = check_launch("prep_dy"))) return rc;
  if (need_dx && L.dx_small && need_dc && L.dc_small && bwd_small_one_launch(p)) {
    ProfScope ps("bwd_small", s);
    launch_bwd_small(dy, packed, t_cache, dx, dcoeffs, om, p, s, lm ? *lm : LossMean{});
    *lm_used = lm != nullptr;
    return check_launch("bwd_small");
  }
  if (need_dx) {
    ProfScope ps("dx_gemm", s);
    if (L.dx_small) launch_dx_small(dy, packed, t_cache, dx, p, s);
    else launch_dx_gemm(dYx, packed, t_cache, dx, p, s);
  }
  if ((rc = check_launch("dx_gemm"))) return rc;
  if (need_dc && L.dc_small) {
    ProfScope ps("dc_gemm", s);
    launch_dc_small(dy, t_cache, dcoeffs, om, p, s);
    return check_launch("dc_small");
  }
  if (need_dc) {
    // the pipelined dC kernel reduces the column-sum partials itself
    const float* colsum_r = nullptr;
    if (!L.dc_pipe) {
      ProfScope ps("colsum", s);
      colsum_r = launch_colsum_reduce(colsum, p, s);
    }
    {
      ProfScope ps("dc_gemm", s);
      const bool map = xf && dc_gemm_maps_basis(p, L);
      launch_dc_gemm(dYc, t_cache, L.dc_pipe ? colsum : colsum_r, part, dcoeffs, om, p, L, s,
                     map ? xf : nullptr);
      if (map && xf_done) *xf_done = true;
    }
    if ((rc = check_launch("dc_gemm"))) return rc;
    if (!L.dc_pipe) {
      ProfScope ps("dc_finalize", s);
      launch_dc_finalize(part, L.dc_splits, colsum_r, dcoeffs, om, p, s);
    } else if (L.dc_splits > 1) {
      ProfScope ps("dc_finalize", s);
      launch_dc_sum(part, L.dc_splits, dcoeffs, om, p, s);
    }
    if ((rc = check_launch("dc_finalize"))) return rc;
  }
  return CKAN_OK;
}

}  // namespace

extern "C" {

const char* ckan_last_error(void) { return g_err.c_str(); }

const char* ckan_version(void) { return "kan_amd-chebykan 0.1.0 (gfx950)"; }

size_t ckan_packed_bytes(const ckan_desc* desc) {
  if (validate_desc(desc) != CKAN_OK) return 0;
  if (valu_route(desc))
    return valu_rec_offset(desc) + align256((size_t)recur_floats(desc->degree) * sizeof(float));
  return packed_bytes(plan_of(desc));
}

size_t ckan_tcache_elems(const ckan_desc* desc) {
  if (validate_desc(desc) != CKAN_OK) return 0;
  if (valu_route(desc)) return (size_t)desc->batch * desc->in_dim;
  const Plan p = plan_of(desc);
  return (size_t)p.B * p.I_sg;
}

size_t ckan_fwd_workspace_bytes(const ckan_desc* desc) {
  if (validate_desc(desc) != CKAN_OK || valu_route(desc)) return 0;
  const Plan p = plan_of(desc);
  if (p.B == 0) return 0;
  return fwd_ws_bytes(p, choose_fwd(p));
}

size_t ckan_bwd_workspace_bytes(const ckan_desc* desc, int need_dx, int need_dcoeffs) {
  if (validate_desc(desc) != CKAN_OK || valu_route(desc)) return 0;
  const Plan p = plan_of(desc);
  return bwd_layout(p, need_dx != 0, need_dcoeffs != 0).total;
}

int ckan_workspace_init(void* ws, size_t ws_bytes, void* stream) {
  if (ws_bytes == 0) return CKAN_OK;
  if (!ws) return fail(CKAN_ERR_INVALID_ARG, "workspace is NULL");
  if (!aligned16(ws) || (ws_bytes & 15))
    return fail(CKAN_ERR_INVALID_ARG, "workspace must be 16-byte aligned and sized");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ProfScope ps("zero", s);
  launch_zero(ws, ws_bytes, s);
  return check_launch("workspace_init");
}

int ckan_pack_coeffs(const ckan_desc* desc, const void* coeffs, void* packed, void* stream) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (!coeffs || !packed) return fail(CKAN_ERR_INVALID_ARG, "coeffs/packed is NULL");
  if (!aligned16(packed)) return fail(CKAN_ERR_INVALID_ARG, "packed buffer must be 16-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (valu_route(desc)) {  // C in fp32 and the Chebyshev recurrence block
    ProfScope ps("pack", s);
    launch_to_f32(coeffs, desc->coeff_dtype == CKAN_DTYPE_BF16, static_cast<float*>(packed),
                  valu_coeffs(desc), s);
    launch_write_recur(valu_rec(desc, packed), CKAN_BASIS_CHEBYSHEV, 0.0, 0.0, desc->degree, 1.0f, s);
    return check_launch("pack_coeffs");
  }
  const Plan p = plan_of(desc);
  ProfScope ps("pack", s);
  launch_pack(coeffs, desc->coeff_dtype == CKAN_DTYPE_BF16, packed, p, s);
  return check_launch("pack_coeffs");
}

int ckan_forward(const ckan_desc* desc, const float* x, const void* packed, float* y,
                 float* t_cache, void* ws, size_t ws_bytes, void* stream) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (desc->batch == 0) return CKAN_OK;
  if (!x || !packed || !y || !t_cache)
    return fail(CKAN_ERR_INVALID_ARG, "x/packed/y/t_cache is NULL");
  if (!aligned16(packed) || !aligned16(t_cache))
    return fail(CKAN_ERR_INVALID_ARG, "packed and t_cache must be 16-byte aligned");
  if (valu_route(desc)) {
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    ProfScope ps("fwd_valu", s);
    launch_forward_valu<float>(x, static_cast<const float*>(packed), y, t_cache, desc->batch,
                               desc->in_dim, desc->out_dim, desc->degree, s,
                               valu_rec(desc, packed), desc->input_map, desc->in_scale,
                               desc->in_shift);
    return check_launch("forward (vector ALU)");
  }
  const Plan p = plan_of(desc);
  const FwdChoice c = choose_fwd(p);
  const size_t need = fwd_ws_bytes(p, c);
  if (ws_bytes < need)
    return fail(CKAN_ERR_WORKSPACE, "forward workspace too small: %zu < %zu bytes", ws_bytes, need);
  if (need && !ws) return fail(CKAN_ERR_INVALID_ARG, "workspace is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (fwd_reads_tcache(c)) {
    ProfScope ps("tanh", s);
    launch_tanh(x, t_cache, p, s);
  }
  if ((rc = check_launch("tanh"))) return rc;
  {
    ProfScope ps("fwd_gemm", s);
    launch_fwd_gemm(x, t_cache, packed, y, ws, p, c, s);
  }
  return check_launch("fwd_gemm");
}

int ckan_forward_noalloc(const ckan_desc* desc, const float* x, const void* packed, float* y,
                         float* t_cache, void* stream) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (desc->batch == 0) return CKAN_OK;
  const size_t need = ckan_fwd_workspace_bytes(desc);
  if (need > CKAN_NOALLOC_SCRATCH_BYTES)
    return fail(CKAN_ERR_WORKSPACE,
                "forward_noalloc: this shape needs %zu bytes of scratch, above the fixed %zu",
                need, (size_t)CKAN_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0 && (rc = scratch_ptr(&ws))) return rc;
  // the split-K partials are written before they are read: nothing in the
  // scratch needs clearing between calls
  return ckan_forward(desc, x, packed, y, t_cache, ws, need > 0 ? (size_t)CKAN_NOALLOC_SCRATCH_BYTES : 0,
                      stream);
}

namespace {
int family_xform(const ckan_basis_spec* spec, int degree, BasisXform* xf);
int family_valid(const ckan_basis_spec* spec, int degree);
}

namespace {
int pack_forward_impl(const ckan_desc* desc, const ckan_basis_spec* spec, const void* coeffs,
                      void* packed, const float* x, float* y, float* t_cache, void* ws,
                      size_t ws_bytes, void* stream, bool t_ready, bool out_tanh);
int forward_packed(const Plan& p, const FwdChoice& c, const void* packed, const float* x, float* y,
                   float* t_cache, void* ws, hipStream_t s, bool t_done, bool sum_in_gemm,
                   bool out_tanh, bool reduce = true);
}

int ckan_pack_forward(const ckan_desc* desc, const ckan_basis_spec* spec, const void* coeffs,
                      void* packed, const float* x, float* y, float* t_cache, void* ws,
                      size_t ws_bytes, void* stream) {
  return pack_forward_impl(desc, spec, coeffs, packed, x, y, t_cache, ws, ws_bytes, stream, false,
                           false);
}

namespace {
int pack_forward_impl(const ckan_desc* desc, const ckan_basis_spec* spec, const void* coeffs,
                      void* packed, const float* x, float* y, float* t_cache, void* ws,
                      size_t ws_bytes, void* stream, bool t_ready, bool out_tanh) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (valu_route(desc)) {
    rc = spec ? ckan_pack_coeffs_basis(desc, spec, coeffs, packed, stream)
              : ckan_pack_coeffs(desc, coeffs, packed, stream);
    if (rc) return rc;
    return ckan_forward(desc, x, packed, y, t_cache, ws, ws_bytes, stream);
  }
  BasisXform xf;
  if (spec && (rc = family_xform(spec, desc->degree, &xf))) return rc;
  if (!coeffs || !packed) return fail(CKAN_ERR_INVALID_ARG, "coeffs/packed is NULL");
  if (!aligned16(packed)) return fail(CKAN_ERR_INVALID_ARG, "packed buffer must be 16-byte aligned");
  const Plan p = plan_of(desc);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool cbf = desc->coeff_dtype == CKAN_DTYPE_BF16;
  if (p.B == 0) {
    ProfScope ps("pack", s);
    launch_pack(coeffs, cbf, packed, p, s, spec ? &xf : nullptr);
    return check_launch("pack_forward");
  }
  if ((!x && !t_ready) || !y || !t_cache) return fail(CKAN_ERR_INVALID_ARG, "x/y/t_cache is NULL");
  if (!aligned16(t_cache)) return fail(CKAN_ERR_INVALID_ARG, "t_cache must be 16-byte aligned");
  const FwdChoice c = choose_fwd(p);
  const size_t need = fwd_ws_bytes(p, c);
  if (ws_bytes < need)
    return fail(CKAN_ERR_WORKSPACE, "forward workspace too small: %zu < %zu bytes", ws_bytes, need);
  if (need && !ws) return fail(CKAN_ERR_INVALID_ARG, "workspace is NULL");
  // the bias partials are summed by the forward GEMM where it can, and the
  // tanh of x rides in the pack launch where the layout allows: fewer launches
  const bool sum_in_gemm = fwd_sums_bias(p, c);
  const bool fuse_tanh = !t_ready && fwd_reads_tcache(c) && pack_tanh_fusable(p, x);
  {
    ProfScope ps(fuse_tanh ? "pack_tanh" : "pack", s);
    launch_pack(coeffs, cbf, packed, p, s, spec ? &xf : nullptr, !sum_in_gemm,
                fuse_tanh ? x : nullptr, fuse_tanh ? t_cache : nullptr);
  }
  if ((rc = check_launch("pack_forward: pack"))) return rc;
  return forward_packed(p, c, packed, x, y, t_cache, ws, s, t_ready || fuse_tanh, sum_in_gemm,
                        out_tanh);
}

// The forward after the pack: the tanh of x unless the cache holds it
// already, then the GEMM.
int forward_packed(const Plan& p, const FwdChoice& c, const void* packed, const float* x, float* y,
                   float* t_cache, void* ws, hipStream_t s, bool t_done, bool sum_in_gemm,
                   bool out_tanh, bool reduce) {
  if (!t_done && fwd_reads_tcache(c)) {
    ProfScope ps("tanh", s);
    launch_tanh(x, t_cache, p, s);
  }
  int rc;
  if ((rc = check_launch("pack_forward: tanh"))) return rc;
  {
    ProfScope ps("fwd_gemm", s);
    launch_fwd_gemm(x, t_cache, packed, y, ws, p, c, s, sum_in_gemm, out_tanh, reduce);
  }
  return check_launch("pack_forward: fwd_gemm");
}
}  // namespace

int ckan_backward(const ckan_desc* desc, const float* t_cache, const void* packed,
                  const float* dy, float* dx, float* dcoeffs, int accumulate, void* ws,
                  size_t ws_bytes, void* stream) {
  const DcOut om{accumulate ? kDcAccumulate : kDcStore};
  return backward_impl(desc, t_cache, packed, dy, dx, dcoeffs, om, ws, ws_bytes, stream);
}

int ckan_basis(const float* t, int64_t n, int32_t degree, float* out, void* stream) {
  if (n < 0 || degree < 0) return fail(CKAN_ERR_INVALID_ARG, "n and degree must be >= 0");
  if (n == 0) return CKAN_OK;
  if (!t || !out) return fail(CKAN_ERR_INVALID_ARG, "t/out is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ProfScope ps("basis", s);
  launch_basis(t, n, degree, out, s);
  return check_launch("basis");
}

int ckan_basis_backward(const float* t, const float* g, int64_t n, int32_t degree, float* dt,
                        void* stream) {
  if (n < 0 || degree < 0) return fail(CKAN_ERR_INVALID_ARG, "n and degree must be >= 0");
  if (n == 0) return CKAN_OK;
  if (!t || !g || !dt) return fail(CKAN_ERR_INVALID_ARG, "t/g/dt is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ProfScope ps("basis_bwd", s);
  launch_basis_bwd(t, g, n, degree, dt, s);
  return check_launch("basis_backward");
}

namespace {
// The fp64 layer; rec: the family's fp64 recurrence block (nullptr: Chebyshev).
int forward_f64_impl(const ckan_desc* desc, const double* rec, const double* x,
                     const double* coeffs, double* y, double* t_cache, void* stream) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (desc->compute != CKAN_COMPUTE_FP32 || desc->coeff_dtype != CKAN_DTYPE_F32)
    return fail(CKAN_ERR_INVALID_ARG, "fp64 path: desc->compute and desc->coeff_dtype must be 0");
  if ((rc = require_tanh_map(desc, "fp64 path"))) return rc;
  if (desc->batch == 0) return CKAN_OK;
  if (!x || !coeffs || !y || !t_cache) return fail(CKAN_ERR_INVALID_ARG, "x/coeffs/y/t_cache is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ProfScope ps("fwd_f64", s);
  launch_forward_valu<double>(x, coeffs, y, t_cache, desc->batch, desc->in_dim,
                              desc->out_dim, desc->degree, s, rec);
  return check_launch("forward_f64");
}

int backward_f64_impl(const ckan_desc* desc, const double* rec, const double* t_cache,
                      const double* coeffs, const double* dy, double* dx, double* dcoeffs,
                      int accumulate, void* stream) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (desc->compute != CKAN_COMPUTE_FP32 || desc->coeff_dtype != CKAN_DTYPE_F32)
    return fail(CKAN_ERR_INVALID_ARG, "fp64 path: desc->compute and desc->coeff_dtype must be 0");
  if ((rc = require_tanh_map(desc, "fp64 path"))) return rc;
  if ((rc = valu_backward_shape_ok(desc))) return rc;
  if (!dx && !dcoeffs) return CKAN_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (desc->batch == 0) {
    if (dcoeffs && !accumulate) {  // fp64 zero is all-zero bits: fill as 2 floats per value
      launch_zero_f32(reinterpret_cast<float*>(dcoeffs),
                      2 * (int64_t)desc->in_dim * desc->out_dim * (desc->degree + 1), s);
      return check_launch("zero dcoeffs");
    }
    return CKAN_OK;
  }
  if (!t_cache || !dy || (dx && !coeffs))
    return fail(CKAN_ERR_INVALID_ARG, "t_cache/dy/coeffs is NULL");
  ProfScope ps("bwd_f64", s);
  const DcOut om{accumulate ? kDcAccumulate : kDcStore};
  launch_backward_valu<double>(t_cache, coeffs, dy, dx, dcoeffs, om, desc->batch, desc->in_dim,
                               desc->out_dim, desc->degree, s, rec);
  return check_launch("backward_f64");
}
}  // namespace

int ckan_forward_f64(const ckan_desc* desc, const double* x, const double* coeffs, double* y,
                     double* t_cache, void* stream) {
  return forward_f64_impl(desc, nullptr, x, coeffs, y, t_cache, stream);
}

int ckan_backward_f64(const ckan_desc* desc, const double* t_cache, const double* coeffs,
                      const double* dy, double* dx, double* dcoeffs, int accumulate, void* stream) {
  return backward_f64_impl(desc, nullptr, t_cache, coeffs, dy, dx, dcoeffs, accumulate, stream);
}

namespace {
// Validates a basis spec (and its degree against `degree` when >= 0) and
// fills the family's recurrence.
int family_of(const ckan_basis_spec* spec, int degree, double* a, double* b, double* c) {
  if (!spec) return fail(CKAN_ERR_INVALID_ARG, "basis spec is NULL");
  if (spec->degree < 0 || spec->degree >= kMaxD)
    return fail(spec->degree < 0 ? CKAN_ERR_INVALID_ARG : CKAN_ERR_UNSUPPORTED,
                "basis degree %d outside 0..%d", spec->degree, kMaxD - 1);
  if (degree >= 0 && spec->degree != degree)
    return fail(CKAN_ERR_INVALID_ARG, "basis degree %d != layer degree %d", spec->degree, degree);
  if (!isfinite(spec->scale)) return fail(CKAN_ERR_INVALID_ARG, "basis scale must be finite");
  if (!family_recurrence(spec->family, spec->degree, spec->alpha, spec->beta, a, b, c))
    return fail(CKAN_ERR_INVALID_ARG, "invalid basis family %d or parameters (alpha=%g, beta=%g; "
                "Jacobi needs alpha, beta > -1)", spec->family, spec->alpha, spec->beta);
  return CKAN_OK;
}

// Validates a basis spec of a layer of degree `degree` up to the vector-ALU
// path's limit (the recurrence-block form of the basis has no matrix).
int family_valid(const ckan_basis_spec* spec, int degree) {
  if (!spec) return fail(CKAN_ERR_INVALID_ARG, "basis spec is NULL");
  if (spec->degree != degree)
    return fail(CKAN_ERR_INVALID_ARG, "basis degree %d != layer degree %d", spec->degree, degree);
  if (!isfinite(spec->scale)) return fail(CKAN_ERR_INVALID_ARG, "basis scale must be finite");
  double a, b, c;
  if (!recur_coef(spec->family, 0, spec->alpha, spec->beta, &a, &b, &c))
    return fail(CKAN_ERR_INVALID_ARG, "invalid basis family %d or parameters (alpha=%g, beta=%g; "
                "Jacobi needs alpha, beta > -1)", spec->family, spec->alpha, spec->beta);
  return CKAN_OK;
}

int family_xform(const ckan_basis_spec* spec, int degree, BasisXform* xf) {
  double a[kMaxD], b[kMaxD], c[kMaxD];
  int rc = family_of(spec, degree, a, b, c);
  if (rc) return rc;
  const int D = spec->degree + 1;
  double M[kMaxD * kMaxD];
  family_to_chebyshev(a, b, c, spec->degree, spec->scale, M);
  for (int i = 0; i < kMaxD * kMaxD; ++i) xf->m[i] = 0.0f;
  for (int n = 0; n < D; ++n)
    for (int k = 0; k < D; ++k) xf->m[n * kMaxD + k] = (float)M[n * D + k];
  return CKAN_OK;
}

}  // namespace

size_t ckan_recurrence_bytes_f64(const ckan_basis_spec* spec) {
  if (!spec || spec->degree < 0 || spec->degree > kValuMaxDegree) return 0;
  return (size_t)(3 * (spec->degree + 1) + 2) * sizeof(double);
}

int ckan_write_recurrence_f64(const ckan_basis_spec* spec, double* rec, void* stream) {
  if (!spec) return fail(CKAN_ERR_INVALID_ARG, "basis spec is NULL");
  if (spec->degree < 0 || spec->degree > kValuMaxDegree)
    return fail(spec->degree < 0 ? CKAN_ERR_INVALID_ARG : CKAN_ERR_UNSUPPORTED,
                "basis degree %d outside 0..%d", spec->degree, kValuMaxDegree);
  int rc = family_valid(spec, spec->degree);
  if (rc) return rc;
  if (!rec) return fail(CKAN_ERR_INVALID_ARG, "rec is NULL");
  if (reinterpret_cast<uintptr_t>(rec) & 7) return fail(CKAN_ERR_INVALID_ARG, "rec must be 8-byte aligned");
  launch_write_recur_f64(rec, spec->family, spec->alpha, spec->beta, spec->degree, spec->scale,
                         reinterpret_cast<hipStream_t>(stream));
  return check_launch("write_recurrence_f64");
}

int ckan_forward_f64_basis(const ckan_desc* desc, const double* rec, const double* x,
                           const double* coeffs, double* y, double* t_cache, void* stream) {
  if (!rec) return fail(CKAN_ERR_INVALID_ARG, "rec is NULL");
  return forward_f64_impl(desc, rec, x, coeffs, y, t_cache, stream);
}

int ckan_backward_f64_basis(const ckan_desc* desc, const double* rec, const double* t_cache,
                            const double* coeffs, const double* dy, double* dx, double* dcoeffs,
                            int accumulate, void* stream) {
  if (!rec) return fail(CKAN_ERR_INVALID_ARG, "rec is NULL");
  return backward_f64_impl(desc, rec, t_cache, coeffs, dy, dx, dcoeffs, accumulate, stream);
}

int ckan_basis_to_chebyshev(const ckan_basis_spec* spec, double* M) {
  double a[kMaxD], b[kMaxD], c[kMaxD];
  int rc = family_of(spec, -1, a, b, c);
  if (rc) return rc;
  if (!M) return fail(CKAN_ERR_INVALID_ARG, "M is NULL");
  family_to_chebyshev(a, b, c, spec->degree, spec->scale, M);
  return CKAN_OK;
}

int ckan_pack_coeffs_basis(const ckan_desc* desc, const ckan_basis_spec* spec, const void* coeffs,
                           void* packed, void* stream) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (valu_route(desc)) {  // C in fp32 and the family's recurrence block
    if ((rc = family_valid(spec, desc->degree))) return rc;
    if (!coeffs || !packed) return fail(CKAN_ERR_INVALID_ARG, "coeffs/packed is NULL");
    if (!aligned16(packed)) return fail(CKAN_ERR_INVALID_ARG, "packed buffer must be 16-byte aligned");
    ProfScope ps("pack", s);
    launch_to_f32(coeffs, desc->coeff_dtype == CKAN_DTYPE_BF16, static_cast<float*>(packed),
                  valu_coeffs(desc), s);
    launch_write_recur(valu_rec(desc, packed), spec->family, spec->alpha, spec->beta, desc->degree,
                       (float)spec->scale, s);
    return check_launch("pack_coeffs_basis");
  }
  BasisXform xf;
  if ((rc = family_xform(spec, desc->degree, &xf))) return rc;
  if (!coeffs || !packed) return fail(CKAN_ERR_INVALID_ARG, "coeffs/packed is NULL");
  if (!aligned16(packed)) return fail(CKAN_ERR_INVALID_ARG, "packed buffer must be 16-byte aligned");
  const Plan p = plan_of(desc);
  ProfScope ps("pack", s);
  launch_pack(coeffs, desc->coeff_dtype == CKAN_DTYPE_BF16, packed, p, s, &xf);
  return check_launch("pack_coeffs_basis");
}

int ckan_coeff_grad_from_chebyshev(const ckan_desc* desc, const ckan_basis_spec* spec,
                                   const float* dcheb, float* dcoeffs, int accumulate, void* stream) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (valu_route(desc)) {
    // the vector-ALU backward already differentiates in the family's basis:
    // the map is the identity (a copy, an accumulation, or nothing in place)
    if ((rc = family_valid(spec, desc->degree))) return rc;
    if (!dcheb || !dcoeffs) return fail(CKAN_ERR_INVALID_ARG, "dcheb/dcoeffs is NULL");
    if (dcheb == dcoeffs && accumulate)
      return fail(CKAN_ERR_INVALID_ARG, "in-place transform (dcheb == dcoeffs) cannot accumulate");
    if (dcheb == dcoeffs) return CKAN_OK;
    ProfScope ps("coeff_from_cheb", s);
    launch_to_f32(dcheb, false, dcoeffs, valu_coeffs(desc), s, accumulate != 0);
    return check_launch("coeff_grad_from_chebyshev");
  }
  BasisXform xf;
  if ((rc = family_xform(spec, desc->degree, &xf))) return rc;
  if (!dcheb || !dcoeffs) return fail(CKAN_ERR_INVALID_ARG, "dcheb/dcoeffs is NULL");
  if (dcheb == dcoeffs && accumulate)
    return fail(CKAN_ERR_INVALID_ARG, "in-place transform (dcheb == dcoeffs) cannot accumulate");
  const Plan p = plan_of(desc);
  ProfScope ps("coeff_from_cheb", s);
  launch_coeff_from_cheb(dcheb, dcoeffs, p, DcOut{accumulate ? kDcAccumulate : kDcStore}, xf, s);
  return check_launch("coeff_grad_from_chebyshev");
}

int ckan_backward_basis(const ckan_desc* desc, const ckan_basis_spec* spec, const float* t_cache,
                        const void* packed, const float* dy, float* dx, float* dcoeffs, void* ws,
                        size_t ws_bytes, void* stream) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  const DcOut om{kDcStore};
  if (valu_route(desc)) {
    // the vector-ALU backward differentiates in the family's basis already
    if ((rc = family_valid(spec, desc->degree))) return rc;
    return backward_impl(desc, t_cache, packed, dy, dx, dcoeffs, om, ws, ws_bytes, stream);
  }
  BasisXform xf;
  if ((rc = family_xform(spec, desc->degree, &xf))) return rc;
  bool used = false, mapped = false;
  if ((rc = backward_core(desc, t_cache, packed, dy, dx, dcoeffs, om, ws, ws_bytes, stream, nullptr,
                          &used, &xf, &mapped)))
    return rc;
  if (!dcoeffs || mapped || desc->batch == 0) return CKAN_OK;  // an empty batch's dC is zero
  const Plan p = plan_of(desc);
  ProfScope ps("coeff_from_cheb", reinterpret_cast<hipStream_t>(stream));
  launch_coeff_from_cheb(dcoeffs, dcoeffs, p, om, xf, reinterpret_cast<hipStream_t>(stream));
  return check_launch("backward_basis: coefficient map");
}

namespace {
// R = M L^order for a layer of degree `degree` (spec NULL: Chebyshev, M = I),
// as floats in r->m[n * kMaxD + k] (transposed: r->m[k * kMaxD + n]); *dout = D + order.
// affine_a != 0: L is the derivative under the affine input map t = a x + b.
int derivative_xform(const ckan_basis_spec* spec, int degree, int order, bool transposed,
                     BasisXform* r, int* dout, double* Rout = nullptr, double affine_a = 0.0) {
  if (degree < 0) return fail(CKAN_ERR_INVALID_ARG, "degree must be >= 0");
  if (order < 0) return fail(CKAN_ERR_INVALID_ARG, "derivative order must be >= 0");
  if (degree + order > kDerivMaxDegree)
    return fail(CKAN_ERR_UNSUPPORTED, "degree %d + derivative order %d exceeds %d", degree, order,
                kDerivMaxDegree);
  // the operator in kernel arguments (and every family basis) stops at
  // degree + order = kMaxD - 1; longer Chebyshev series go row by row
  if (degree + order >= kMaxD && (spec || r))
    return fail(CKAN_ERR_UNSUPPORTED, "%s: degree %d + derivative order %d exceeds %d",
                spec ? "family basis" : "operator", degree, order, kMaxD - 1);
  const int D = degree + 1, DO = D + order;
  std::vector<double> M((size_t)D * D, 0.0);
  if (spec) {
    double a[kMaxD], b[kMaxD], c[kMaxD];
    int rc = family_of(spec, degree, a, b, c);
    if (rc) return rc;
    family_to_chebyshev(a, b, c, degree, spec->scale, M.data());
  } else {
    for (int n = 0; n < D; ++n) M[(size_t)n * D + n] = 1.0;
  }
  std::vector<double> R((size_t)D * DO);
  const bool ok = affine_a != 0.0
                      ? affine_derivative_to_chebyshev(M.data(), degree, order, affine_a, R.data())
                      : derivative_to_chebyshev(M.data(), degree, order, R.data());
  if (!ok) return fail(CKAN_ERR_UNSUPPORTED, "derivative of order %d at degree %d", order, degree);
  if (Rout)
    for (size_t q = 0; q < (size_t)D * DO; ++q) Rout[q] = R[q];
  if (r) {
    for (int q = 0; q < kMaxD * kMaxD; ++q) r->m[q] = 0.0f;
    for (int n = 0; n < D; ++n)
      for (int k = 0; k < DO; ++k)
        r->m[transposed ? k * kMaxD + n : n * kMaxD + k] = (float)R[(size_t)n * DO + k];
  }
  if (dout) *dout = DO;
  return CKAN_OK;
}

// Chebyshev layers whose derivative series is longer than the operator in
// kernel arguments: the row-by-row kernels (launch_cheb_deriv_rows).
inline bool deriv_by_rows(const ckan_basis_spec* spec, int degree, int order) {
  return !spec && order >= 0 && degree + order >= kMaxD;
}

// Derivative calls: fp32 coefficients; the affine input map only where the
// operator fits in kernel arguments (the row-by-row kernels serve tanh).
int check_f32_layer(const ckan_desc* desc, const ckan_basis_spec* spec, int order) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (desc->input_map == CKAN_INPUT_AFFINE && deriv_by_rows(spec, desc->degree, order))
    return fail(CKAN_ERR_UNSUPPORTED, "derivatives under the affine input map: degree %d + order "
                "%d exceeds %d", desc->degree, order, kMaxD - 1);
  if (desc->coeff_dtype != CKAN_DTYPE_F32)
    return fail(CKAN_ERR_UNSUPPORTED, "derivatives take fp32 coefficients");
  return CKAN_OK;
}

// The chain factor of the input map in derivative_xform (0: tanh).
inline double map_slope(const ckan_desc* desc) {
  return desc->input_map == CKAN_INPUT_AFFINE ? (double)desc->in_scale : 0.0;
}
}  // namespace

int ckan_derivative_matrix(const ckan_basis_spec* spec, int32_t degree, int32_t order, double* R) {
  if (!R) return fail(CKAN_ERR_INVALID_ARG, "R is NULL");
  return derivative_xform(spec, degree, order, false, nullptr, nullptr, R);
}

int ckan_derivative_coeffs(const ckan_desc* desc, const ckan_basis_spec* spec, int32_t order,
                           const float* coeffs, float* out, void* stream) {
  int rc = check_f32_layer(desc, spec, order);
  if (rc) return rc;
  const int64_t rows = (int64_t)desc->in_dim * desc->out_dim;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (deriv_by_rows(spec, desc->degree, order)) {
    if ((rc = derivative_xform(nullptr, desc->degree, order, false, nullptr, nullptr))) return rc;
    if (!coeffs || !out) return fail(CKAN_ERR_INVALID_ARG, "coeffs/out is NULL");
    ProfScope ps("deriv_coeffs", s);
    launch_cheb_deriv_rows(coeffs, out, rows, desc->degree, order, false, 0, s);
    return check_launch("derivative_coeffs");
  }
  BasisXform r;
  int dout = 0;
  if ((rc = derivative_xform(spec, desc->degree, order, false, &r, &dout, nullptr,
                             map_slope(desc))))
    return rc;
  if (!coeffs || !out) return fail(CKAN_ERR_INVALID_ARG, "coeffs/out is NULL");
  ProfScope ps("deriv_coeffs", s);
  launch_coeff_xform(coeffs, out, rows, desc->degree + 1, dout, 0, r, s);
  return check_launch("derivative_coeffs");
}

int ckan_derivative_coeffs_backward(const ckan_desc* desc, const ckan_basis_spec* spec,
                                    int32_t order, const float* dout_grad, float* dcoeffs,
                                    void* stream) {
  int rc = check_f32_layer(desc, spec, order);
  if (rc) return rc;
  const int64_t rows = (int64_t)desc->in_dim * desc->out_dim;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (deriv_by_rows(spec, desc->degree, order)) {
    if ((rc = derivative_xform(nullptr, desc->degree, order, true, nullptr, nullptr))) return rc;
    if (!dout_grad || !dcoeffs) return fail(CKAN_ERR_INVALID_ARG, "dout_grad/dcoeffs is NULL");
    ProfScope ps("deriv_coeffs_bwd", s);
    launch_cheb_deriv_rows(dout_grad, dcoeffs, rows, desc->degree, order, true, 0, s);
    return check_launch("derivative_coeffs_backward");
  }
  BasisXform rt;
  int dout = 0;
  if ((rc = derivative_xform(spec, desc->degree, order, true, &rt, &dout, nullptr,
                             map_slope(desc))))
    return rc;
  if (!dout_grad || !dcoeffs) return fail(CKAN_ERR_INVALID_ARG, "dout_grad/dcoeffs is NULL");
  ProfScope ps("deriv_coeffs_bwd", s);
  launch_coeff_xform(dout_grad, dcoeffs, rows, dout, desc->degree + 1, 0, rt, s);
  return check_launch("derivative_coeffs_backward");
}

size_t ckan_jacobian_workspace_bytes(const ckan_desc* desc) {
  if (validate_desc(desc) != CKAN_OK) return 0;
  return (size_t)desc->in_dim * desc->out_dim * (desc->degree + 2) * sizeof(float);
}

int ckan_jacobian(const ckan_desc* desc, const ckan_basis_spec* spec, const float* x,
                  const float* coeffs, float* jac, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_f32_layer(desc, spec, 1);
  if (rc) return rc;
  const bool by_rows = deriv_by_rows(spec, desc->degree, 1);
  BasisXform r;
  int dout = 0;
  if ((rc = derivative_xform(spec, desc->degree, 1, false, by_rows ? nullptr : &r, &dout, nullptr,
                             map_slope(desc))))
    return rc;
  if (desc->batch == 0) return CKAN_OK;
  if (!x || !coeffs || !jac) return fail(CKAN_ERR_INVALID_ARG, "x/coeffs/jac is NULL");
  const size_t need = ckan_jacobian_workspace_bytes(desc);
  if (!ws || ws_bytes < need)
    return fail(CKAN_ERR_WORKSPACE, "jacobian workspace needs %zu bytes, got %zu", need, ws_bytes);
  const int64_t rows = (int64_t)desc->in_dim * desc->out_dim;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ProfScope ps("jacobian", s);
  float* c1t = reinterpret_cast<float*>(ws);
  if (by_rows)
    launch_cheb_deriv_rows(coeffs, c1t, rows, desc->degree, 1, false, desc->out_dim, s);
  else
    launch_coeff_xform(coeffs, c1t, rows, desc->degree + 1, dout, desc->out_dim, r, s);
  launch_jacobian(x, c1t, jac, desc->batch, desc->in_dim, desc->out_dim, dout, desc->input_map,
                  desc->in_scale, desc->in_shift, s);
  return check_launch("jacobian");
}

int ckan_family_basis(const ckan_basis_spec* spec, const float* t, int64_t n, float* out,
                      void* stream) {
  int rc = family_valid(spec, spec ? spec->degree : 0);
  if (rc) return rc;
  if (spec->degree < 0 || spec->degree > kValuMaxDegree)
    return fail(spec->degree < 0 ? CKAN_ERR_INVALID_ARG : CKAN_ERR_UNSUPPORTED,
                "basis degree %d outside 0..%d", spec->degree, kValuMaxDegree);
  if (n < 0) return fail(CKAN_ERR_INVALID_ARG, "n must be >= 0");
  if (n == 0) return CKAN_OK;
  if (!t || !out) return fail(CKAN_ERR_INVALID_ARG, "t/out is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ProfScope ps("basis", s);
  launch_basis_family(t, n, spec->degree, spec->family, spec->alpha, spec->beta, out, s);
  return check_launch("family_basis");
}

int ckan_family_basis_backward(const ckan_basis_spec* spec, const float* t, const float* g,
                               int64_t n, float* dt, void* stream) {
  int rc = family_valid(spec, spec ? spec->degree : 0);
  if (rc) return rc;
  if (spec->degree < 0 || spec->degree > kValuMaxDegree)
    return fail(spec->degree < 0 ? CKAN_ERR_INVALID_ARG : CKAN_ERR_UNSUPPORTED,
                "basis degree %d outside 0..%d", spec->degree, kValuMaxDegree);
  if (n < 0) return fail(CKAN_ERR_INVALID_ARG, "n must be >= 0");
  if (n == 0) return CKAN_OK;
  if (!t || !g || !dt) return fail(CKAN_ERR_INVALID_ARG, "t/g/dt is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ProfScope ps("basis_bwd", s);
  launch_basis_family_bwd(t, g, n, spec->degree, spec->family, spec->alpha, spec->beta, dt,
                          s);
  return check_launch("family_basis_backward");
}

int ckan_sgd_step(float* p, const float* g, int64_t n, float lr, float weight_decay,
                  void* stream) {
  if (n < 0) return fail(CKAN_ERR_INVALID_ARG, "n must be >= 0");
  if (n == 0) return CKAN_OK;
  if (!p || !g) return fail(CKAN_ERR_INVALID_ARG, "p/g is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ProfScope ps("sgd", s);
  launch_sgd(p, g, n, lr, weight_decay, s);
  return check_launch("sgd_step");
}

int ckan_adam_step(float* p, const float* g, float* m, float* v, int64_t n, int64_t step,
                   double lr, double beta1, double beta2, double eps, double weight_decay,
                   void* stream) {
  if (n < 0) return fail(CKAN_ERR_INVALID_ARG, "n must be >= 0");
  if (step < 1) return fail(CKAN_ERR_INVALID_ARG, "step must be >= 1 (got %lld)", (long long)step);
  if (!(beta1 >= 0.0 && beta1 < 1.0) || !(beta2 >= 0.0 && beta2 < 1.0))
    return fail(CKAN_ERR_INVALID_ARG, "betas must lie in [0, 1)");
  if (n == 0) return CKAN_OK;
  if (!p || !g || !m || !v) return fail(CKAN_ERR_INVALID_ARG, "p/g/m/v is NULL");
  const double bc1 = 1.0 - pow(beta1, (double)step);
  const double bc2 = 1.0 - pow(beta2, (double)step);
  const double step_size = lr / bc1;
  const double bc2_sqrt = sqrt(bc2);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ProfScope ps("adam", s);
  launch_adam(p, g, m, v, n, (float)(1.0 - beta1), (float)beta2, (float)(1.0 - beta2),
              (float)bc2_sqrt, (float)eps, (float)(-step_size), (float)weight_decay, s);
  return check_launch("adam_step");
}

int ckan_profile_enable(int on) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_on = on != 0;
  return CKAN_OK;
}

size_t ckan_profile_report(char* buf, size_t len) {
  std::vector<ProfRec> recs;
  {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    recs.swap(g_prof);
  }
  std::vector<std::string> names;
  std::vector<double> tot;
  std::vector<long> cnt;
  for (auto& r : recs) {
    float ms = 0.0f;
    if (hipEventSynchronize(r.b) == hipSuccess) hipEventElapsedTime(&ms, r.a, r.b);
    hipEventDestroy(r.a);
    hipEventDestroy(r.b);
    size_t k = 0;
    for (; k < names.size(); ++k)
      if (names[k] == r.name) break;
    if (k == names.size()) {
      names.push_back(r.name);
      tot.push_back(0.0);
      cnt.push_back(0);
    }
    tot[k] += ms;
    cnt[k] += 1;
  }
  std::string out;
  char line[160];
  for (size_t k = 0; k < names.size(); ++k) {
    snprintf(line, sizeof(line), "%s %ld %.6f\n", names[k].c_str(), cnt[k], tot[k]);
    out += line;
  }
  if (buf && len) {
    const size_t n = out.size() < len - 1 ? out.size() : len - 1;
    memcpy(buf, out.data(), n);
    buf[n] = 0;
  }
  return out.size() + 1;
}

}  // extern "C"

bool ckan::layer_reads_tcache(const ckan_desc* desc) {
  if (validate_desc(desc) != CKAN_OK || valu_route(desc)) return false;
  const Plan p = plan_of(desc);
  return p.I == p.I_sg && fwd_reads_tcache(choose_fwd(p));
}

bool ckan::layer_out_tanh_ok(const ckan_desc* desc) {
  if (validate_desc(desc) != CKAN_OK || valu_route(desc)) return false;
  return fwd_out_tanh_ok(plan_of(desc));
}

bool ckan::pack_pair_fits(const ckan_desc* a, const ckan_desc* b) {
  if (validate_desc(a) != CKAN_OK || validate_desc(b) != CKAN_OK || valu_route(a) || valu_route(b))
    return false;
  if (a->coeff_dtype != CKAN_DTYPE_F32 || b->coeff_dtype != CKAN_DTYPE_F32) return false;
  if (a->batch != b->batch || a->out_dim != b->in_dim || a->batch < 1) return false;
  return pack_pair_ok(plan_of(a), plan_of(b)) && layer_out_tanh_ok(a) && layer_reads_tcache(b);
}

int ckan::pack2_forward_ex(const ckan_desc* da, const void* Ca, void* pka, const float* xa,
                           float* ta, bool ta_ready, const ckan_desc* db, const void* Cb,
                           void* pkb, float* tb, float* outb, bool outb_tanh, void* ws,
                           size_t ws_bytes, void* stream) {
  if (!pack_pair_fits(da, db) || (ta_ready && !layer_reads_tcache(da)) ||
      (outb_tanh && !layer_out_tanh_ok(db)))
    return fail(CKAN_ERR_INVALID_ARG, "pack2_forward_ex: the layer pair does not allow one pack launch");
  if (!Ca || !pka || !Cb || !pkb || !ta || !tb || !outb || (!xa && !ta_ready))
    return fail(CKAN_ERR_INVALID_ARG, "pack2_forward_ex: NULL pointer");
  if (!aligned16(pka) || !aligned16(pkb) || !aligned16(ta) || !aligned16(tb))
    return fail(CKAN_ERR_INVALID_ARG, "pack2_forward_ex: packed buffers and caches must be 16-byte aligned");
  const Plan pa = plan_of(da), pb = plan_of(db);
  const FwdChoice ca = choose_fwd(pa), cb = choose_fwd(pb);
  const size_t need = fwd_ws_bytes(pa, ca) > fwd_ws_bytes(pb, cb) ? fwd_ws_bytes(pa, ca) : fwd_ws_bytes(pb, cb);
  if (ws_bytes < need)
    return fail(CKAN_ERR_WORKSPACE, "forward workspace too small: %zu < %zu bytes", ws_bytes, need);
  if (need && !ws) return fail(CKAN_ERR_INVALID_ARG, "workspace is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool sum_a = fwd_sums_bias(pa, ca), sum_b = fwd_sums_bias(pb, cb);
  const bool fuse_tanh = !ta_ready && fwd_reads_tcache(ca) && pack_tanh_fusable(pa, xa);
  {
    ProfScope ps("pack2", s);
    launch_pack_pair(reinterpret_cast<const float*>(Ca), pka, pa, !sum_a, fuse_tanh ? xa : nullptr,
                     fuse_tanh ? ta : nullptr, reinterpret_cast<const float*>(Cb), pkb, pb, !sum_b, s);
  }
  int rc;
  if ((rc = check_launch("pack2_forward: pack"))) return rc;
  if ((rc = forward_packed(pa, ca, pka, xa, tb, ta, ws, s, ta_ready || fuse_tanh, sum_a, true)))
    return rc;
  return forward_packed(pb, cb, pkb, nullptr, outb, tb, ws, s, true, sum_b, outb_tanh);
}

bool ckan::pack2_tail_ce_fits(const ckan_desc* a, const ckan_desc* b) {
  if (!pack_pair_fits(a, b) || a->compute != CKAN_COMPUTE_FP32 || b->compute != CKAN_COMPUTE_FP32 ||
      b->input_map != CKAN_INPUT_TANH)
    return false;
  const Plan pa = plan_of(a);
  return fwd_tail_ce_ok(pa, choose_fwd(pa), b->out_dim, b->degree + 1);
}

int ckan::pack2_forward_tail_ce(const ckan_desc* da, const void* Ca, void* pka, const float* xa,
                                float* ta, bool ta_ready, const ckan_desc* db, const void* Cb,
                                void* pkb, float* tb, float* yb, const int64_t* labels, float* dyb,
                                float* loss_part, void* ws, size_t ws_bytes, void* stream) {
  if (!pack2_tail_ce_fits(da, db) || (ta_ready && !layer_reads_tcache(da)))
    return fail(CKAN_ERR_INVALID_ARG, "pack2_forward_tail_ce: the layer pair does not allow the fused tail");
  if (!Ca || !pka || !Cb || !pkb || !ta || !tb || !yb || !labels || !dyb || !loss_part ||
      (!xa && !ta_ready))
    return fail(CKAN_ERR_INVALID_ARG, "pack2_forward_tail_ce: NULL pointer");
  if (!aligned16(pka) || !aligned16(pkb) || !aligned16(ta) || !aligned16(tb))
    return fail(CKAN_ERR_INVALID_ARG, "pack2_forward_tail_ce: packed buffers and caches must be 16-byte aligned");
  const Plan pa = plan_of(da), pb = plan_of(db);
  const FwdChoice ca = choose_fwd(pa);
  const size_t need = fwd_ws_bytes(pa, ca);
  if (ws_bytes < need)
    return fail(CKAN_ERR_WORKSPACE, "forward workspace too small: %zu < %zu bytes", ws_bytes, need);
  if (need && !ws) return fail(CKAN_ERR_INVALID_ARG, "workspace is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // b's forward runs in the tail from its fp32 coefficients: b's packed
  // bias slot is not filled (the step's backward reads only b's dX operand,
  // and a later forward packs again)
  const bool sum_a = fwd_sums_bias(pa, ca);
  const bool fuse_tanh = !ta_ready && fwd_reads_tcache(ca) && pack_tanh_fusable(pa, xa);
  {
    ProfScope ps("pack2", s);
    launch_pack_pair(reinterpret_cast<const float*>(Ca), pka, pa, !sum_a, fuse_tanh ? xa : nullptr,
                     fuse_tanh ? ta : nullptr, reinterpret_cast<const float*>(Cb), pkb, pb, false, s);
  }
  int rc;
  if ((rc = check_launch("pack2_forward_tail_ce: pack"))) return rc;
  if ((rc = forward_packed(pa, ca, pka, xa, tb, ta, ws, s, ta_ready || fuse_tanh, sum_a, true, false)))
    return rc;
  {
    ProfScope ps("fwd_tail", s);
    launch_fwd_tail_ce(pka, ws, pa, ca, sum_a, tb, reinterpret_cast<const float*>(Cb), db->out_dim,
                       db->degree + 1, yb, labels, dyb, loss_part, s);
  }
  return check_launch("pack2_forward_tail_ce: tail");
}

bool ckan::self_pack_pair_fits(const ckan_desc* a, const ckan_desc* b) {
  if (!pack2_tail_ce_fits(a, b)) return false;
  const Plan pa = plan_of(a), pb = plan_of(b);
  const FwdChoice ca = choose_fwd(pa);
  // a's bias as per-input-block partials, summed by the tail
  return pa.P == pb.P && pa.esz == pb.esz && dc_pack_ok(pa) && dc_pack_ok(pb) && dx_small_ok(pb) &&
         (pa.NIB == 1 || fwd_sums_bias(pa, ca));
}

int ckan::self_pack_layer(const ckan_desc* desc, const void* C, void* packed, void* stream) {
  if (validate_desc(desc) != CKAN_OK || valu_route(desc))
    return fail(CKAN_ERR_INVALID_ARG, "self_pack_layer: not a packed-kernel layer");
  if (!C || !packed || !aligned16(packed))
    return fail(CKAN_ERR_INVALID_ARG, "self_pack_layer: NULL or misaligned buffer");
  const Plan p = plan_of(desc);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  {
    ProfScope ps("pack", s);
    launch_pack(C, false, packed, p, s, nullptr, !fwd_sums_bias(p, choose_fwd(p)));
  }
  return check_launch("self_pack_layer");
}

int ckan::forward_tail_ce_packed(const ckan_desc* da, const void* pka, const float* xa, float* ta,
                                 const ckan_desc* db, const void* Cb, float* tb, float* yb,
                                 const int64_t* labels, float* dyb, float* loss_part, float* dya,
                                 void* ws, size_t ws_bytes, void* stream) {
  if (!self_pack_pair_fits(da, db))
    return fail(CKAN_ERR_INVALID_ARG, "forward_tail_ce_packed: the layer pair does not allow it");
  if (!pka || !xa || !ta || !Cb || !tb || !yb || !labels || !dyb || !loss_part || !dya)
    return fail(CKAN_ERR_INVALID_ARG, "forward_tail_ce_packed: NULL pointer");
  if (!aligned16(pka) || !aligned16(ta) || !aligned16(tb))
    return fail(CKAN_ERR_INVALID_ARG, "forward_tail_ce_packed: packed buffer and caches must be 16-byte aligned");
  const Plan pa = plan_of(da);
  const FwdChoice ca = choose_fwd(pa);
  const size_t need = fwd_ws_bytes(pa, ca);
  if (ws_bytes < need)
    return fail(CKAN_ERR_WORKSPACE, "forward workspace too small: %zu < %zu bytes", ws_bytes, need);
  if (need && !ws) return fail(CKAN_ERR_INVALID_ARG, "workspace is NULL");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool sum_a = fwd_sums_bias(pa, ca);
  int rc;
  if (fwd_maps_x_ok(pa, ca, xa)) {  // the GEMM maps x and writes a's tanh cache
    ProfScope ps("fwd_gemm", s);
    launch_fwd_gemm(xa, ta, pka, tb, ws, pa, ca, s, sum_a, true, false, true);
  } else if ((rc = forward_packed(pa, ca, pka, xa, tb, ta, ws, s, false, sum_a, true, false))) {
    return rc;
  }
  if ((rc = check_launch("forward_tail_ce_packed: forward"))) return rc;
  {
    ProfScope ps("fwd_tail", s);
    launch_fwd_tail_ce(pka, ws, pa, ca, sum_a, tb, reinterpret_cast<const float*>(Cb), db->out_dim,
                       db->degree + 1, yb, labels, dyb, loss_part, s, dya);
  }
  return check_launch("forward_tail_ce_packed: tail");
}

int ckan::backward_self_packed(const ckan_desc* da, const float* ta, const float* dya, float* Ca,
                               const DcOut& oma, void* pka, const ckan_desc* db, const float* tb,
                               const float* dyb, float* Cb, const DcOut& omb, void* pkb,
                               const LossMean& lm, void* stream) {
  if (!self_pack_pair_fits(da, db))
    return fail(CKAN_ERR_INVALID_ARG, "backward_self_packed: the layer pair does not allow it");
  if (oma.mode < kDcSgd || omb.mode < kDcSgd)
    return fail(CKAN_ERR_INVALID_ARG, "backward_self_packed: needs an optimizer step");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  {
    ProfScope ps("dc_pack", s);
    const DcPackArgs a{dya, ta, Ca, oma, plan_of(da), pka, true, false};
    const DcPackArgs b{dyb, tb, Cb, omb, plan_of(db), pkb, false, true};
    launch_dc_pack(a, &b, s, lm);
  }
  return check_launch("backward_self_packed");
}

int ckan::pack_forward_ex(const ckan_desc* desc, const void* coeffs, void* packed, const float* x,
                          float* out, float* t_cache, void* ws, size_t ws_bytes, void* stream,
                          bool t_ready, bool out_tanh, const ckan_basis_spec* spec) {
  if ((t_ready && !layer_reads_tcache(desc)) || (out_tanh && !layer_out_tanh_ok(desc)))
    return fail(CKAN_ERR_INVALID_ARG, "pack_forward_ex: the layer's forward path does not allow "
                "a precomputed tanh cache / a tanh output");
  return pack_forward_impl(desc, spec, coeffs, packed, x, out, t_cache, ws, ws_bytes, stream,
                           t_ready, out_tanh);
}

bool ckan::layer_on_valu(const ckan_desc* desc) { return valu_route(desc); }

int ckan::basis_check(const ckan_basis_spec* spec, int degree, BasisXform* xf) {
  if (degree > kMfmaMaxDegree) return family_valid(spec, degree);
  BasisXform tmp;
  return family_xform(spec, degree, xf ? xf : &tmp);
}
