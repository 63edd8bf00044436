// Symmetric-contraction launchers and C ABI entry points.
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/ictc_mi355x.h"
#include "sc_launch.h"

namespace ictc {
// Shared with capi.hip (error reporting).
int set_error(int code, const char* msg);
}

namespace {

using ictc::sc::Args;
constexpr int kBlock = 256;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return ictc::set_error(code, buf);
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ICTC_OK;
  return fail(ICTC_ERR_RUNTIME, "%s: %s", what, hipGetErrorString(e));
}

int64_t partial_bytes(int64_t nodes, int species, int nw, int channels) {
  return ictc::sc::partial_bytes(nodes, species, nw, channels);
}

// Host-side table of path counts and weight slots per configuration.
struct Shape {
  int P[4][3];
  int nw, nx, no, terms;
};

template <class T>
Shape shape_of() {
  Shape s{};
  for (int L = 0; L < 4; ++L)
    for (int n = 0; n < 3; ++n) s.P[L][n] = T::P[L][n];
  s.nw = T::NW;
  s.nx = T::NX;
  s.no = T::NO;
  s.terms = T::TERMS;
  return s;
}

template <class F>
int dispatch(int li, int lt, int corr, F&& f) {
#define ICTC_SC_CASE(A, B, C) \
  if (li == A && lt == B && corr == C) return f.template run<ictc::Sc<A, B, C>>();
  ICTC_FOR_EACH_SC(ICTC_SC_CASE)
#undef ICTC_SC_CASE
  return fail(ICTC_ERR_UNSUPPORTED, "symmetric contraction (lmax=%d, target_lmax=%d, correlation=%d) not compiled",
              li, lt, corr);
}

struct GetShape {
  Shape* out;
  template <class T>
  int run() {
    *out = shape_of<T>();
    return ICTC_OK;
  }
};

int check_common(int li, int lt, int corr, int C, int S, int64_t N, Shape* sh) {
  if (C < 1 || C > 4096) return fail(ICTC_ERR_ARGUMENT, "channels=%d out of range", C);
  if (S < 1) return fail(ICTC_ERR_ARGUMENT, "num_species must be positive");
  if (N < 0) return fail(ICTC_ERR_ARGUMENT, "negative node count");
  return dispatch(li, lt, corr, GetShape{sh});
}

Args make_args(const float* x, const int64_t* species, const float* const* w, int64_t N, int S, int C,
               const Shape& sh) {
  Args a;
  a.x = x;
  a.species = species;
  for (int L = 0; L < 4; ++L)
    for (int n = 0; n < 3; ++n) a.w.w[L][n] = (sh.P[L][n] > 0 && w) ? w[L * 3 + n] : nullptr;
  a.nodes = N;
  a.num_species = S;
  a.channels = C;
  return a;
}

int check_weights(const float* const* w, const Shape& sh) {
  if (!w) return fail(ICTC_ERR_ARGUMENT, "null weight table");
  for (int L = 0; L < 4; ++L)
    for (int n = 0; n < 3; ++n)
      if (sh.P[L][n] > 0 && !w[L * 3 + n]) return fail(ICTC_ERR_ARGUMENT, "null weight for L=%d nu=%d", L, n + 1);
  return ICTC_OK;
}

template <int MODE>
struct Fwd {
  Args a;
  const float* h;
  float* out;
  hipStream_t st;
  template <class T>
  int run() {
    return hip_status(ictc::sc::Launch<T>::fwd(a, h, out, MODE, st), "sc fwd launch");
  }
};

template <int MODE>
struct Dx {
  Args a;
  const float *go, *h;
  float* dx;
  hipStream_t st;
  template <class T>
  int run() {
    return hip_status(ictc::sc::Launch<T>::dx(a, go, h, dx, MODE, st), "sc dx launch");
  }
};

template <int MODE>
struct Dw {
  Args a;
  const float *go, *h;
  const int32_t *ptr, *order;
  float* const* dw;
  float* partial;
  hipStream_t st;
  template <class T>
  int run() {
    return hip_status(ictc::sc::Launch<T>::dw(a, go, h, ptr, order, dw, partial, MODE, st), "sc dw launch");
  }
};

}  // namespace

extern "C" {

int ictc_sc_shape(int lmax, int target_lmax, int correlation, int* paths, int* num_weights) {
  Shape sh;
  if (int rc = dispatch(lmax, target_lmax, correlation, GetShape{&sh})) return rc;
  if (paths)
    for (int L = 0; L < 4; ++L)
      for (int n = 0; n < 3; ++n) paths[L * 3 + n] = sh.P[L][n];
  if (num_weights) *num_weights = sh.nw;
  return ICTC_OK;
}

int ictc_sc_terms(int lmax, int target_lmax, int correlation) {
  Shape sh;
  if (int rc = dispatch(lmax, target_lmax, correlation, GetShape{&sh})) return rc;
  return sh.terms;
}

int64_t ictc_sc_workspace_bytes(int lmax, int target_lmax, int correlation, int channels, int64_t nodes,
                                int num_species) {
  Shape sh;
  if (dispatch(lmax, target_lmax, correlation, GetShape{&sh})) return -1;
  if (nodes < 0 || num_species < 1 || channels < 1) return -1;
  return partial_bytes(nodes, num_species, sh.nw, channels) + (int64_t)(num_species + 1) * (int64_t)sizeof(int32_t);
}

int ictc_sc_fwd(int li, int lt, int corr, int C, const float* x, const int64_t* species, int S,
                const float* const* weights, int64_t N, float* out, void* stream) {
  Shape sh;
  if (int rc = check_common(li, lt, corr, C, S, N, &sh)) return rc;
  if (N == 0) return ICTC_OK;
  if (!x || !species || !out) return fail(ICTC_ERR_ARGUMENT, "ictc_sc_fwd: null operand");
  if (int rc = check_weights(weights, sh)) return rc;
  return dispatch(li, lt, corr, Fwd<0>{make_args(x, species, weights, N, S, C, sh), nullptr, out, (hipStream_t)stream});
}

int ictc_sc_jvp(int li, int lt, int corr, int C, const float* x, const int64_t* species, int S,
                const float* const* weights, int64_t N, const float* tangent, float* out, void* stream) {
  Shape sh;
  if (int rc = check_common(li, lt, corr, C, S, N, &sh)) return rc;
  if (N == 0) return ICTC_OK;
  if (!x || !species || !out || !tangent) return fail(ICTC_ERR_ARGUMENT, "ictc_sc_jvp: null operand");
  if (int rc = check_weights(weights, sh)) return rc;
  return dispatch(li, lt, corr, Fwd<1>{make_args(x, species, weights, N, S, C, sh), tangent, out, (hipStream_t)stream});
}

int ictc_sc_bwd_x(int li, int lt, int corr, int C, const float* x, const int64_t* species, int S,
                  const float* const* weights, int64_t N, const float* grad, float* dx, void* stream) {
  Shape sh;
  if (int rc = check_common(li, lt, corr, C, S, N, &sh)) return rc;
  if (N == 0) return ICTC_OK;
  if (!x || !species || !grad || !dx) return fail(ICTC_ERR_ARGUMENT, "ictc_sc_bwd_x: null operand");
  if (int rc = check_weights(weights, sh)) return rc;
  return dispatch(li, lt, corr,
                  Dx<0>{make_args(x, species, weights, N, S, C, sh), grad, nullptr, dx, (hipStream_t)stream});
}

int ictc_sc_hvp(int li, int lt, int corr, int C, const float* x, const int64_t* species, int S,
                const float* const* weights, int64_t N, const float* grad, const float* tangent, float* dx,
                void* stream) {
  Shape sh;
  if (int rc = check_common(li, lt, corr, C, S, N, &sh)) return rc;
  if (N == 0) return ICTC_OK;
  if (!x || !species || !grad || !dx || !tangent) return fail(ICTC_ERR_ARGUMENT, "ictc_sc_hvp: null operand");
  if (int rc = check_weights(weights, sh)) return rc;
  return dispatch(li, lt, corr,
                  Dx<1>{make_args(x, species, weights, N, S, C, sh), grad, tangent, dx, (hipStream_t)stream});
}

static int sc_dw_common(int mode, int li, int lt, int corr, int C, const float* x, int S, int64_t N,
                        const float* grad, const float* tangent, const int32_t* ptr, const int32_t* order,
                        float* const* dweights, void* workspace, int64_t workspace_bytes, void* stream) {
  Shape sh;
  if (int rc = check_common(li, lt, corr, C, S, N, &sh)) return rc;
  if (!dweights) return fail(ICTC_ERR_ARGUMENT, "null weight-gradient table");
  for (int L = 0; L < 4; ++L)
    for (int n = 0; n < 3; ++n)
      if (sh.P[L][n] > 0 && !dweights[L * 3 + n])
        return fail(ICTC_ERR_ARGUMENT, "null weight gradient for L=%d nu=%d", L, n + 1);
  if (!x || !grad || !ptr || !order || !workspace || (mode == 1 && !tangent))
    return fail(ICTC_ERR_ARGUMENT, "ictc_sc_bwd_w: null operand");
  const int64_t need = ictc_sc_workspace_bytes(li, lt, corr, C, N, S);
  if (workspace_bytes < need)
    return fail(ICTC_ERR_ARGUMENT, "sc workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)need);
  const float* no_w[12] = {};
  Args a = make_args(x, nullptr, no_w, N > 0 ? N : 1, S, C, sh);
  a.nodes = N > 0 ? N : 1;
  if (N == 0) a.nodes = 0;
  if (mode == 0)
    return dispatch(li, lt, corr,
                    Dw<0>{a, grad, nullptr, ptr, order, dweights, (float*)workspace, (hipStream_t)stream});
  return dispatch(li, lt, corr, Dw<1>{a, grad, tangent, ptr, order, dweights, (float*)workspace, (hipStream_t)stream});
}

int ictc_sc_bwd_w(int li, int lt, int corr, int C, const float* x, int S, int64_t N, const float* grad,
                  const int32_t* species_ptr, const int32_t* species_order, float* const* dweights, void* workspace,
                  int64_t workspace_bytes, void* stream) {
  return sc_dw_common(0, li, lt, corr, C, x, S, N, grad, nullptr, species_ptr, species_order, dweights, workspace,
                      workspace_bytes, stream);
}

int ictc_sc_bwd_w_jvp(int li, int lt, int corr, int C, const float* x, int S, int64_t N, const float* grad,
                      const float* tangent, const int32_t* species_ptr, const int32_t* species_order,
                      float* const* dweights, void* workspace, int64_t workspace_bytes, void* stream) {
  return sc_dw_common(1, li, lt, corr, C, x, S, N, grad, tangent, species_ptr, species_order, dweights, workspace,
                      workspace_bytes, stream);
}

}  // extern "C"
