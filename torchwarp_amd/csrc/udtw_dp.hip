// uDTW / soft-DTW host entry points for gfx950: argument checks, the
// hyper-parameters of the sweep and the C ABI. The sweep kernels and their
// launchers are in udtw_sweep.hpp.

#include "udtw_sweep.hpp"
#include "../../include/torchwarp_hip.h"

namespace tw {

template <typename T, int SRC>
static int launch_pen(bool pen, bool backward, const UdtwArgs<T>& a, int B, hipStream_t s,
                      const char* what) {
  return backward ? launch_sweep<T, SRC, true>(pen, a, B, s, what)
                  : launch_sweep<T, SRC, false>(pen, a, B, s, what);
}

template <typename T>
static void set_hyper(UdtwArgs<T>& a, double gamma, double beta, double eps, double band) {
  a.k = (T)(1.4426950408889634 / gamma);
  a.inv_k = (T)(gamma * 0.6931471805599453);
  a.inv_gamma = (T)(1.0 / gamma);
  a.beta = (T)beta;
  a.beta_ln2 = (T)(beta * 0.6931471805599453);
  a.eps = (T)eps;
  a.band = (T)band;
  a.hv1 = (T)0;
  a.hv0 = (T)0.5;
}

template <typename T>
static void set_sigma(UdtwArgs<T>& a, int sigma) {
  a.sigma = sigma != 0;
  a.hv1 = (T)(a.sigma ? 0.5 : 0.0);
  a.hv0 = (T)(a.sigma ? 0.0 : 0.5);
}

static int check_dims(const char* what, int B, int N, int M, double gamma) {
  if (B < 0 || N <= 0 || M <= 0) return fail(TW_EINVAL, "%s: bad sizes B=%d N=%d M=%d", what, B, N, M);
  if (N > M) return fail(TW_EINVAL, "%s: expected N <= M (got %d > %d)", what, N, M);
  if (!(gamma > 0)) return fail(TW_EINVAL, "%s: gamma must be > 0", what);
  return TW_OK;
}

template <typename T>
static int cost_fwd(const T* C, const T* Q, int B, int N, int M, double gamma, double band, T* R,
                    T* P, T* out_r, T* out_p, hipStream_t s, const char* what) {
  if (int e = check_dims(what, B, N, M, gamma)) return e;
  if (B == 0) return TW_OK;
  if (!C || !R || !out_r || !out_p) return fail(TW_EINVAL, "%s: null pointer", what);
  if (Q && !P) return fail(TW_EINVAL, "%s: a penalty needs the P buffer", what);
  UdtwArgs<T> a = {};
  a.C = C;
  a.Q = Q;
  a.R = R;
  a.P = P;
  a.out_r = out_r;
  a.out_p = out_p;
  a.N = N;
  a.M = M;
  set_hyper(a, gamma, 0.0, 1.0, band);
  return launch_pen<T, SRC_COST>(Q != nullptr, false, a, B, s, what);
}

template <typename T>
static int cost_bwd(const T* C, const T* Q, const T* R, const T* P, const T* gr, const T* gp,
                    int B, int N, int M, double gamma, double band, int gstride, T* dC, T* dQ,
                    hipStream_t s, const char* what) {
  if (int e = check_dims(what, B, N, M, gamma)) return e;
  if (B == 0) return TW_OK;
  if (!C || !R || !gr || !dC) return fail(TW_EINVAL, "%s: null pointer", what);
  const bool pen = Q != nullptr;
  if (pen && (!P || !gp)) return fail(TW_EINVAL, "%s: a penalty needs P and grad_pen", what);
  UdtwArgs<T> a = {};
  a.C = C;
  a.Q = Q;
  a.R = const_cast<T*>(R);  // read-only in the backward
  a.P = const_cast<T*>(P);
  a.gr = gr;
  a.gp = gp;
  a.dC = dC;
  a.dQ = pen ? dQ : nullptr;
  a.N = N;
  a.M = M;
  if (gstride != 0 && gstride != 1) return fail(TW_EINVAL, "%s: grad_stride must be 0 or 1", what);
  a.gstride = gstride;
  set_hyper(a, gamma, 0.0, 1.0, band);
  return launch_pen<T, SRC_COST>(pen, true, a, B, s, what);
}

template <typename T>
int udtw_cost_fwd_any(const T* C, const T* Q, int B, int N, int M, double gamma, double band,
                      T* R, T* P, T* out_r, T* out_p, hipStream_t s, const char* what) {
  return cost_fwd<T>(C, Q, B, N, M, gamma, band, R, P, out_r, out_p, s, what);
}
template <typename T>
int udtw_cost_bwd_any(const T* C, const T* Q, const T* R, const T* P, const T* gr, const T* gp,
                      int B, int N, int M, double gamma, T* dC, T* dQ, hipStream_t s,
                      const char* what) {
  return cost_bwd<T>(C, Q, R, P, gr, gp, B, N, M, gamma, 0.0, 1, dC, dQ, s, what);
}
template int udtw_cost_fwd_any<float>(const float*, const float*, int, int, int, double, double,
                                      float*, float*, float*, float*, hipStream_t, const char*);
template int udtw_cost_fwd_any<double>(const double*, const double*, int, int, int, double,
                                       double, double*, double*, double*, double*, hipStream_t,
                                       const char*);
template int udtw_cost_bwd_any<float>(const float*, const float*, const float*, const float*,
                                      const float*, const float*, int, int, int, double, float*,
                                      float*, hipStream_t, const char*);
template int udtw_cost_bwd_any<double>(const double*, const double*, const double*,
                                       const double*, const double*, const double*, int, int,
                                       int, double, double*, double*, hipStream_t, const char*);

}  // namespace tw

// ------------------------------------------------------------------ C ABI

using namespace tw;

extern "C" {

int tw_udtw_cost_fwd_f32(const float* cost, const float* pen, int B, int N, int M, float gamma,
                         float bandwidth, float* R, float* P, float* out_dist, float* out_pen,
                         hipStream_t stream) {
  return cost_fwd<float>(cost, pen, B, N, M, gamma, bandwidth, R, P, out_dist, out_pen, stream,
                         "tw_udtw_cost_fwd_f32");
}

int tw_udtw_cost_fwd_f64(const double* cost, const double* pen, int B, int N, int M,
                         double gamma, double bandwidth, double* R, double* P, double* out_dist,
                         double* out_pen, hipStream_t stream) {
  return cost_fwd<double>(cost, pen, B, N, M, gamma, bandwidth, R, P, out_dist, out_pen, stream,
                          "tw_udtw_cost_fwd_f64");
}

int tw_udtw_cost_bwd_f32(const float* cost, const float* pen, const float* R, const float* P,
                         const float* grad_dist, const float* grad_pen, int B, int N, int M,
                         float gamma, float bandwidth, int grad_stride, float* d_cost,
                         float* d_pen, hipStream_t stream) {
  return cost_bwd<float>(cost, pen, R, P, grad_dist, grad_pen, B, N, M, gamma, bandwidth,
                         grad_stride, d_cost, d_pen, stream, "tw_udtw_cost_bwd_f32");
}

int tw_udtw_cost_bwd_f64(const double* cost, const double* pen, const double* R,
                         const double* P, const double* grad_dist, const double* grad_pen, int B,
                         int N, int M, double gamma, double bandwidth, int grad_stride,
                         double* d_cost, double* d_pen, hipStream_t stream) {
  return cost_bwd<double>(cost, pen, R, P, grad_dist, grad_pen, B, N, M, gamma, bandwidth,
                          grad_stride, d_cost, d_pen, stream, "tw_udtw_cost_bwd_f64");
}

}  // extern "C"

// Features path: defined with the pairwise-distance kernels it uses for D > 1,
// which keep the squared distances (and their adjoint) in the sweeps'
// diagonal-major layout.
namespace tw {

template <typename T>
int sqdist_raw(const T* X, const T* Y, int P, int R, int C, int D, T* out, hipStream_t s,
               const char* what);
template <typename T>
int sqdist_raw_bwd(const T* X, const T* Y, const T* dS, int P, int R, int C, int D, T* dX, T* dY,
                   hipStream_t s, const char* what);

template <typename T>
static int feat_fwd(const T* X, const T* Y, const T* vx, const T* vy, int B, int N, int M, int D,
                    double gamma, double beta, double eps, double band, int sigma, T* R, T* P,
                    T* out_r, T* out_p, T* ws, size_t ws_bytes, hipStream_t s,
                    const char* what) {
  if (int e = check_dims(what, B, N, M, gamma)) return e;
  if (D <= 0) return fail(TW_EINVAL, "%s: D must be > 0", what);
  if (B == 0) return TW_OK;
  if (!X || !Y || !vx || !vy || !R || !out_r || !out_p)
    return fail(TW_EINVAL, "%s: null pointer", what);
  const bool pen = beta != 0.0;
  if (pen && !P) return fail(TW_EINVAL, "%s: beta != 0 needs the P buffer", what);
  UdtwArgs<T> a = {};
  a.VX = vx;
  a.VY = vy;
  a.R = R;
  a.P = P;
  a.out_r = out_r;
  a.out_p = out_p;
  a.N = N;
  a.M = M;
  set_hyper(a, gamma, beta, eps, band);
  set_sigma(a, sigma);
  if (D == 1) {
    a.X = X;
    a.Y = Y;
    return launch_pen<T, SRC_FEAT1>(pen, false, a, B, s, what);
  }
  const size_t need = (size_t)B * N * M * sizeof(T);
  if (!ws || ws_bytes < need)
    return fail(TW_ESIZE, "%s: workspace of %zu bytes needed", what, need);
  if (int e = sqdist_raw<T>(X, Y, B, N, M, D, ws, s, what)) return e;
  a.C = ws;
  return launch_pen<T, SRC_SQ>(pen, false, a, B, s, what);
}

template <typename T>
static int feat_bwd(const T* X, const T* Y, const T* vx, const T* vy, const T* R, const T* P,
                    const T* gr, const T* gp, int B, int N, int M, int D, double gamma,
                    double beta, double eps, double band, int sigma, int gstride, T* dX, T* dY,
                    T* dvx, T* dvy, const T* ws_fwd, T* ws, size_t ws_bytes, hipStream_t s,
                    const char* what) {
  if (int e = check_dims(what, B, N, M, gamma)) return e;
  if (D <= 0) return fail(TW_EINVAL, "%s: D must be > 0", what);
  if (B == 0) return TW_OK;
  if (!X || !Y || !vx || !vy || !R || !gr || !dX || !dY)
    return fail(TW_EINVAL, "%s: null pointer", what);
  if ((dvx == nullptr) != (dvy == nullptr))
    return fail(TW_EINVAL, "%s: pass both or neither variance gradient", what);
  const bool pen = beta != 0.0;
  if (pen && (!P || !gp)) return fail(TW_EINVAL, "%s: beta != 0 needs P and grad_pen", what);
  UdtwArgs<T> a = {};
  a.VX = vx;
  a.VY = vy;
  a.R = const_cast<T*>(R);  // read-only in the backward
  a.P = const_cast<T*>(P);
  a.gr = gr;
  a.gp = gp;
  a.dVX = dvx;
  a.dVY = dvy;
  a.N = N;
  a.M = M;
  if (gstride != 0 && gstride != 1) return fail(TW_EINVAL, "%s: grad_stride must be 0 or 1", what);
  a.gstride = gstride;
  set_hyper(a, gamma, beta, eps, band);
  set_sigma(a, sigma);
  if (D == 1) {
    a.X = X;
    a.Y = Y;
    a.dX = dX;
    a.dY = dY;
    return launch_pen<T, SRC_FEAT1>(pen, true, a, B, s, what);
  }
  const size_t need = (size_t)B * N * M * sizeof(T);
  if (!ws || ws_bytes < need)
    return fail(TW_ESIZE, "%s: workspace of %zu bytes needed", what, need);
  // the raw squared distances: the forward's, or recomputed into the
  // workspace; the sweep writes their adjoint into the workspace (in place
  // when they are there: each cell is read and written by the same thread)
  if (!ws_fwd) {
    if (int e = sqdist_raw<T>(X, Y, B, N, M, D, ws, s, what)) return e;
  }
  a.C = ws_fwd ? ws_fwd : ws;
  a.dC = ws;
  if (int e = launch_pen<T, SRC_SQ>(pen, true, a, B, s, what)) return e;
  return sqdist_raw_bwd<T>(X, Y, ws, B, N, M, D, dX, dY, s, what);
}

}  // namespace tw

extern "C" {

size_t tw_udtw_feat_workspace_bytes(int B, int N, int M, int D, int elem_size) {
  if (D <= 1 || B <= 0 || N <= 0 || M <= 0) return 0;
  return (size_t)B * N * M * (size_t)elem_size;
}

int tw_udtw_feat_fwd_f32(const float* X, const float* Y, const float* vx, const float* vy, int B,
                         int N, int M, int D, float gamma, float beta, float eps,
                         float bandwidth, int sigma, float* R, float* P, float* out_dist,
                         float* out_pen, float* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  return feat_fwd<float>(X, Y, vx, vy, B, N, M, D, gamma, beta, eps, bandwidth, sigma, R, P,
                         out_dist, out_pen, workspace, workspace_bytes, stream,
                         "tw_udtw_feat_fwd_f32");
}

int tw_udtw_feat_fwd_f64(const double* X, const double* Y, const double* vx, const double* vy,
                         int B, int N, int M, int D, double gamma, double beta, double eps,
                         double bandwidth, int sigma, double* R, double* P, double* out_dist,
                         double* out_pen, double* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  return feat_fwd<double>(X, Y, vx, vy, B, N, M, D, gamma, beta, eps, bandwidth, sigma, R, P,
                          out_dist, out_pen, workspace, workspace_bytes, stream,
                          "tw_udtw_feat_fwd_f64");
}

int tw_udtw_feat_bwd_f32(const float* X, const float* Y, const float* vx, const float* vy,
                         const float* R, const float* P, const float* grad_dist,
                         const float* grad_pen, int B, int N, int M, int D, float gamma,
                         float beta, float eps, float bandwidth, int sigma, int grad_stride,
                         float* dX, float* dY, float* dvx, float* dvy,
                         const float* fwd_workspace, float* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  return feat_bwd<float>(X, Y, vx, vy, R, P, grad_dist, grad_pen, B, N, M, D, gamma, beta, eps,
                         bandwidth, sigma, grad_stride, dX, dY, dvx, dvy, fwd_workspace,
                         workspace, workspace_bytes, stream, "tw_udtw_feat_bwd_f32");
}

int tw_udtw_feat_bwd_f64(const double* X, const double* Y, const double* vx, const double* vy,
                         const double* R, const double* P, const double* grad_dist,
                         const double* grad_pen, int B, int N, int M, int D, double gamma,
                         double beta, double eps, double bandwidth, int sigma, int grad_stride,
                         double* dX, double* dY, double* dvx, double* dvy,
                         const double* fwd_workspace, double* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  return feat_bwd<double>(X, Y, vx, vy, R, P, grad_dist, grad_pen, B, N, M, D, gamma, beta, eps,
                          bandwidth, sigma, grad_stride, dX, dY, dvx, dvy, fwd_workspace,
                          workspace, workspace_bytes, stream, "tw_udtw_feat_bwd_f64");
}

}  // extern "C"
