// uDTW / soft-DTW host entry points for gfx950: argument checks, the
// hyper-parameters of the sweep and the C ABI. The sweep kernels and their
// launchers are in udtw_sweep.hpp.

#include "udtw_sweep.hpp"
#include "udtw_band.hpp"
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

// float calls carry R in double precision (the RD kernels) when the
// accumulated cost can grow large against float32's spacing. R sums up to
// N + M - 1 costs and the backward's weights are exponentials of differences
// of neighbouring R values in units of gamma / log2(e): once
// (N + M - 1) log2(e) / gamma passes kRdScale, float32 R loses the low bits
// those differences need (at N = M = 1024, gamma = 0.1 the gradients would
// carry ~5e-2 relative error; 1e-3 with R in double). One row per thread
// must serve N (the RD kernels' layout), and a pair's R plane in double must
// stay below 2 GiB. TORCHWARP_UDTW_RD = 0 / 1 forces it off / on (where those
// hold).
constexpr double kRdScale = 2048.0;

template <typename T>
static bool carry_double(int N, int M, double gamma) {
  if (sizeof(T) != 4 || N <= 0 || M <= 0 || !(gamma > 0)) return false;
  static const int mode = [] {
    const char* e = getenv("TORCHWARP_UDTW_RD");
    return e ? atoi(e) : -1;
  }();
  if (mode == 0) return false;
  const int n = N < M ? N : M, m = N < M ? M : N;
  if (!mw_long<T>(n) && pick_shape<T>(n, false).rows != 1) return false;
  if ((long long)n * m * 8 >= (1LL << 31)) return false;   // a pair's R plane stays below 2 GiB
  if (mode == 1) return true;
  return (double)(n + m - 1) * 1.4426950408889634 / gamma > kRdScale;
}

// Bytes of the S / dS plane (D > 1) and where the MW hand-off records start
// in a feature-path backward workspace (8-byte aligned).
template <typename T>
static size_t splane_bytes(int B, int N, int M, int D) {
  return D > 1 ? (size_t)B * N * M * sizeof(T) : 0;
}
static size_t align8(size_t n) { return (n + 7) & ~(size_t)7; }

static int check_dims(const char* what, int B, int N, int M, double gamma) {
  if (B < 0 || N <= 0 || M <= 0) return fail(TW_EINVAL, "%s: bad sizes B=%d N=%d M=%d", what, B, N, M);
  if (N > M) return fail(TW_EINVAL, "%s: expected N <= M (got %d > %d)", what, N, M);
  if (!(gamma > 0)) return fail(TW_EINVAL, "%s: gamma must be > 0", what);
  return TW_OK;
}

template <typename T>
static int cost_fwd(const T* C, const T* Q, int B, int N, int M, double gamma, double band, T* R,
                    T* P, T* out_r, T* out_p, hipStream_t s, const char* what,
                    bool allow_rd = true) {
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
  a.rd = allow_rd && carry_double<T>(N, M, gamma);
  set_hyper(a, gamma, 0.0, 1.0, band);
  if (band_path(N, M, band)) return band_cost_fwd<T>(a, B, s, what);
  return launch_pen<T, SRC_COST>(Q != nullptr, false, a, B, s, what);
}

template <typename T>
static int cost_bwd(const T* C, const T* Q, const T* R, const T* P, const T* gr, const T* gp,
                    int B, int N, int M, double gamma, double band, int gstride, T* dC, T* dQ,
                    T* ws, size_t ws_bytes, hipStream_t s, const char* what,
                    bool allow_rd = true) {
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
  a.rd = allow_rd && carry_double<T>(N, M, gamma);
  const size_t need = mw_hand_bytes<T>(B, N, M);
  if (need && (!ws || ws_bytes < need))
    return fail(TW_ESIZE, "%s: workspace of %zu bytes needed", what, need);
  a.hand = need ? reinterpret_cast<unsigned long long*>(ws) : nullptr;
  set_hyper(a, gamma, 0.0, 1.0, band);
  if (band_path(N, M, band)) return band_cost_bwd<T>(a, B, s, what, ws, ws_bytes);
  return launch_pen<T, SRC_COST>(pen, true, a, B, s, what);
}

template <typename T>
int udtw_cost_fwd_any(const T* C, const T* Q, int B, int N, int M, double gamma, double band,
                      T* R, T* P, T* out_r, T* out_p, hipStream_t s, const char* what) {
  return cost_fwd<T>(C, Q, B, N, M, gamma, band, R, P, out_r, out_p, s, what, false);
}
template <typename T>
int udtw_cost_bwd_any(const T* C, const T* Q, const T* R, const T* P, const T* gr, const T* gp,
                      int B, int N, int M, double gamma, T* dC, T* dQ, T* ws, size_t ws_bytes,
                      hipStream_t s, const char* what) {
  return cost_bwd<T>(C, Q, R, P, gr, gp, B, N, M, gamma, 0.0, 1, dC, dQ, ws, ws_bytes, s, what,
                     false);
}
template <typename T>
size_t udtw_cost_hand_bytes(int B, int N, int M) {
  return mw_hand_bytes<T>(B, N < M ? N : M, N < M ? M : N);
}
template size_t udtw_cost_hand_bytes<float>(int, int, int);
template size_t udtw_cost_hand_bytes<double>(int, int, int);
template int udtw_cost_fwd_any<float>(const float*, const float*, int, int, int, double, double,
                                      float*, float*, float*, float*, hipStream_t, const char*);
template int udtw_cost_fwd_any<double>(const double*, const double*, int, int, int, double,
                                       double, double*, double*, double*, double*, hipStream_t,
                                       const char*);
template int udtw_cost_bwd_any<float>(const float*, const float*, const float*, const float*,
                                      const float*, const float*, int, int, int, double, float*,
                                      float*, float*, size_t, hipStream_t, const char*);
template int udtw_cost_bwd_any<double>(const double*, const double*, const double*,
                                       const double*, const double*, const double*, int, int,
                                       int, double, double*, double*, double*, size_t,
                                       hipStream_t, const char*);

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
                         float* d_pen, float* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  return cost_bwd<float>(cost, pen, R, P, grad_dist, grad_pen, B, N, M, gamma, bandwidth,
                         grad_stride, d_cost, d_pen, workspace, workspace_bytes, stream,
                         "tw_udtw_cost_bwd_f32");
}

int tw_udtw_cost_bwd_f64(const double* cost, const double* pen, const double* R,
                         const double* P, const double* grad_dist, const double* grad_pen, int B,
                         int N, int M, double gamma, double bandwidth, int grad_stride,
                         double* d_cost, double* d_pen, double* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  return cost_bwd<double>(cost, pen, R, P, grad_dist, grad_pen, B, N, M, gamma, bandwidth,
                          grad_stride, d_cost, d_pen, workspace, workspace_bytes, stream,
                          "tw_udtw_cost_bwd_f64");
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
  a.rd = carry_double<T>(N, M, gamma);
  set_hyper(a, gamma, beta, eps, band);
  set_sigma(a, sigma);
  // a band narrower than the grid: cost, penalty, R and P in the band layout
  // (D = 1 too), built in the workspace
  const bool banded = band_feat_path(N, M, D, band);
  if (D == 1 && !banded) {
    a.X = X;
    a.Y = Y;
    return launch_pen<T, SRC_FEAT1>(pen, false, a, B, s, what);
  }
  const size_t need = (size_t)B * N * M * sizeof(T);
  if (!ws || ws_bytes < need)
    return fail(TW_ESIZE, "%s: workspace of %zu bytes needed", what, need);
  if (banded) return band_feat_fwd<T>(a, X, Y, D, B, ws, s, what);
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
  a.rd = carry_double<T>(N, M, gamma);
  set_hyper(a, gamma, beta, eps, band);
  set_sigma(a, sigma);
  // a band narrower than the grid: the forward left the band's cost and
  // penalty in its workspace and R / P band-compressed (D = 1 too); the
  // workspace takes dC, dQ (and C, rebuilt when the forward's is not given)
  if (band_feat_path(N, M, D, band)) {
    const size_t need = (size_t)B * N * M * sizeof(T);
    if (!ws || ws_bytes < need)
      return fail(TW_ESIZE, "%s: workspace of %zu bytes needed", what, need);
    return band_feat_bwd<T>(a, X, Y, D, B, ws_fwd, ws, dX, dY, s, what);
  }
  // workspace: the S / dS plane (D > 1), then the MW hand-off records
  const size_t sp = splane_bytes<T>(B, N, M, D), hb = mw_hand_bytes<T>(B, N, M);
  const size_t need = hb ? align8(sp) + hb : sp;
  if (need && (!ws || ws_bytes < need))
    return fail(TW_ESIZE, "%s: workspace of %zu bytes needed", what, need);
  a.hand = hb ? reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws) + align8(sp))
              : nullptr;
  if (D == 1) {
    a.X = X;
    a.Y = Y;
    a.dX = dX;
    a.dY = dY;
    return launch_pen<T, SRC_FEAT1>(pen, true, a, B, s, what);
  }
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

size_t tw_udtw_carry_bytes(int B, int N, int M, double gamma, int elem_size) {
  if (B <= 0 || N <= 0 || M <= 0 || (elem_size != 4 && elem_size != 8)) return 0;
  const bool rd = elem_size == 4 && carry_double<float>(N, M, gamma);
  return (size_t)B * N * M * (rd ? 8 : (size_t)elem_size);
}

size_t tw_udtw_feat_workspace_bytes(int B, int N, int M, int D, int elem_size) {
  if (B <= 0 || N <= 0 || M <= 0 || D <= 0 || (elem_size != 4 && elem_size != 8)) return 0;
  const int n = N < M ? N : M, m = N < M ? M : N;
  const size_t sp = D > 1 ? (size_t)B * N * M * (size_t)elem_size : 0;
  const size_t hb = elem_size == 4 ? mw_hand_bytes<float>(B, n, m) : mw_hand_bytes<double>(B, n, m);
  return hb ? align8(sp) + hb : sp;
}

size_t tw_udtw_feat_band_workspace_bytes(int B, int N, int M, int D, double bandwidth,
                                         int elem_size) {
  if (B <= 0 || N <= 0 || M <= 0 || D <= 0 || (elem_size != 4 && elem_size != 8)) return 0;
  const int n = N < M ? N : M, m = N < M ? M : N;
  if (band_feat_path(n, m, D, bandwidth)) return (size_t)B * N * M * (size_t)elem_size;
  return tw_udtw_feat_workspace_bytes(B, N, M, D, elem_size);
}

size_t tw_udtw_cost_workspace_bytes(int B, int N, int M, int elem_size) {
  if (B <= 0 || N <= 0 || M <= 0 || (elem_size != 4 && elem_size != 8)) return 0;
  const int n = N < M ? N : M, m = N < M ? M : N;
  return elem_size == 4 ? mw_hand_bytes<float>(B, n, m) : mw_hand_bytes<double>(B, n, m);
}

size_t tw_udtw_cost_band_workspace_bytes(int B, int N, int M, double bandwidth, int elem_size) {
  if (B <= 0 || N <= 0 || M <= 0 || (elem_size != 4 && elem_size != 8)) return 0;
  const int n = N < M ? N : M, m = N < M ? M : N;
  const size_t band = band_cost_workspace_elems(B, n, m, bandwidth) * (size_t)elem_size;
  const size_t hand = tw_udtw_cost_workspace_bytes(B, N, M, elem_size);
  return band > hand ? band : hand;
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
