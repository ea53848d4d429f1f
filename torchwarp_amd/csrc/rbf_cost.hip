// RBF-style base cost between the rows of two feature blocks, per pair p:
//   cost[r, c] = sum_d 2 - 2 exp(-sigma (a_rd - b_cd)^2)
// (jeanie/distances.py:41-51). The per-feature exponential is not a matrix
// product, so there is no MFMA form: the kernels stream the features, which
// stay in L1/L2 (a pair's rows are reused by every output of the pair), and
// are bound by one exponential per (r, c, d) term. The [.., T, U, D]
// difference tensor of the reference is never formed.
//
// Backward, with t = a_rd - b_cd and e = exp(-sigma t^2):
//   dA[r, d] =  4 sigma sum_c dcost[r, c] t e
//   dB[c, d] = -4 sigma sum_r dcost[r, c] t e
// one thread per output element along d (coalesced feature reads), summing
// in a fixed order.

#include "tw_capi.hpp"
#include "tw_common.hpp"
#include "../../include/torchwarp_hip.h"

namespace tw {

__device__ __forceinline__ float exp_v(float x) { return expf(x); }
__device__ __forceinline__ double exp_v(double x) { return exp(x); }

template <typename T>
__global__ void __launch_bounds__(256) rbf_fwd_kernel(const T* __restrict__ A,
                                                      const T* __restrict__ Bm,
                                                      T* __restrict__ out, int R, int C, int D,
                                                      T sigma) {
  const int p = blockIdx.y;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long long)R * C) return;
  const int r = (int)(idx / C), c = (int)(idx % C);
  const T* a = A + ((size_t)p * R + r) * D;
  const T* b = Bm + ((size_t)p * C + c) * D;
  T acc = 0;
  for (int d = 0; d < D; ++d) {
    const T t = a[d] - b[d];
    acc += (T)2 - (T)2 * exp_v(-sigma * (t * t));
  }
  out[(size_t)p * R * C + idx] = acc;
}

// COLS false: dA (owned = rows of A, summed over the columns of the cost);
// COLS true: dB (owned = rows of Bm, summed over the cost's rows).
template <typename T, bool COLS>
__global__ void __launch_bounds__(256) rbf_bwd_kernel(const T* __restrict__ A,
                                                      const T* __restrict__ Bm,
                                                      const T* __restrict__ dcost,
                                                      T* __restrict__ dOut, int R, int C, int D,
                                                      T sigma) {
  const int p = blockIdx.y;
  const int nown = COLS ? C : R, nsum = COLS ? R : C;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long long)nown * D) return;
  const int o = (int)(idx / D), d = (int)(idx % D);
  const T* self = (COLS ? Bm + (size_t)p * C * D : A + (size_t)p * R * D) + (size_t)o * D + d;
  const T* other = (COLS ? A + (size_t)p * R * D : Bm + (size_t)p * C * D) + d;
  const T* g = dcost + (size_t)p * R * C;
  const T x = *self;
  T acc = 0;
  for (int s = 0; s < nsum; ++s) {
    const T t = COLS ? other[(size_t)s * D] - x : x - other[(size_t)s * D];
    const T gs = COLS ? g[(size_t)s * C + o] : g[(size_t)o * C + s];
    acc += gs * t * exp_v(-sigma * (t * t));
  }
  dOut[(size_t)p * nown * D + idx] = (COLS ? (T)-4 : (T)4) * sigma * acc;
}

static inline unsigned rbf_blocks(long long n) { return (unsigned)((n + 255) / 256); }
// Pairs per launch: the pair index is grid.y (at most 65535).
constexpr int kRbfMaxPairs = 65535;

template <typename T>
static int rbf_check(const T* A, const T* Bm, int P, int R, int C, int D, double sigma,
                     const char* what) {
  if (P < 0 || R < 0 || C < 0 || D < 0) return fail(TW_EINVAL, "%s: bad sizes", what);
  if (!(sigma > 0.0)) return fail(TW_EINVAL, "%s: sigma must be > 0", what);
  if ((long long)R * C > (1LL << 40) || (long long)(R > C ? R : C) * D > (1LL << 40))
    return fail(TW_ESIZE, "%s: plane too large", what);
  if (P > 0 && D > 0 && ((R > 0 && !A) || (C > 0 && !Bm)))
    return fail(TW_EINVAL, "%s: null pointer", what);
  return TW_OK;
}

template <typename T>
static int rbf_fwd(const T* A, const T* Bm, int P, int R, int C, int D, T sigma, T* out,
                   hipStream_t s, const char* what) {
  if (int e = rbf_check(A, Bm, P, R, C, D, (double)sigma, what)) return e;
  if (P == 0 || R == 0 || C == 0) return TW_OK;
  if (!out) return fail(TW_EINVAL, "%s: null pointer", what);
  for (int p0 = 0; p0 < P; p0 += kRbfMaxPairs) {
    const int np = P - p0 < kRbfMaxPairs ? P - p0 : kRbfMaxPairs;
    hipLaunchKernelGGL(rbf_fwd_kernel<T>, dim3(rbf_blocks((long long)R * C), np), dim3(256), 0, s,
                       A + (size_t)p0 * R * D, Bm + (size_t)p0 * C * D, out + (size_t)p0 * R * C,
                       R, C, D, sigma);
    if (int e = check_launch(what)) return e;
  }
  return TW_OK;
}

template <typename T>
static int rbf_bwd(const T* A, const T* Bm, const T* dcost, int P, int R, int C, int D, T sigma,
                   T* dA, T* dB, hipStream_t s, const char* what) {
  if (int e = rbf_check(A, Bm, P, R, C, D, (double)sigma, what)) return e;
  if (P == 0 || D == 0) return TW_OK;
  if ((R > 0 && !dA) || (C > 0 && !dB) || ((long long)R * C > 0 && !dcost))
    return fail(TW_EINVAL, "%s: null pointer", what);
  // with no terms to sum (R or C zero) the kernels write zero gradients
  for (int p0 = 0; p0 < P; p0 += kRbfMaxPairs) {
    const int np = P - p0 < kRbfMaxPairs ? P - p0 : kRbfMaxPairs;
    const size_t oa = (size_t)p0 * R * D, ob = (size_t)p0 * C * D, oc = (size_t)p0 * R * C;
    const T* dc = dcost ? dcost + oc : dcost;
    if (R > 0)
      hipLaunchKernelGGL((rbf_bwd_kernel<T, false>), dim3(rbf_blocks((long long)R * D), np),
                         dim3(256), 0, s, A + oa, Bm + ob, dc, dA + oa, R, C, D, sigma);
    if (C > 0)
      hipLaunchKernelGGL((rbf_bwd_kernel<T, true>), dim3(rbf_blocks((long long)C * D), np),
                         dim3(256), 0, s, A + oa, Bm + ob, dc, dB + ob, R, C, D, sigma);
    if (int e = check_launch(what)) return e;
  }
  return TW_OK;
}

}  // namespace tw

using namespace tw;

extern "C" {

int tw_rbf_cost_fwd_f32(const float* A, const float* Bm, int P, int R, int C, int D, float sigma,
                        float* cost, hipStream_t stream) {
  return rbf_fwd<float>(A, Bm, P, R, C, D, sigma, cost, stream, "tw_rbf_cost_fwd_f32");
}

int tw_rbf_cost_fwd_f64(const double* A, const double* Bm, int P, int R, int C, int D,
                        double sigma, double* cost, hipStream_t stream) {
  return rbf_fwd<double>(A, Bm, P, R, C, D, sigma, cost, stream, "tw_rbf_cost_fwd_f64");
}

int tw_rbf_cost_bwd_f32(const float* A, const float* Bm, const float* d_cost, int P, int R, int C,
                        int D, float sigma, float* dA, float* dB, hipStream_t stream) {
  return rbf_bwd<float>(A, Bm, d_cost, P, R, C, D, sigma, dA, dB, stream, "tw_rbf_cost_bwd_f32");
}

int tw_rbf_cost_bwd_f64(const double* A, const double* Bm, const double* d_cost, int P, int R,
                        int C, int D, double sigma, double* dA, double* dB, hipStream_t stream) {
  return rbf_bwd<double>(A, Bm, d_cost, P, R, C, D, sigma, dA, dB, stream,
                         "tw_rbf_cost_bwd_f64");
}

}  // extern "C"
