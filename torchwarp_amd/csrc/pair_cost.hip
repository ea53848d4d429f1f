// Pairwise (squared) Euclidean cost between the rows of two feature blocks.
//
// For every pair p: A [R, D] (query frames, or x steps) and Bm [C, D]
// (support frames, or y steps), S[r,c] = |a_r|^2 + |b_c|^2 - 2 a_r . b_c
// (the GEMM form the reference uses, jeanie/distances.py:25-31,
// udtw/_autograd.py:24-29). Metrics:
//   RAW  S unclamped (uDTW keeps the raw value for its gradient mask)
//   SQ   max(S, 0)
//   EUC  sqrt(max(S, 0)), zero gradient at zero distance (distances.py:34-38)
// Backward, from dcost: dS = dcost * (EUC ? 0.5 / cost : 1) where S > 0
// (cost > 0), else 0, then
//   dA = 2 (rowsum(dS) A - dS Bm),  dB = 2 (colsum(dS) Bm - dS^T A).
//
// fp32 with D a multiple of 4 runs on the matrix cores (v_mfma_f32_16x16x4f32,
// one 16x16 output tile per wavefront); every other case on plain FMA.

#include "tw_capi.hpp"
#include "tw_common.hpp"
#include "../../include/torchwarp_hip.h"

namespace tw {

enum { MET_RAW = 0, MET_SQ = 1, MET_EUC = 2 };

template <typename T, int MET>
__device__ __forceinline__ T finish_cost(T s) {
  if (MET == MET_RAW) return s;
  const T sq = s > (T)0 ? s : (T)0;
  return MET == MET_EUC ? sqrt_v(sq) : sq;
}

template <typename T, int MET>
__device__ __forceinline__ T cost_adjoint(T dcost, T cost) {
  if (MET == MET_RAW) return dcost;
  if (!(cost > (T)0)) return (T)0;
  return MET == MET_EUC ? (T)0.5 * dcost / cost : dcost;
}

// ------------------------------------------------------------ FMA kernels

template <typename T, int MET>
__global__ void __launch_bounds__(256) pair_fwd_fma(const T* __restrict__ A,
                                                    const T* __restrict__ Bm, T* __restrict__ out,
                                                    int R, int C, int D) {
  const int p = blockIdx.y;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long long)R * C) return;
  const int r = (int)(idx / C), c = (int)(idx % C);
  const T* a = A + ((size_t)p * R + r) * D;
  const T* bb = Bm + ((size_t)p * C + c) * D;
  T aa = 0, bq = 0, ab = 0;
  for (int d = 0; d < D; ++d) {
    const T x = a[d], y = bb[d];
    aa += x * x;
    bq += y * y;
    ab += x * y;
  }
  out[(size_t)p * R * C + idx] = finish_cost<T, MET>(aa + bq - (T)2 * ab);
}

// dA[r, d] = 2 (sum_c dS[r,c] a[r,d] - sum_c dS[r,c] b[c,d])
template <typename T, int MET>
__global__ void __launch_bounds__(256) pair_bwd_a_fma(const T* __restrict__ A,
                                                      const T* __restrict__ Bm,
                                                      const T* __restrict__ cost,
                                                      const T* __restrict__ dcost,
                                                      T* __restrict__ dA, int R, int C, int D) {
  const int p = blockIdx.y;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long long)R * D) return;
  const int r = (int)(idx / D), d = (int)(idx % D);
  const size_t prc = (size_t)p * R * C + (size_t)r * C;
  T rs = 0, acc = 0;
  for (int c = 0; c < C; ++c) {
    const T ds = cost_adjoint<T, MET>(dcost[prc + c], MET == MET_RAW ? (T)0 : cost[prc + c]);
    rs += ds;
    acc += ds * Bm[((size_t)p * C + c) * D + d];
  }
  dA[((size_t)p * R + r) * D + d] = (T)2 * (rs * A[((size_t)p * R + r) * D + d] - acc);
}

// dB[c, d] = 2 (sum_r dS[r,c] b[c,d] - sum_r dS[r,c] a[r,d])
template <typename T, int MET>
__global__ void __launch_bounds__(256) pair_bwd_b_fma(const T* __restrict__ A,
                                                      const T* __restrict__ Bm,
                                                      const T* __restrict__ cost,
                                                      const T* __restrict__ dcost,
                                                      T* __restrict__ dB, int R, int C, int D) {
  const int p = blockIdx.y;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long long)C * D) return;
  const int c = (int)(idx / D), d = (int)(idx % D);
  T cs = 0, acc = 0;
  for (int r = 0; r < R; ++r) {
    const size_t o = (size_t)p * R * C + (size_t)r * C + c;
    const T ds = cost_adjoint<T, MET>(dcost[o], MET == MET_RAW ? (T)0 : cost[o]);
    cs += ds;
    acc += ds * A[((size_t)p * R + r) * D + d];
  }
  dB[((size_t)p * C + c) * D + d] = (T)2 * (cs * Bm[((size_t)p * C + c) * D + d] - acc);
}

// ------------------------------------------------------------- launchers

static inline unsigned blocks_for(long long n) { return (unsigned)((n + 255) / 256); }

template <typename T>
int pair_cost_fwd(const T* A, const T* Bm, int P, int R, int C, int D, int metric, T* out,
                  hipStream_t s, const char* what) {
  if (P < 0 || R <= 0 || C <= 0 || D <= 0) return fail(TW_EINVAL, "%s: bad sizes", what);
  if (!A || !Bm || !out) return fail(TW_EINVAL, "%s: null pointer", what);
  if (P == 0) return TW_OK;
  if (P > 65535) return fail(TW_ESIZE, "%s: at most 65535 pairs per call", what);
  dim3 grid(blocks_for((long long)R * C), P), block(256);
  switch (metric) {
    case MET_RAW: hipLaunchKernelGGL((pair_fwd_fma<T, MET_RAW>), grid, block, 0, s, A, Bm, out, R, C, D); break;
    case MET_SQ: hipLaunchKernelGGL((pair_fwd_fma<T, MET_SQ>), grid, block, 0, s, A, Bm, out, R, C, D); break;
    case MET_EUC: hipLaunchKernelGGL((pair_fwd_fma<T, MET_EUC>), grid, block, 0, s, A, Bm, out, R, C, D); break;
    default: return fail(TW_EINVAL, "%s: unknown metric %d", what, metric);
  }
  return check_launch(what);
}

template <typename T>
int pair_cost_bwd(const T* A, const T* Bm, const T* cost, const T* dcost, int P, int R, int C,
                  int D, int metric, T* dA, T* dB, hipStream_t s, const char* what) {
  if (P < 0 || R <= 0 || C <= 0 || D <= 0) return fail(TW_EINVAL, "%s: bad sizes", what);
  if (!A || !Bm || !dcost || !dA || !dB) return fail(TW_EINVAL, "%s: null pointer", what);
  if (metric != MET_RAW && !cost) return fail(TW_EINVAL, "%s: metric needs the cost", what);
  if (P == 0) return TW_OK;
  if (P > 65535) return fail(TW_ESIZE, "%s: at most 65535 pairs per call", what);
  dim3 ga(blocks_for((long long)R * D), P), gb(blocks_for((long long)C * D), P), block(256);
#define TW_PAIR_BWD(MET_)                                                                     \
  hipLaunchKernelGGL((pair_bwd_a_fma<T, MET_>), ga, block, 0, s, A, Bm, cost, dcost, dA, R,   \
                     C, D);                                                                   \
  hipLaunchKernelGGL((pair_bwd_b_fma<T, MET_>), gb, block, 0, s, A, Bm, cost, dcost, dB, R,   \
                     C, D);
  switch (metric) {
    case MET_RAW: TW_PAIR_BWD(MET_RAW) break;
    case MET_SQ: TW_PAIR_BWD(MET_SQ) break;
    case MET_EUC: TW_PAIR_BWD(MET_EUC) break;
    default: return fail(TW_EINVAL, "%s: unknown metric %d", what, metric);
  }
#undef TW_PAIR_BWD
  return check_launch(what);
}

template <typename T>
int sqdist_raw(const T* X, const T* Y, int P, int R, int C, int D, T* out, hipStream_t s,
               const char* what) {
  return pair_cost_fwd<T>(X, Y, P, R, C, D, MET_RAW, out, s, what);
}

template <typename T>
int sqdist_raw_bwd(const T* X, const T* Y, const T* dS, int P, int R, int C, int D, T* dX, T* dY,
                   hipStream_t s, const char* what) {
  return pair_cost_bwd<T>(X, Y, nullptr, dS, P, R, C, D, MET_RAW, dX, dY, s, what);
}

template int sqdist_raw<float>(const float*, const float*, int, int, int, int, float*,
                               hipStream_t, const char*);
template int sqdist_raw<double>(const double*, const double*, int, int, int, int, double*,
                                hipStream_t, const char*);
template int sqdist_raw_bwd<float>(const float*, const float*, const float*, int, int, int, int,
                                   float*, float*, hipStream_t, const char*);
template int sqdist_raw_bwd<double>(const double*, const double*, const double*, int, int, int,
                                    int, double*, double*, hipStream_t, const char*);
template int pair_cost_fwd<float>(const float*, const float*, int, int, int, int, int, float*,
                                  hipStream_t, const char*);
template int pair_cost_fwd<double>(const double*, const double*, int, int, int, int, int,
                                   double*, hipStream_t, const char*);
template int pair_cost_bwd<float>(const float*, const float*, const float*, const float*, int,
                                  int, int, int, int, float*, float*, hipStream_t, const char*);
template int pair_cost_bwd<double>(const double*, const double*, const double*, const double*,
                                   int, int, int, int, int, double*, double*, hipStream_t,
                                   const char*);

}  // namespace tw

using namespace tw;

extern "C" {

int tw_pair_cost_fwd_f32(const float* A, const float* Bm, int P, int R, int C, int D, int metric,
                         float* cost, hipStream_t stream) {
  return pair_cost_fwd<float>(A, Bm, P, R, C, D, metric, cost, stream, "tw_pair_cost_fwd_f32");
}

int tw_pair_cost_fwd_f64(const double* A, const double* Bm, int P, int R, int C, int D,
                         int metric, double* cost, hipStream_t stream) {
  return pair_cost_fwd<double>(A, Bm, P, R, C, D, metric, cost, stream, "tw_pair_cost_fwd_f64");
}

int tw_pair_cost_bwd_f32(const float* A, const float* Bm, const float* cost, const float* d_cost,
                         int P, int R, int C, int D, int metric, float* dA, float* dB,
                         hipStream_t stream) {
  return pair_cost_bwd<float>(A, Bm, cost, d_cost, P, R, C, D, metric, dA, dB, stream,
                              "tw_pair_cost_bwd_f32");
}

int tw_pair_cost_bwd_f64(const double* A, const double* Bm, const double* cost,
                         const double* d_cost, int P, int R, int C, int D, int metric,
                         double* dA, double* dB, hipStream_t stream) {
  return pair_cost_bwd<double>(A, Bm, cost, d_cost, P, R, C, D, metric, dA, dB, stream,
                               "tw_pair_cost_bwd_f64");
}

}  // extern "C"
