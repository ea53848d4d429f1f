// Hard (gamma = 0) alignment DP with backtrack for gfx950, float64.
//
// Reference: paths.py:85-127 (_optimal_3d / optimal_path). For a cost D
// [K, T, U] (K = 1 for a plain cost matrix):
//   r[k,0,0] = D[k,0,0] (every k, or only k = start_view)
//   r[k,t,u] = D[k,t,u] + best, best = the first strict minimum of r[kk,a,b]
//              scanned as kk = max(0,k-s) .. min(K-1,k+s) ascending and, for
//              each kk, (a,b) = (t-1,u-1), (t-1,u), (t,u-1); a cell with no
//              finite predecessor keeps r = inf and the zero back pointer.
// The path ends at the first k attaining the minimum of r[:, T-1, U-1] and
// follows the back pointers to (0, 0); a zero back pointer jumps to (0,0,0)
// exactly as the reference's zero-initialised array does.
//
// Every r is one IEEE float64 addition of D and an exact copy of a
// predecessor's r, so values, comparisons and therefore the indices are
// bitwise those of the float64 reference regardless of evaluation order.
// One workgroup per batch item sweeps the anti-diagonals (cells (k, t) of a
// diagonal spread over the threads, r and the back pointers in the caller's
// workspace); thread 0 then walks the back pointers and writes the path in
// forward order.

#include "tw_capi.hpp"
#include "tw_common.hpp"
#include "../../include/torchwarp_hip.h"

namespace tw {

constexpr int kNoArg = -1;   // back pointer of a cell without finite predecessor

__global__ void __launch_bounds__(1024) optimal_path_kernel(const double* __restrict__ D, int K,
                                                            int Tn, int Un, int shift,
                                                            int start_view, double* r, int* back,
                                                            int* path, int* plen) {
  const int b = blockIdx.x;
  const long long plane = (long long)Tn * Un, pair = K * plane;
  const double* Db = D + b * pair;
  double* rb = r + b * pair;
  int* bb = back + b * pair;
  const double INF = __builtin_inf();
  const int Dn = Tn + Un - 1;

  for (int d = 0; d < Dn; ++d) {
    const int lo = max(0, d - Un + 1), hi = min(Tn - 1, d);
    const int cells = (hi - lo + 1) * K;
    for (int idx = threadIdx.x; idx < cells; idx += blockDim.x) {
      const int t = lo + idx / K, k = idx - (idx / K) * K, u = d - t;
      const long long o = k * plane + (long long)t * Un + u;
      double val;
      int code = kNoArg;
      if (d == 0) {
        val = (start_view < 0 || k == start_view) ? Db[o] : INF;
      } else {
        double best = INF;
        const int klo = max(0, k - shift), khi = min(K - 1, k + shift);
        for (int kk = klo; kk <= khi; ++kk) {
          const double* rk = rb + kk * plane;
          if (t > 0 && u > 0) {
            const double v = rk[(long long)(t - 1) * Un + u - 1];
            if (v < best) {
              best = v;
              code = kk * 4 + 0;
            }
          }
          if (t > 0) {
            const double v = rk[(long long)(t - 1) * Un + u];
            if (v < best) {
              best = v;
              code = kk * 4 + 1;
            }
          }
          if (u > 0) {
            const double v = rk[(long long)t * Un + u - 1];
            if (v < best) {
              best = v;
              code = kk * 4 + 2;
            }
          }
        }
        val = code != kNoArg ? Db[o] + best : INF;
      }
      rb[o] = val;
      bb[o] = code;
    }
    __syncthreads();
  }

  if (threadIdx.x == 0) {
    const long long last = (long long)(Tn - 1) * Un + Un - 1;
    int k = 0;
    double m = rb[last];
    for (int kk = 1; kk < K; ++kk) {
      const double v = rb[kk * plane + last];
      if (v < m) {   // first minimum, as np.argmin
        m = v;
        k = kk;
      }
    }
    int t = Tn - 1, u = Un - 1, L = 0;
    int* pb = path + (long long)b * Dn * 3;
    pb[0] = t;
    pb[1] = u;
    pb[2] = k;
    L = 1;
    while ((t != 0 || u != 0) && L < Dn) {
      const int code = bb[k * plane + (long long)t * Un + u];
      if (code == kNoArg) {
        k = t = u = 0;
      } else {
        const int p = code & 3;
        k = code >> 2;
        if (p != 2) --t;
        if (p != 1) --u;
      }
      pb[3 * L] = t;
      pb[3 * L + 1] = u;
      pb[3 * L + 2] = k;
      ++L;
    }
    for (int i = 0, j = L - 1; i < j; ++i, --j)
      for (int c = 0; c < 3; ++c) {
        const int x = pb[3 * i + c];
        pb[3 * i + c] = pb[3 * j + c];
        pb[3 * j + c] = x;
      }
    plen[b] = L;
  }
}

}  // namespace tw

using namespace tw;

extern "C" {

int tw_optimal_path_f64(const double* cost, int B, int K, int T, int U, int max_shift,
                        int start_view, double* r_ws, int* back_ws, int* path, int* path_len,
                        hipStream_t stream) {
  const char* what = "tw_optimal_path_f64";
  if (B < 0 || K <= 0 || T <= 0 || U <= 0) return fail(TW_EINVAL, "%s: bad sizes", what);
  if (max_shift < 0) return fail(TW_EINVAL, "%s: max_shift must be >= 0", what);
  if (start_view >= K) return fail(TW_EINVAL, "%s: start_view %d out of range", what, start_view);
  if (B == 0) return TW_OK;
  if (!cost || !r_ws || !back_ws || !path || !path_len)
    return fail(TW_EINVAL, "%s: null pointer", what);
  if ((long long)K * T >= (1LL << 29) || (long long)K * 4 >= (1LL << 31))
    return fail(TW_ESIZE, "%s: too many viewpoints", what);
  const int cells = (T < U ? T : U) * K;
  int threads = ((cells + 63) / 64) * 64;
  threads = threads < 64 ? 64 : (threads > 1024 ? 1024 : threads);
  hipLaunchKernelGGL(optimal_path_kernel, dim3(B), dim3(threads), 0, stream, cost, K, T, U,
                     max_shift, start_view < 0 ? -1 : start_view, r_ws, back_ws, path, path_len);
  return check_launch(what);
}

}  // extern "C"
