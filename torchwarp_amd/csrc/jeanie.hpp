// JEANIE DP kernels shared between the compilation units of the path: the
// launch arguments, the caller-layout index and the wavefront-per-pair
// kernels' launchers (jeanie_wave.hip).

#pragma once

#include "tw_capi.hpp"
#include "tw_common.hpp"

namespace tw {

template <typename T>
struct JeanieArgs {
  const T* C;
  const T* R;   // backward input
  T* Rw;        // forward output
  T* out;
  const T* gout;
  const T* gR;
  T* dC;
  int K1, K2, K, Tn, Un, s1, s2;
  int swap;
  T k;       // log2(e) / gamma
  T inv_k;   // gamma ln 2
};

template <typename T>
__device__ __forceinline__ size_t jidx(const JeanieArgs<T>& a, int n, int t, int u) {
  const size_t plane = (size_t)a.Tn * a.Un;
  return (size_t)n * plane + (a.swap ? (size_t)u * a.Tn + t : (size_t)t * a.Un + u);
}

// Wavefront-per-pair kernels (jeanie_wave.hip). Each returns TW_OK after
// launching, or kJ3Unsupported when the shape needs the other kernels.
constexpr int kJ3Unsupported = -1000;
template <typename T>
int jeanie3_fwd(const JeanieArgs<T>& a, int B, hipStream_t s, const char* what);
template <typename T>
int jeanie3_bwd(const JeanieArgs<T>& a, int B, hipStream_t s, const char* what);

}  // namespace tw
