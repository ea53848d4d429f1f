// JEANIE temporal-viewpoint DP for gfx950 (cost path), forward and backward.
//
// Reference: jeanie_cuda.cu:144-295 (kernels), jeanie/_torch_dp.py:14-75,
// jeanie/functional.py:28-61. For a pair b, viewpoints n = (n1, n2) on a
// K1 x K2 grid and temporal cells (t, u):
//   R[n,0,0] = C[n,0,0]
//   R[n,t,u] = C[n,t,u] + softmin_g{ R[n',t',u'] : |n1'-n1| <= s1, |n2'-n2| <= s2,
//                                   (t',u') in {(t-1,u), (t,u-1), (t-1,u-1)} }
//   out      = softmin_g{ R[n,T-1,U-1] }
// Backward: Rbar_k = sum_s 2^((E_s - R_k) log2(e)/g) Rbar_s (+ dL/dR_k),
// E_s = R_s - C_s, seeded with grad_out * softmax_n(-R[n,T-1,U-1]/g); dC = Rbar.
//
// Layout: C, R, dL/dR and dC share one natural layout [B, K1*K2, T, U]; with
// `swap` set, the (t, u) plane is stored transposed ([U, T]) -- the DP runs on
// the T <= U orientation without copying the caller's tensor. R is the true
// (unscaled) accumulator, since callers may request it.
//
// One workgroup per pair; each diagonal's cells (t, n) are spread over the
// threads. The two previous diagonals live in LDS (3 rolling slabs of T*K);
// when they do not fit, the kernel reads them back from the R output in
// global memory (full-fence barrier per diagonal).

#include <stdlib.h>

#include "jeanie.hpp"
#include "../../include/torchwarp_hip.h"

namespace tw {

template <typename T, bool LDSBUF>
__global__ void __launch_bounds__(1024) jeanie_fwd_kernel(JeanieArgs<T> a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* buf = reinterpret_cast<T*>(smem_raw);   // [3][T*K] (LDSBUF)
  const int K = a.K, Tn = a.Tn, Un = a.Un, K2 = a.K2;
  const int b = blockIdx.x;
  const size_t pair = (size_t)K * Tn * Un;
  const T* Cb = a.C + b * pair;
  T* Rb = a.Rw + b * pair;
  const int slab = Tn * K;
  const T INF = inf_v<T>();
  const int Dn = Tn + Un - 1;

  // R of a cell on a previous diagonal
  auto Rget = [&](int d, int t, int n) -> T {
    if (LDSBUF) return buf[(d % 3) * slab + t * K + n];
    return Rb[jidx(a, n, t, d - t)];
  };

  for (int d = 0; d < Dn; ++d) {
    const int lo = max(0, d - Un + 1), hi = min(Tn - 1, d);
    const int cells = (hi - lo + 1) * K;
    for (int idx = threadIdx.x; idx < cells; idx += blockDim.x) {
      const int t = lo + idx / K, n = idx - (idx / K) * K, u = d - t;
      const size_t o = jidx(a, n, t, u);
      T rv = Cb[o];
      if (d > 0) {
        const int n1 = n / K2, n2 = n - n1 * K2;
        const int a1lo = max(0, n1 - a.s1), a1hi = min(a.K1 - 1, n1 + a.s1);
        const int a2lo = max(0, n2 - a.s2), a2hi = min(K2 - 1, n2 + a.s2);
        T m = INF;
        for (int a1 = a1lo; a1 <= a1hi; ++a1)
          for (int a2 = a2lo; a2 <= a2hi; ++a2) {
            const int pn = a1 * K2 + a2;
            if (t > 0) m = fmin(m, Rget(d - 1, t - 1, pn));
            if (u > 0) m = fmin(m, Rget(d - 1, t, pn));
            if (t > 0 && u > 0) m = fmin(m, Rget(d - 2, t - 1, pn));
          }
        T s = 0;
        for (int a1 = a1lo; a1 <= a1hi; ++a1)
          for (int a2 = a2lo; a2 <= a2hi; ++a2) {
            const int pn = a1 * K2 + a2;
            if (t > 0) s += ex2((m - Rget(d - 1, t - 1, pn)) * a.k);
            if (u > 0) s += ex2((m - Rget(d - 1, t, pn)) * a.k);
            if (t > 0 && u > 0) s += ex2((m - Rget(d - 2, t - 1, pn)) * a.k);
          }
        rv += m - a.inv_k * lg2(s);
      }
      if (LDSBUF) buf[(d % 3) * slab + t * K + n] = rv;
      Rb[o] = rv;
    }
    if (LDSBUF)
      lds_barrier();
    else
      __syncthreads();
  }
  if (threadIdx.x == 0) {
    T m = INF;
    for (int n = 0; n < K; ++n) m = fmin(m, Rget(Dn - 1, Tn - 1, n));
    T s = 0;
    for (int n = 0; n < K; ++n) s += ex2((m - Rget(Dn - 1, Tn - 1, n)) * a.k);
    a.out[b] = m - a.inv_k * lg2(s);
  }
}

template <typename T, bool LDSBUF>
__global__ void __launch_bounds__(1024) jeanie_bwd_kernel(JeanieArgs<T> a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* Gb = reinterpret_cast<T*>(smem_raw);    // Rbar  [3][T*K] (LDSBUF)
  const int K = a.K, Tn = a.Tn, Un = a.Un, K2 = a.K2;
  const int slab = Tn * K;
  T* Eb = Gb + 3 * slab;                     // R - C [3][T*K] (LDSBUF)
  __shared__ T fin_s;
  const int b = blockIdx.x;
  const size_t pair = (size_t)K * Tn * Un;
  const T* Cb = a.C + b * pair;
  const T* Rb = a.R + b * pair;
  const T* gRb = a.gR ? a.gR + b * pair : nullptr;
  T* dCb = a.dC + b * pair;
  const T INF = inf_v<T>();
  const int Dn = Tn + Un - 1;
  const T gout = a.gout[b];

  auto Gget = [&](int d, int t, int n) -> T {
    if (LDSBUF) return Gb[(d % 3) * slab + t * K + n];
    return dCb[jidx(a, n, t, d - t)];
  };
  auto Eget = [&](int d, int t, int n) -> T {
    if (LDSBUF) return Eb[(d % 3) * slab + t * K + n];
    const size_t o = jidx(a, n, t, d - t);
    return Rb[o] - Cb[o];
  };

  if (threadIdx.x == 0) {
    T m = INF;
    for (int n = 0; n < K; ++n) m = fmin(m, Rb[jidx(a, n, Tn - 1, Un - 1)]);
    T s = 0;
    for (int n = 0; n < K; ++n) s += ex2((m - Rb[jidx(a, n, Tn - 1, Un - 1)]) * a.k);
    fin_s = m - a.inv_k * lg2(s);
  }
  __syncthreads();
  const T fin = fin_s;

  for (int d = Dn - 1; d >= 0; --d) {
    const int lo = max(0, d - Un + 1), hi = min(Tn - 1, d);
    const int cells = (hi - lo + 1) * K;
    for (int idx = threadIdx.x; idx < cells; idx += blockDim.x) {
      const int t = lo + idx / K, n = idx - (idx / K) * K, u = d - t;
      const size_t o = jidx(a, n, t, u);
      const T rk = Rb[o];
      T acc;
      if (d == Dn - 1) {
        acc = gout * ex2((fin - rk) * a.k);
      } else {
        const int n1 = n / K2, n2 = n - n1 * K2;
        const int a1lo = max(0, n1 - a.s1), a1hi = min(a.K1 - 1, n1 + a.s1);
        const int a2lo = max(0, n2 - a.s2), a2hi = min(K2 - 1, n2 + a.s2);
        acc = 0;
        for (int a1 = a1lo; a1 <= a1hi; ++a1)
          for (int a2 = a2lo; a2 <= a2hi; ++a2) {
            const int sn = a1 * K2 + a2;
            if (t + 1 < Tn) acc += ex2((Eget(d + 1, t + 1, sn) - rk) * a.k) * Gget(d + 1, t + 1, sn);
            if (u + 1 < Un) acc += ex2((Eget(d + 1, t, sn) - rk) * a.k) * Gget(d + 1, t, sn);
            if (t + 1 < Tn && u + 1 < Un)
              acc += ex2((Eget(d + 2, t + 1, sn) - rk) * a.k) * Gget(d + 2, t + 1, sn);
          }
      }
      if (gRb) acc += gRb[o];
      if (LDSBUF) {
        Gb[(d % 3) * slab + t * K + n] = acc;
        Eb[(d % 3) * slab + t * K + n] = rk - Cb[o];
      }
      dCb[o] = acc;
    }
    if (LDSBUF)
      lds_barrier();
    else
      __syncthreads();
  }
}

// --------------------------------------------------------- JEANIE v2
//
// The viewpoint window is a product W1 x W2 (|n1'-n1| <= s1, |n2'-n2| <= s2)
// and a softmin over a union of disjoint sets is the softmin of their
// softmins, so
//   R[n,t,u] = C + softmin{ Rw[n,t-1,u], Rw[n,t,u-1], Rw[n,t-1,u-1] },
//   Rw[n,.]  = softmin_{a1 in W1(n1)} S2[a1,n2],  S2[a1,n2] = softmin_{a2 in W2(n2)} R[a1,a2]
// exactly: a cell costs 3 + (2 s2 + 1) + (2 s1 + 1) exps instead of
// 3 (2 s1 + 1)(2 s2 + 1). The backward runs the same three stages in reverse:
//   RWbar[n,tau] = sum_{s in temporal successors} Rbar_s 2^(Fh_s - Rwh[n,tau]),  Fh = Rh - Ch
//   S2bar[a1,n2] = sum_{n1: |n1-a1| <= s1} RWbar[n1,n2] 2^(Rwh[n1,n2] - S2h[a1,n2])
//   Rbar[a1,a2]  = sum_{n2: |n2-a2| <= s2} S2bar[a1,n2] 2^(S2h[a1,n2] - Rh[a1,a2]) (+ seeds)
// with Rw and S2 recomputed from R (cheaper than carrying them through HBM).
//
// Threads: one group of KP lanes (KP = power of two >= K, <= 64) per DP row
// t, one lane per viewpoint n = n1 K2 + n2, so a group never straddles a
// wavefront: window neighbours come from ds_bpermute shuffles with no
// barrier. Only the temporal "up" value crosses groups, through a two-slot
// LDS ring (one barrier per diagonal); "left" and "diagonal" stay in
// registers. With STAGE the pair's cost (and R) sits in LDS as [t][u][n]
// (n fastest: conflict-free per diagonal) and moves to and from HBM with
// coalesced loops in the caller's layout.

template <typename T, int SMAX>
__device__ __forceinline__ T win_softmin(T v, int lane, int stride, int pos, int cnt, int s) {
  if (s == 0) return v;
  T w[2 * SMAX + 1];
  T m = inf_v<T>();
#pragma unroll
  for (int o = -SMAX; o <= SMAX; ++o) {
    T x = __shfl(v, lane + o * stride);
    const bool in = o >= -s && o <= s && pos + o >= 0 && pos + o < cnt;
    x = in ? x : inf_v<T>();
    w[o + SMAX] = x;
    m = fmin(m, x);
  }
  T sum = 0;
#pragma unroll
  for (int o = -SMAX; o <= SMAX; ++o)
    if (o >= -s && o <= s) sum += ex2(m - w[o + SMAX]);
  return m - lg2(sum);
}

// sum over window neighbours q = lane + o stride of g[q] 2^(h[q] - x)
template <typename T, int SMAX>
__device__ __forceinline__ T win_adjoint(T g, T h, T x, int lane, int stride, int pos, int cnt,
                                         int s) {
  if (s == 0) return g;
  T acc = 0;
#pragma unroll
  for (int o = -SMAX; o <= SMAX; ++o) {
    const T gq = __shfl(g, lane + o * stride);
    const T hq = __shfl(h, lane + o * stride);
    const bool in = o >= -s && o <= s && pos + o >= 0 && pos + o < cnt;
    if (o >= -s && o <= s) acc += in ? gq * ex2(hq - x) : (T)0;
  }
  return acc;
}

// The same two reductions along the stride-1 axis (neighbouring lanes), with
// DPP wave shifts instead of LDS-routed shuffles; offsets beyond +-1 chain
// shifts. The shift's source lane is masked by `pos` exactly as above.
template <typename T>
__device__ __forceinline__ T lane_shift(T v, int o) {
  // o in [-2, 2]: value of lane (l + o)
  if (o == -1) return shift_prev(v, v);
  if (o == 1) return shift_next(v, v);
  if (o == -2) return shift_prev(shift_prev(v, v), v);
  if (o == 2) return shift_next(shift_next(v, v), v);
  return v;
}

template <typename T, int SMAX>
__device__ __forceinline__ T win_softmin_dpp(T v, int pos, int cnt, int s) {
  if (s == 0) return v;
  T w[2 * SMAX + 1];
  T m = inf_v<T>();
#pragma unroll
  for (int o = -SMAX; o <= SMAX; ++o) {
    T x = lane_shift(v, o);
    const bool in = o >= -s && o <= s && pos + o >= 0 && pos + o < cnt;
    x = in ? x : inf_v<T>();
    w[o + SMAX] = x;
    m = fmin(m, x);
  }
  T sum = 0;
#pragma unroll
  for (int o = -SMAX; o <= SMAX; ++o)
    if (o >= -s && o <= s) sum += ex2(m - w[o + SMAX]);
  return m - lg2(sum);
}

template <typename T, int SMAX>
__device__ __forceinline__ T win_adjoint_dpp(T g, T h, T x, int pos, int cnt, int s) {
  if (s == 0) return g;
  T acc = 0;
#pragma unroll
  for (int o = -SMAX; o <= SMAX; ++o) {
    if (o < -s || o > s) continue;
    const T gq = lane_shift(g, o);
    const T hq = lane_shift(h, o);
    const bool in = pos + o >= 0 && pos + o < cnt;
    acc += in ? gq * ex2(hq - x) : (T)0;
  }
  return acc;
}

// softmin over the K lanes of a group (in the scaled domain)
template <typename T>
__device__ __forceinline__ T group_softmin(T v, int KP) {
  T m = v;
  for (int o = 1; o < KP; o <<= 1) m = fmin(m, __shfl_xor(m, o));
  T sum = ex2(m - v);
  for (int o = 1; o < KP; o <<= 1) sum += __shfl_xor(sum, o);
  return m - lg2(sum);
}

// (t, u) of position r of a caller-layout plane ([T][U], or [U][T] with swap), as t * U + u
template <typename T>
__device__ __forceinline__ int caller_tu(const JeanieArgs<T>& a, int r) {
  const int inner = a.swap ? a.Tn : a.Un;
  const int q = r / inner, rem = r - q * inner;
  const int t = a.swap ? rem : q, u = a.swap ? q : rem;
  return t * a.Un + u;
}

template <typename T, bool STAGE, int SMAX>
__global__ void __launch_bounds__(1024) jeanie2_fwd_kernel(JeanieArgs<T> a, int KP) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int K = a.K, Tn = a.Tn, Un = a.Un, K2 = a.K2, K1 = a.K1;
  const int b = blockIdx.x, tid = threadIdx.x, nthr = blockDim.x, lane = tid & 63;
  const int t = tid / KP, n = tid - t * KP;
  const bool vn = n < K && t < Tn;
  const int n1 = vn ? n / K2 : 0, n2 = vn ? n - n1 * K2 : 0;
  const int plane = Tn * Un;
  const size_t pair = (size_t)K * plane;
  const T* Cb = a.C + b * pair;
  T* Rb = a.Rw + b * pair;
  const T INF = inf_v<T>();
  const int Dn = Tn + Un - 1;

  T* ring = reinterpret_cast<T*>(smem_raw);   // [2][nthr] Rwh of the last diagonal
  T* Cs = ring + 2 * nthr;                    // STAGE: [t][u][n] scaled cost
  T* Rs = Cs + pair;                          // STAGE: [t][u][n] R (unscaled)
  if (STAGE) {
    // eight loads in flight per thread, then the scattered LDS stores
    for (int e0 = 0; e0 < (int)pair; e0 += 8 * nthr) {
      T v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = e0 + j * nthr + tid;
        v[j] = e < (int)pair ? Cb[e] : (T)0;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = e0 + j * nthr + tid;
        const int nn = e / plane;
        if (e < (int)pair) Cs[caller_tu(a, e - nn * plane) * K + nn] = v[j] * a.k;
      }
    }
    __syncthreads();
  }

  // rows t_lo .. t_lo + 64/KP - 1 share this wavefront; a wavefront with no
  // row on the diagonal only publishes the neutral values its neighbours read
  const int t_lo = __builtin_amdgcn_readfirstlane(tid >> 6) * (64 / KP);
  const int t_hi = t_lo + 64 / KP - 1;
  T lf = INF, dgv = INF, rh = INF;
  for (int d = 0; d < Dn; ++d) {
    if (t_lo > min(Tn - 1, d) || t_hi < max(0, d - Un + 1)) {
      ring[(d & 1) * nthr + tid] = INF;
      lf = dgv = rh = INF;
      lds_barrier();
      continue;
    }
    const int u = d - t;
    const bool valid = vn && u >= 0 && u < Un;
    T up = (d > 0 && t > 0) ? ring[((d - 1) & 1) * nthr + tid - KP] : INF;
    T ch = (T)0;
    if (valid) ch = STAGE ? Cs[(t * Un + u) * K + n] : Cb[jidx(a, n, t, u)] * a.k;
    if (d == 0) {
      rh = ch;   // cells (n, 0, 0): every viewpoint may start
    } else {
      const T m = min3(up, lf, dgv);
      const T sum = ex2(m - up) + ex2(m - lf) + ex2(m - dgv);
      rh = ch + m - lg2(sum);
    }
    rh = valid ? rh : INF;
    const T s2h = win_softmin_dpp<T, SMAX>(rh, n2, K2, a.s2);
    T rwh = win_softmin<T, SMAX>(s2h, lane, K2, n1, K1, a.s1);
    rwh = valid ? rwh : INF;
    if (valid) {
      const T rv = rh * a.inv_k;
      if (STAGE)
        Rs[(t * Un + u) * K + n] = rv;
      else
        Rb[jidx(a, n, t, u)] = rv;
    }
    ring[(d & 1) * nthr + tid] = rwh;
    dgv = up;
    lf = rwh;
    lds_barrier();
  }
  // out = softmin over the viewpoints of R[., T-1, U-1] (the last row group holds them)
  const T fin = group_softmin(vn ? rh : INF, KP);
  if (t == Tn - 1 && n == 0) a.out[b] = fin * a.inv_k;
  if (STAGE) {
    __syncthreads();
    for (int e = tid; e < (int)pair; e += nthr) {
      const int nn = e / plane;
      Rb[e] = Rs[caller_tu(a, e - nn * plane) * K + nn];
    }
  }
}

template <typename T, bool STAGE, int SMAX>
__global__ void __launch_bounds__(1024) jeanie2_bwd_kernel(JeanieArgs<T> a, int KP) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int K = a.K, Tn = a.Tn, Un = a.Un, K2 = a.K2, K1 = a.K1;
  const int b = blockIdx.x, tid = threadIdx.x, nthr = blockDim.x, lane = tid & 63;
  const int t = tid / KP, n = tid - t * KP;
  const bool vn = n < K && t < Tn;
  const int n1 = vn ? n / K2 : 0, n2 = vn ? n - n1 * K2 : 0;
  const int plane = Tn * Un;
  const size_t pair = (size_t)K * plane;
  const T* Cb = a.C + b * pair;
  const T* Rb = a.R + b * pair;
  const T* gRb = a.gR ? a.gR + b * pair : nullptr;
  T* dCb = a.dC + b * pair;
  const T INF = inf_v<T>();
  const int Dn = Tn + Un - 1;
  const T gout = a.gout[b];

  T* ringF = reinterpret_cast<T*>(smem_raw);   // [2][nthr] Fh = Rh - Ch of the last diagonal
  T* ringG = ringF + 2 * nthr;                 // [2][nthr] Rbar of the last diagonal
  T* Cs = ringG + 2 * nthr;                    // STAGE: [t][u][n] scaled cost, then dC
  T* Rs = Cs + pair;                           // STAGE: [t][u][n] scaled R
  if (STAGE) {
    for (int e0 = 0; e0 < (int)pair; e0 += 4 * nthr) {
      T vc[4], vr[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = e0 + j * nthr + tid;
        vc[j] = e < (int)pair ? Cb[e] : (T)0;
        vr[j] = e < (int)pair ? Rb[e] : (T)0;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = e0 + j * nthr + tid;
        const int nn = e / plane;
        const int l = caller_tu(a, e - nn * plane) * K + nn;
        if (e < (int)pair) {
          Cs[l] = vc[j] * a.k;
          Rs[l] = vr[j] * a.k;
        }
      }
    }
    __syncthreads();
  }

  const int t_lo = __builtin_amdgcn_readfirstlane(tid >> 6) * (64 / KP);
  const int t_hi = t_lo + 64 / KP - 1;
  T Fr = -INF, Gr = 0, Fdg = -INF, Gdg = 0, fin = INF;
  for (int d = Dn - 1; d >= 0; --d) {
    if (t_lo > min(Tn - 1, d) || t_hi < max(0, d - Un + 1)) {
      // no row of this wavefront on diagonal d (see the forward)
      ringF[(d & 1) * nthr + tid] = -INF;
      ringG[(d & 1) * nthr + tid] = (T)0;
      Fr = Fdg = -INF;
      Gr = Gdg = (T)0;
      lds_barrier();
      continue;
    }
    const int u = d - t;
    const bool valid = vn && u >= 0 && u < Un;
    const bool has_down = d < Dn - 1 && t + 1 < Tn;
    const int dslot = ((d + 1) & 1) * nthr + tid + KP;
    const T Fd = has_down ? ringF[dslot] : -INF;
    const T Gd = has_down ? ringG[dslot] : (T)0;
    T rh = INF, ch = 0;
    if (valid) {
      if (STAGE) {
        const int l = (t * Un + u) * K + n;
        rh = Rs[l];
        ch = Cs[l];
      } else {
        const size_t o = jidx(a, n, t, u);
        rh = Rb[o] * a.k;
        ch = Cb[o] * a.k;
      }
    }
    if (d == Dn - 1) fin = group_softmin(rh, KP);   // valid lanes: the last row group
    const T s2h = win_softmin_dpp<T, SMAX>(rh, n2, K2, a.s2);
    const T rwh = win_softmin<T, SMAX>(s2h, lane, K2, n1, K1, a.s1);
    T wbar = Gr * ex2(Fr - rwh) + Gd * ex2(Fd - rwh) + Gdg * ex2(Fdg - rwh);
    wbar = valid ? wbar : (T)0;
    const T s2bar = win_adjoint<T, SMAX>(wbar, valid ? rwh : (T)0, s2h, lane, K2, n1, K1, a.s1);
    T rbar = win_adjoint_dpp<T, SMAX>(valid ? s2bar : (T)0, valid ? s2h : (T)0, rh, n2, K2, a.s2);
    if (d == Dn - 1) rbar += gout * ex2(fin - rh);
    if (gRb && valid) rbar += gRb[jidx(a, n, t, u)];
    rbar = valid ? rbar : (T)0;
    const T F = valid ? rh - ch : -INF;
    if (valid) {
      if (STAGE)
        Cs[(t * Un + u) * K + n] = rbar;   // the cell's cost is no longer needed
      else
        dCb[jidx(a, n, t, u)] = rbar;
    }
    ringF[(d & 1) * nthr + tid] = F;
    ringG[(d & 1) * nthr + tid] = rbar;
    Fdg = Fd;
    Gdg = Gd;
    Fr = F;
    Gr = rbar;
    lds_barrier();
  }
  if (STAGE) {
    __syncthreads();
    for (int e = tid; e < (int)pair; e += nthr) {
      const int nn = e / plane;
      dCb[e] = Cs[caller_tu(a, e - nn * plane) * K + nn];
    }
  }
}

// Launch shape of the v2 kernels: 0 threads when the shape needs the
// general kernels (more than 64 viewpoints, shifts above 2, > 1024 threads).
struct J2Shape {
  int KP, threads, smax;
};
static J2Shape jeanie2_shape(int K, int Tn, int s1, int s2) {
  J2Shape sh = {0, 0, 0};
  if (K > 64 || s1 > 2 || s2 > 2) return sh;
  int kp = 1;
  while (kp < K) kp <<= 1;
  const int threads = ((Tn * kp + 63) / 64) * 64;
  if (threads > 1024) return sh;
  sh.KP = kp;
  sh.threads = threads;
  sh.smax = (s1 > 1 || s2 > 1) ? 2 : 1;
  return sh;
}

// The wavefront-per-pair kernels serve every shape they support unless
// TORCHWARP_JEANIE_V2=1 selects the workgroup-per-pair kernels (for
// comparisons).
static bool j3_enabled() {
  static const bool on = [] {
    const char* e = getenv("TORCHWARP_JEANIE_V2");
    return !(e && e[0] == '1');
  }();
  return on;
}

static int jeanie_threads(int cells) {
  int t = ((cells + 63) / 64) * 64;
  return t < 64 ? 64 : (t > 1024 ? 1024 : t);
}

template <typename T>
static int jeanie_check(const char* what, int B, int K1, int K2, int Tn, int Un, int s1, int s2,
                        double gamma) {
  if (B < 0 || K1 <= 0 || K2 <= 0 || Tn <= 0 || Un <= 0)
    return fail(TW_EINVAL, "%s: bad sizes", what);
  if (s1 < 0 || s2 < 0) return fail(TW_EINVAL, "%s: shifts must be >= 0", what);
  if (!(gamma > 0)) return fail(TW_EINVAL, "%s: gamma must be > 0", what);
  if (Tn > Un) return fail(TW_EINVAL, "%s: expected T <= U after orientation", what);
  return TW_OK;
}

template <typename T>
static void jeanie_fill(JeanieArgs<T>& a, int K1, int K2, int Tn, int Un, int s1, int s2,
                        int swap, double gamma) {
  a.K1 = K1;
  a.K2 = K2;
  a.K = K1 * K2;
  a.Tn = Tn;
  a.Un = Un;
  a.s1 = s1 < K1 - 1 ? s1 : K1 - 1;
  a.s2 = s2 < K2 - 1 ? s2 : K2 - 1;
  a.swap = swap;
  a.k = (T)(1.4426950408889634 / gamma);
  a.inv_k = (T)(gamma * 0.6931471805599453);
}

template <typename T>
int jeanie_cost_fwd(const T* C, int B, int K1, int K2, int Tn, int Un, int swap, int s1, int s2,
                    double gamma, T* R, T* out, hipStream_t s, const char* what) {
  if (int e = jeanie_check<T>(what, B, K1, K2, Tn, Un, s1, s2, gamma)) return e;
  if (B == 0) return TW_OK;
  if (!C || !R || !out) return fail(TW_EINVAL, "%s: null pointer", what);
  JeanieArgs<T> a = {};
  a.C = C;
  a.Rw = R;
  a.out = out;
  jeanie_fill(a, K1, K2, Tn, Un, s1, s2, swap, gamma);
  if (j3_enabled()) {
    const int e = jeanie3_fwd<T>(a, B, s, what);
    if (e != kJ3Unsupported) return e;
  }
  const J2Shape sh = jeanie2_shape(a.K, Tn, a.s1, a.s2);
  if (sh.threads) {
    const size_t ring = (size_t)2 * sh.threads * sizeof(T);
    const size_t stage = ring + (size_t)2 * a.K * Tn * Un * sizeof(T);
    const bool st = stage <= (size_t)(64 * 1024) && stage <= (size_t)max_lds_bytes();
    const size_t lds = st ? stage : ring;
#define TW_J2F(ST_, SM_) \
  hipLaunchKernelGGL((jeanie2_fwd_kernel<T, ST_, SM_>), dim3(B), dim3(sh.threads), lds, s, a, sh.KP)
    if (st) {
      if (sh.smax == 1) TW_J2F(true, 1); else TW_J2F(true, 2);
    } else {
      if (sh.smax == 1) TW_J2F(false, 1); else TW_J2F(false, 2);
    }
#undef TW_J2F
    return check_launch(what);
  }
  const int threads = jeanie_threads(Tn * a.K);
  const size_t lds = (size_t)3 * Tn * a.K * sizeof(T);
  if (lds <= (size_t)max_lds_bytes())
    hipLaunchKernelGGL((jeanie_fwd_kernel<T, true>), dim3(B), dim3(threads), lds, s, a);
  else
    hipLaunchKernelGGL((jeanie_fwd_kernel<T, false>), dim3(B), dim3(threads), 0, s, a);
  return check_launch(what);
}

template <typename T>
int jeanie_cost_bwd(const T* C, const T* R, const T* gout, const T* gR, int B, int K1, int K2,
                    int Tn, int Un, int swap, int s1, int s2, double gamma, T* dC, hipStream_t s,
                    const char* what) {
  if (int e = jeanie_check<T>(what, B, K1, K2, Tn, Un, s1, s2, gamma)) return e;
  if (B == 0) return TW_OK;
  if (!C || !R || !gout || !dC) return fail(TW_EINVAL, "%s: null pointer", what);
  JeanieArgs<T> a = {};
  a.C = C;
  a.R = R;
  a.gout = gout;
  a.gR = gR;
  a.dC = dC;
  jeanie_fill(a, K1, K2, Tn, Un, s1, s2, swap, gamma);
  if (j3_enabled()) {
    const int e = jeanie3_bwd<T>(a, B, s, what);
    if (e != kJ3Unsupported) return e;
  }
  const J2Shape sh = jeanie2_shape(a.K, Tn, a.s1, a.s2);
  if (sh.threads) {
    const size_t ring = (size_t)4 * sh.threads * sizeof(T);
    const size_t stage = ring + (size_t)2 * a.K * Tn * Un * sizeof(T);
    const bool st = stage <= (size_t)(64 * 1024) && stage <= (size_t)max_lds_bytes();
    const size_t lds = st ? stage : ring;
#define TW_J2B(ST_, SM_) \
  hipLaunchKernelGGL((jeanie2_bwd_kernel<T, ST_, SM_>), dim3(B), dim3(sh.threads), lds, s, a, sh.KP)
    if (st) {
      if (sh.smax == 1) TW_J2B(true, 1); else TW_J2B(true, 2);
    } else {
      if (sh.smax == 1) TW_J2B(false, 1); else TW_J2B(false, 2);
    }
#undef TW_J2B
    return check_launch(what);
  }
  const int threads = jeanie_threads(Tn * a.K);
  const size_t lds = (size_t)6 * Tn * a.K * sizeof(T);
  if (lds + sizeof(T) <= (size_t)max_lds_bytes())
    hipLaunchKernelGGL((jeanie_bwd_kernel<T, true>), dim3(B), dim3(threads), lds, s, a);
  else
    hipLaunchKernelGGL((jeanie_bwd_kernel<T, false>), dim3(B), dim3(threads), 0, s, a);
  return check_launch(what);
}

// ----------------------------------------------------------------- FVM
// Viewpoint softmin at every temporal cell (jeanie/fvm.py:36-37):
//   temporal[t,u] = -g ln sum_n exp(-C[n,t,u]/g)
// written in the DP orientation ([U,T] when `swap`), and its adjoint
//   dC[n,t,u] = exp((temporal[t,u] - C[n,t,u])/g) * dtemporal[t,u].

// KU > 0: all K <= KU viewpoints of a cell are loaded at once (unrolled,
// every load in flight together); KU = 0: a loop for larger K.
template <typename T, int KU>
__global__ void __launch_bounds__(256) fvm_softmin_fwd(const T* __restrict__ C, T* __restrict__ tmp,
                                                       int K, int Tn, int Un, int swap, T k,
                                                       T inv_k) {
  // workgroup w covers cells (w % bpp) * 256 .. of pair w / bpp
  const int plane = Tn * Un, bpp = (plane + 255) / 256;
  const int b = (int)blockIdx.x / bpp;
  const int cell = ((int)blockIdx.x - b * bpp) * 256 + (int)threadIdx.x;
  if (cell >= plane) return;
  const T* c = C + (size_t)b * K * plane + cell;
  const T INF = inf_v<T>();
  T m = INF, s = 0;
  if (KU > 0) {
    T v[KU > 0 ? KU : 1];
#pragma unroll
    for (int n = 0; n < KU; ++n) v[n] = n < K ? c[(size_t)n * plane] : INF;
#pragma unroll
    for (int n = 0; n < KU; ++n) m = fmin(m, v[n]);
#pragma unroll
    for (int n = 0; n < KU; ++n) s += n < K ? ex2((m - v[n]) * k) : (T)0;
  } else {
    for (int n = 0; n < K; ++n) m = fmin(m, c[(size_t)n * plane]);
    for (int n = 0; n < K; ++n) s += ex2((m - c[(size_t)n * plane]) * k);
  }
  const int t = cell / Un, u = cell - t * Un;
  const int o = swap ? u * Tn + t : cell;
  tmp[(size_t)b * plane + o] = m - inv_k * lg2(s);
}

template <typename T, int KU>
__global__ void __launch_bounds__(256) fvm_softmin_bwd(const T* __restrict__ C,
                                                       const T* __restrict__ tmp,
                                                       const T* __restrict__ dtmp,
                                                       T* __restrict__ dC, int K, int Tn, int Un,
                                                       int swap, T k) {
  const int plane = Tn * Un, bpp = (plane + 255) / 256;
  const int b = (int)blockIdx.x / bpp;
  const int cell = ((int)blockIdx.x - b * bpp) * 256 + (int)threadIdx.x;
  if (cell >= plane) return;
  const int t = cell / Un, u = cell - t * Un;
  const int o = swap ? u * Tn + t : cell;
  const T tv = tmp[(size_t)b * plane + o], g = dtmp[(size_t)b * plane + o];
  const T* c = C + (size_t)b * K * plane + cell;
  T* dc = dC + (size_t)b * K * plane + cell;
  if (KU > 0) {
    T v[KU > 0 ? KU : 1];
#pragma unroll
    for (int n = 0; n < KU; ++n) v[n] = n < K ? c[(size_t)n * plane] : (T)0;
#pragma unroll
    for (int n = 0; n < KU; ++n)
      if (n < K) dc[(size_t)n * plane] = ex2((tv - v[n]) * k) * g;
  } else {
    for (int n = 0; n < K; ++n) dc[(size_t)n * plane] = ex2((tv - c[(size_t)n * plane]) * k) * g;
  }
}

template <typename T>
int udtw_cost_fwd_any(const T* C, const T* Q, int B, int N, int M, double gamma, double band,
                      T* R, T* P, T* out_r, T* out_p, hipStream_t s, const char* what);
template <typename T>
int udtw_cost_bwd_any(const T* C, const T* Q, const T* R, const T* P, const T* gr, const T* gp,
                      int B, int N, int M, double gamma, T* dC, T* dQ, T* ws, size_t ws_bytes,
                      hipStream_t s, const char* what);
template <typename T>
size_t udtw_cost_hand_bytes(int B, int N, int M);

// FVM backward workspace: dtemporal [B, T*U], then (8-byte aligned) the
// hand-off records of the soft-DTW backward over several workgroups per
// pair (sequences longer than one workgroup holds).
template <typename T>
static size_t fvm_ws_bytes(int B, int Tn, int Un, size_t* hand_at) {
  const size_t dt = (size_t)B * Tn * Un * sizeof(T), at = (dt + 7) & ~(size_t)7;
  const size_t hb = udtw_cost_hand_bytes<T>(B, Tn, Un);
  if (hand_at) *hand_at = at;
  return hb ? at + hb : dt;
}

template <typename T>
int fvm_fwd(const T* C, int B, int K, int Tn, int Un, double gamma, T* tmp, T* R, T* out,
            T* pen_scratch, hipStream_t s, const char* what) {
  if (B < 0 || K <= 0 || Tn <= 0 || Un <= 0 || !(gamma > 0))
    return fail(TW_EINVAL, "%s: bad arguments", what);
  if (B == 0) return TW_OK;
  if (!C || !tmp || !R || !out || !pen_scratch) return fail(TW_EINVAL, "%s: null pointer", what);
  const int swap = Tn > Un;
  const T k = (T)(1.4426950408889634 / gamma), inv_k = (T)(gamma * 0.6931471805599453);
  // pair and cell block in grid.x (any batch size)
  dim3 grid((unsigned)((long long)B * ((Tn * Un + 255) / 256)));
  if (K <= 32)
    hipLaunchKernelGGL((fvm_softmin_fwd<T, 32>), grid, dim3(256), 0, s, C, tmp, K, Tn, Un, swap,
                       k, inv_k);
  else
    hipLaunchKernelGGL((fvm_softmin_fwd<T, 0>), grid, dim3(256), 0, s, C, tmp, K, Tn, Un, swap,
                       k, inv_k);
  if (int e = check_launch(what)) return e;
  const int N = swap ? Un : Tn, M = swap ? Tn : Un;
  return udtw_cost_fwd_any<T>(tmp, nullptr, B, N, M, gamma, 0.0, R, nullptr, out, pen_scratch,
                              s, what);
}

template <typename T>
int fvm_bwd(const T* C, const T* tmp, const T* R, const T* gout, int B, int K, int Tn, int Un,
            double gamma, T* dC, T* ws, size_t ws_bytes, hipStream_t s, const char* what) {
  if (B < 0 || K <= 0 || Tn <= 0 || Un <= 0 || !(gamma > 0))
    return fail(TW_EINVAL, "%s: bad arguments", what);
  if (B == 0) return TW_OK;
  if (!C || !tmp || !R || !gout || !dC || !ws) return fail(TW_EINVAL, "%s: null pointer", what);
  const int swap = Tn > Un;
  const int N = swap ? Un : Tn, M = swap ? Tn : Un;
  size_t hand_at = 0;
  const size_t need = fvm_ws_bytes<T>(B, Tn, Un, &hand_at);
  if (ws_bytes < need) return fail(TW_ESIZE, "%s: workspace of %zu bytes needed", what, need);
  T* hand = need > hand_at ? reinterpret_cast<T*>(reinterpret_cast<char*>(ws) + hand_at) : nullptr;
  if (int e = udtw_cost_bwd_any<T>(tmp, nullptr, R, nullptr, gout, nullptr, B, N, M, gamma, ws,
                                   nullptr, hand, hand ? need - hand_at : 0, s, what))
    return e;
  const T k = (T)(1.4426950408889634 / gamma);
  // pair and cell block in grid.x (any batch size)
  dim3 grid((unsigned)((long long)B * ((Tn * Un + 255) / 256)));
  if (K <= 32)
    hipLaunchKernelGGL((fvm_softmin_bwd<T, 32>), grid, dim3(256), 0, s, C, tmp, ws, dC, K, Tn, Un,
                       swap, k);
  else
    hipLaunchKernelGGL((fvm_softmin_bwd<T, 0>), grid, dim3(256), 0, s, C, tmp, ws, dC, K, Tn, Un,
                       swap, k);
  return check_launch(what);
}

template int fvm_bwd<float>(const float*, const float*, const float*, const float*, int, int,
                            int, int, double, float*, float*, size_t, hipStream_t, const char*);
template int fvm_bwd<double>(const double*, const double*, const double*, const double*, int,
                             int, int, int, double, double*, double*, size_t, hipStream_t,
                             const char*);
size_t fvm_workspace_bytes(int B, int Tn, int Un, int es) {
  return es == 4 ? fvm_ws_bytes<float>(B, Tn, Un, nullptr)
                 : fvm_ws_bytes<double>(B, Tn, Un, nullptr);
}

// ------------------------------------------------------ JEANIE from features

template <typename T>
int pair_cost_fwd(const T* A, const T* Bm, int P, int R, int C, int D, int metric, T* out,
                  hipStream_t s, const char* what);
template <typename T>
int pair_cost_bwd(const T* A, const T* Bm, const T* cost, const T* dcost, int P, int R, int C,
                  int D, int metric, T* dA, T* dB, hipStream_t s, const char* what);

template <typename T>
int jeanie_feat_fwd(const T* q, const T* sup, int B, int K1, int K2, int Tq, int Us, int D,
                    int s1, int s2, double gamma, int metric, T* cost, T* R, T* out,
                    hipStream_t s, const char* what) {
  if (metric != 1 && metric != 2)
    return fail(TW_EINVAL, "%s: metric must be 1 (squared) or 2 (Euclidean)", what);
  if (B == 0) return TW_OK;
  if (int e = pair_cost_fwd<T>(q, sup, B, K1 * K2 * Tq, Us, D, metric, cost, s, what)) return e;
  const int swap = Tq > Us;
  return jeanie_cost_fwd<T>(cost, B, K1, K2, swap ? Us : Tq, swap ? Tq : Us, swap, s1, s2, gamma,
                            R, out, s, what);
}

template <typename T>
int jeanie_feat_bwd(const T* q, const T* sup, const T* cost, const T* R, const T* gout,
                    const T* gR, int B, int K1, int K2, int Tq, int Us, int D, int s1, int s2,
                    double gamma, int metric, T* dq, T* dsup, T* ws, hipStream_t s,
                    const char* what) {
  if (metric != 1 && metric != 2)
    return fail(TW_EINVAL, "%s: metric must be 1 (squared) or 2 (Euclidean)", what);
  if (B == 0) return TW_OK;
  if (!ws) return fail(TW_EINVAL, "%s: workspace needed", what);
  const int swap = Tq > Us;
  if (int e = jeanie_cost_bwd<T>(cost, R, gout, gR, B, K1, K2, swap ? Us : Tq, swap ? Tq : Us,
                                 swap, s1, s2, gamma, ws, s, what))
    return e;
  return pair_cost_bwd<T>(q, sup, cost, ws, B, K1 * K2 * Tq, Us, D, metric, dq, dsup, s, what);
}

}  // namespace tw

using namespace tw;

extern "C" {

int tw_jeanie_cost_fwd_f32(const float* cost, int B, int K1, int K2, int T, int U, int swap_tu,
                           int s1, int s2, float gamma, float* R, float* out, hipStream_t stream) {
  return jeanie_cost_fwd<float>(cost, B, K1, K2, T, U, swap_tu, s1, s2, gamma, R, out, stream,
                                "tw_jeanie_cost_fwd_f32");
}
int tw_jeanie_cost_fwd_f64(const double* cost, int B, int K1, int K2, int T, int U, int swap_tu,
                           int s1, int s2, double gamma, double* R, double* out,
                           hipStream_t stream) {
  return jeanie_cost_fwd<double>(cost, B, K1, K2, T, U, swap_tu, s1, s2, gamma, R, out, stream,
                                 "tw_jeanie_cost_fwd_f64");
}
int tw_jeanie_cost_bwd_f32(const float* cost, const float* R, const float* grad_out,
                           const float* grad_R, int B, int K1, int K2, int T, int U, int swap_tu,
                           int s1, int s2, float gamma, float* d_cost, hipStream_t stream) {
  return jeanie_cost_bwd<float>(cost, R, grad_out, grad_R, B, K1, K2, T, U, swap_tu, s1, s2,
                                gamma, d_cost, stream, "tw_jeanie_cost_bwd_f32");
}
int tw_jeanie_cost_bwd_f64(const double* cost, const double* R, const double* grad_out,
                           const double* grad_R, int B, int K1, int K2, int T, int U,
                           int swap_tu, int s1, int s2, double gamma, double* d_cost,
                           hipStream_t stream) {
  return jeanie_cost_bwd<double>(cost, R, grad_out, grad_R, B, K1, K2, T, U, swap_tu, s1, s2,
                                 gamma, d_cost, stream, "tw_jeanie_cost_bwd_f64");
}

int tw_jeanie_feat_fwd_f32(const float* query, const float* support, int B, int K1, int K2, int T,
                           int U, int D, int s1, int s2, float gamma, int metric, float* cost,
                           float* R, float* out, hipStream_t stream) {
  return jeanie_feat_fwd<float>(query, support, B, K1, K2, T, U, D, s1, s2, gamma, metric, cost,
                                R, out, stream, "tw_jeanie_feat_fwd_f32");
}
int tw_jeanie_feat_fwd_f64(const double* query, const double* support, int B, int K1, int K2,
                           int T, int U, int D, int s1, int s2, double gamma, int metric,
                           double* cost, double* R, double* out, hipStream_t stream) {
  return jeanie_feat_fwd<double>(query, support, B, K1, K2, T, U, D, s1, s2, gamma, metric, cost,
                                 R, out, stream, "tw_jeanie_feat_fwd_f64");
}
int tw_jeanie_feat_bwd_f32(const float* query, const float* support, const float* cost,
                           const float* R, const float* grad_out, const float* grad_R, int B,
                           int K1, int K2, int T, int U, int D, int s1, int s2, float gamma,
                           int metric, float* d_query, float* d_support, float* workspace,
                           hipStream_t stream) {
  return jeanie_feat_bwd<float>(query, support, cost, R, grad_out, grad_R, B, K1, K2, T, U, D, s1,
                                s2, gamma, metric, d_query, d_support, workspace, stream,
                                "tw_jeanie_feat_bwd_f32");
}
int tw_jeanie_feat_bwd_f64(const double* query, const double* support, const double* cost,
                           const double* R, const double* grad_out, const double* grad_R, int B,
                           int K1, int K2, int T, int U, int D, int s1, int s2, double gamma,
                           int metric, double* d_query, double* d_support, double* workspace,
                           hipStream_t stream) {
  return jeanie_feat_bwd<double>(query, support, cost, R, grad_out, grad_R, B, K1, K2, T, U, D,
                                 s1, s2, gamma, metric, d_query, d_support, workspace, stream,
                                 "tw_jeanie_feat_bwd_f64");
}

int tw_fvm_cost_fwd_f32(const float* cost, int B, int K, int T, int U, float gamma,
                        float* temporal, float* R, float* out, float* scratch,
                        hipStream_t stream) {
  return fvm_fwd<float>(cost, B, K, T, U, gamma, temporal, R, out, scratch, stream,
                        "tw_fvm_cost_fwd_f32");
}
int tw_fvm_cost_fwd_f64(const double* cost, int B, int K, int T, int U, double gamma,
                        double* temporal, double* R, double* out, double* scratch,
                        hipStream_t stream) {
  return fvm_fwd<double>(cost, B, K, T, U, gamma, temporal, R, out, scratch, stream,
                         "tw_fvm_cost_fwd_f64");
}
size_t tw_fvm_workspace_bytes(int B, int K, int T, int U, int elem_size) {
  if (B <= 0 || K <= 0 || T <= 0 || U <= 0) return 0;
  return elem_size == 4 ? fvm_ws_bytes<float>(B, T, U, nullptr)
                        : fvm_ws_bytes<double>(B, T, U, nullptr);
}

int tw_fvm_cost_bwd_f32(const float* cost, const float* temporal, const float* R,
                        const float* grad_out, int B, int K, int T, int U, float gamma,
                        float* d_cost, float* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  return fvm_bwd<float>(cost, temporal, R, grad_out, B, K, T, U, gamma, d_cost, workspace,
                        workspace_bytes, stream, "tw_fvm_cost_bwd_f32");
}
int tw_fvm_cost_bwd_f64(const double* cost, const double* temporal, const double* R,
                        const double* grad_out, int B, int K, int T, int U, double gamma,
                        double* d_cost, double* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  return fvm_bwd<double>(cost, temporal, R, grad_out, B, K, T, U, gamma, d_cost, workspace,
                         workspace_bytes, stream, "tw_fvm_cost_bwd_f64");
}

}  // extern "C"
