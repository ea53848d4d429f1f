// JEANIE temporal-viewpoint DP for gfx950 with one wavefront per pair:
// forward and backward on the cost path (reference: jeanie_cuda.cu:144-295,
// jeanie/_torch_dp.py:14-75, jeanie/functional.py:28-61).
//
// The window softmin is evaluated separably in the base-2 scaled domain
// (Rh = R log2(e)/g); a softmin over a union of disjoint sets is the softmin
// of their softmins, so with viewpoints n = n1 K2 + n2:
//   S2[n1,n2] = softmin_{|o|<=s2} R[n1, n2+o]
//   Rw[n1,n2] = softmin_{|o|<=s1} S2[n1+o, n2]
//   R[n,t,u]  = C[n,t,u] + softmin(Rw[n,t-1,u], Rw[n,t,u-1], Rw[n,t-1,u-1])
// and R[n,0,0] = C[n,0,0]. The backward runs the three stages in reverse
// (successor weights -> RWbar -> S2bar -> Rbar), recomputing S2 and Rw from R.
//
// Mapping. A wavefront owns one pair and walks it in row pairs: its 32-lane
// halves own rows t = 2r and 2r + 1, lane n of a half owns viewpoint n
// (K <= 32). At step v of a row pair, half h computes column u = v - h, one
// column behind the other half (U + 1 steps per row pair). Per cell:
//  * the window softmins gather neighbouring viewpoints of the same cell:
//    stride 1 by DPP wave shifts, stride K2 by DPP row shifts joined across
//    16-lane rows by v_permlane16_swap (K2 = 5; other strides by
//    ds_bpermute);
//  * the temporal predecessors are Rw values of the lane's own viewpoint:
//    "left" is its own last step; half 1's "up" is half 0's last step, handed
//    over by v_permlane32_swap at the end of every step; half 0's "up" is the
//    row above the pair, which half 1 produced during the previous row pair:
//    half 0 receives it in the same swap and keeps it, by column, in a
//    register array until the next row pair reads it;
//  * the cost (and in the backward R and dL/dR) of a row pair is loaded into
//    a register ring during the previous row pair, and each result is
//    stored as soon as it is known.
// Nothing crosses wavefronts and nothing goes through the LDS. The backward
// runs the same sweep on the grid flipped in t and u, so its "predecessors"
// are the cell's successors. The padded-lane variants below (windows of one
// neighbour each way) drop the per-neighbour masks.
//
// Work per pair: ceil(T/2) (U + 1) steps of one cell per lane, against
// T + U - 1 diagonal steps of the workgroup-per-pair kernels (jeanie_dp.hip)
// that keep a lane per (t, n) busy only while row t is on the diagonal.

#include "jeanie.hpp"

namespace tw {


__device__ __forceinline__ float med3(float a, float b, float c) {
  return __builtin_amdgcn_fmed3f(a, b, c);
}
__device__ __forceinline__ double med3(double a, double b, double c) {
  return fmax(fmin(a, b), fmin(fmax(a, b), c));
}

// base-2 softmin of three values: the smallest one contributes exp2(0) = 1
template <typename T>
__device__ __forceinline__ T softmin3h(T a, T b, T c) {
  const T m = fmin(a, fmin(b, c));
  const T md = med3(a, b, c);
  const T mx = fmax(a, fmax(b, c));
  return m - lg2((T)1 + ex2(m - md) + ex2(m - mx));
}

// lane l + o (|o| <= 2) of v along the stride-1 viewpoint axis (DPP wave shifts)
template <typename T>
__device__ __forceinline__ T nb1(T v, int o) {
  const T INF = inf_v<T>();
  if (o == -1) return shift_prev(v, INF);
  if (o == 1) return shift_next(v, INF);
  if (o == -2) return shift_prev(shift_prev(v, INF), INF);
  return shift_next(shift_next(v, INF), INF);
}

// the value of lane idx/4 (ds_bpermute byte index)
__device__ __forceinline__ float bperm(float v, int idx) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(idx, __float_as_int(v)));
}
__device__ __forceinline__ double bperm(double v, int idx) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_ds_bpermute(idx, (int)b);
  const int hi = __builtin_amdgcn_ds_bpermute(idx, (int)(b >> 32));
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// The value of lane l - K / l + K (0 < K < 16) within each 32-lane half,
// without the LDS: a DPP row shift serves the lanes whose source lies in their
// own 16-lane row, and the rest take a row shift by 16 - K of the
// neighbouring row, moved across by v_permlane16_swap. Lanes whose source is
// outside their half get an unspecified value (the window masks them).
template <int K>
__device__ __forceinline__ unsigned lane_minus(unsigned v) {
  static_assert(K > 0 && K < 16, "row shifts reach 15 lanes");
  const unsigned a = __builtin_amdgcn_update_dpp(0u, v, 0x110 + K, 0xf, 0xf, false);       // row_shr:K
  const unsigned b = __builtin_amdgcn_update_dpp(0u, v, 0x100 + 16 - K, 0xf, 0xf, false);  // row_shl:16-K
  const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);  // r[0]: odd rows <- even rows
  return (__lane_id() & 15) >= K ? a : r[0];
}
template <int K>
__device__ __forceinline__ unsigned lane_plus(unsigned v) {
  static_assert(K > 0 && K < 16, "row shifts reach 15 lanes");
  const unsigned a = __builtin_amdgcn_update_dpp(0u, v, 0x100 + K, 0xf, 0xf, false);       // row_shl:K
  const unsigned c = __builtin_amdgcn_update_dpp(0u, v, 0x110 + 16 - K, 0xf, 0xf, false);  // row_shr:16-K
  const auto r = __builtin_amdgcn_permlane16_swap(c, c, false, false);  // r[1]: even rows <- odd rows
  return (__lane_id() & 15) < 16 - K ? a : r[1];
}
template <int K>
__device__ __forceinline__ float lane_shift(float v, bool up) {
  const unsigned x = __float_as_uint(v);
  return __uint_as_float(up ? lane_plus<K>(x) : lane_minus<K>(x));
}
template <int K>
__device__ __forceinline__ double lane_shift(double v, bool up) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const unsigned lo = (unsigned)b, hi = (unsigned)(b >> 32);
  const unsigned rl = up ? lane_plus<K>(lo) : lane_minus<K>(lo);
  const unsigned rh = up ? lane_plus<K>(hi) : lane_minus<K>(hi);
  return __longlong_as_double((long long)(((unsigned long long)rh << 32) | rl));
}

// Neighbour o (|o| <= 2) along viewpoint axis 1, whose stride is K2: with a
// compile-time stride KS (1: DPP wave shifts; 2..7: lane_shift), else by
// ds_bpermute with the lane's precomputed byte index.
template <typename T, int KS>
__device__ __forceinline__ T nbk(T v, int o, int idx) {
  if constexpr (KS == 1) {
    return nb1(v, o);
  } else if constexpr (KS > 1) {
    static_assert(2 * KS < 16, "two strides within a row shift");
    if (o == -1) return lane_shift<KS>(v, false);
    if (o == 1) return lane_shift<KS>(v, true);
    if (o == -2) return lane_shift<2 * KS>(v, false);
    return lane_shift<2 * KS>(v, true);
  } else {
    return bperm(v, idx);
  }
}

// The halves of a wavefront exchanged: lanes 0-31 take lanes 32-63 and back
// (v_permlane32_swap of a register with itself).
__device__ __forceinline__ float swap_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(__lane_id() < 32 ? r[1] : r[0]);
}
__device__ __forceinline__ double swap_halves(double v) {
  const long long b = __double_as_longlong(v);
  const unsigned lo = (unsigned)b, hi = (unsigned)(b >> 32);
  const auto rl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
  const auto rh = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
  const bool low = __lane_id() < 32;
  const unsigned long long l = low ? rl[1] : rl[0], h = low ? rh[1] : rh[0];
  return __longlong_as_double((long long)((h << 32) | l));
}

// Per-lane window of a viewpoint: which neighbours o = -2..2 exist along each
// axis, and the ds_bpermute byte indices of the stride-K2 neighbours.
struct J3Win {
  bool a1[5], a2[5];   // axis 1 (stride K2) / axis 2 (stride 1) neighbour o - 2 in the window
  int idx1[5];
  __device__ void init(int lane, int n1, int n2, int K1, int K2, int s1, int s2) {
#pragma unroll
    for (int q = 0; q < 5; ++q) {
      const int o = q - 2;
      a1[q] = (o >= -s1 && o <= s1 && n1 + o >= 0 && n1 + o < K1);
      a2[q] = (o >= -s2 && o <= s2 && n2 + o >= 0 && n2 + o < K2);
      idx1[q] = ((lane + o * K2) & 63) << 2;
    }
  }
};

// softmin over the window of axis 2 (stride 1), then of axis 1 (stride K2)
// (Cross-lane moves run in every lane and are masked afterwards: a lane that
// skipped one would hand its neighbour a stale value.)
template <typename T, int SMAX>
__device__ __forceinline__ T win2(T v, const J3Win& w, int s2) {
  const T INF = inf_v<T>();
  if (s2 == 0) return v;
  if (SMAX == 1) {
    const T lo = nb1(v, -1), hi = nb1(v, 1);
    return softmin3h(w.a2[1] ? lo : INF, v, w.a2[3] ? hi : INF);
  }
  T x[5];
#pragma unroll
  for (int q = 0; q < 5; ++q) x[q] = q == 2 ? v : nb1(v, q - 2);
  T m = INF;
#pragma unroll
  for (int q = 0; q < 5; ++q) {
    x[q] = (q == 2 || w.a2[q]) ? x[q] : INF;
    m = fmin(m, x[q]);
  }
  T s = 0;
#pragma unroll
  for (int q = 0; q < 5; ++q) s += ex2(m - x[q]);
  return m - lg2(s);
}
template <typename T, int SMAX, int KS>
__device__ __forceinline__ T win1(T v, const J3Win& w, int s1) {
  const T INF = inf_v<T>();
  if (s1 == 0) return v;
  if (SMAX == 1) {
    const T lo = nbk<T, KS>(v, -1, w.idx1[1]), hi = nbk<T, KS>(v, 1, w.idx1[3]);
    return softmin3h(w.a1[1] ? lo : INF, v, w.a1[3] ? hi : INF);
  }
  T x[5];
#pragma unroll
  for (int q = 0; q < 5; ++q) x[q] = q == 2 ? v : nbk<T, KS>(v, q - 2, w.idx1[q]);
  T m = INF;
#pragma unroll
  for (int q = 0; q < 5; ++q) {
    x[q] = (q == 2 || w.a1[q]) ? x[q] : INF;
    m = fmin(m, x[q]);
  }
  T s = 0;
#pragma unroll
  for (int q = 0; q < 5; ++q) s += ex2(m - x[q]);
  return m - lg2(s);
}

// Adjoints of the window stages: sum over the window's neighbours q of
// g[q] 2^(hq[q] - x) (the window is symmetric, so the lanes whose window holds
// this lane are its window neighbours).
template <typename T, int SMAX, int KS>
__device__ __forceinline__ T win1_adj(T g, T hq, T x, const J3Win& w, int s1) {
  if (s1 == 0) return g;
  T acc = g * ex2(hq - x);
#pragma unroll
  for (int q = 0; q < 5; ++q) {
    if (q == 2 || (SMAX == 1 && (q == 0 || q == 4))) continue;
    const T gq = nbk<T, KS>(g, q - 2, w.idx1[q]), hh = nbk<T, KS>(hq, q - 2, w.idx1[q]);
    acc += w.a1[q] ? gq * ex2(hh - x) : (T)0;
  }
  return acc;
}
template <typename T, int SMAX>
__device__ __forceinline__ T win2_adj(T g, T hq, T x, const J3Win& w, int s2) {
  if (s2 == 0) return g;
  T acc = g * ex2(hq - x);
#pragma unroll
  for (int q = 0; q < 5; ++q) {
    if (q == 2 || (SMAX == 1 && (q == 0 || q == 4))) continue;
    const T gq = nb1(g, q - 2), hh = nb1(hq, q - 2);
    acc += w.a2[q] ? gq * ex2(hh - x) : (T)0;
  }
  return acc;
}

// Lane geometry of the sweep. Row pair r puts half h on row 2r + h, and step
// v of the row pair on column v - h (of the grid flipped in t and u for the
// backward). UC >= U is the compile-time row length: a row pair takes UC + 1
// steps, so the steps of a row pair unroll with constant columns; columns
// >= U lie outside the grid.
template <typename T>
struct J3Lane {
  int lb, ts, us, rlim, Un, h;
  bool vn, flip;
  __device__ void init(int n, int h_, const JeanieArgs<T>& a, bool flip_) {
    const int es = (int)sizeof(T);
    h = h_;
    Un = a.Un;
    flip = flip_;
    vn = n < a.K;
    ts = (a.swap ? 1 : a.Un) * es;
    us = (a.swap ? a.Tn : 1) * es;
    rlim = (a.Tn - h + 1) >> 1;   // row pairs whose row 2r + h < T
    const int pl = n * a.Tn * a.Un * es;
    // byte offset of the cell at step 0 of row pair 0
    lb = flip ? pl + (a.Tn - 1 - h) * ts + (a.Un - 1 + h) * us : pl + h * (ts - us);
  }
  // byte offset of column 0 of row pair r (or kOob when the lane's row is outside)
  __device__ __forceinline__ int base(int r) const {
    return (vn && r < rlim) ? (flip ? lb - 2 * r * ts : lb + 2 * r * ts) : kOob;
  }
  // this lane's cell at step v is inside the grid (given its row is)
  __device__ __forceinline__ bool col_ok(int v) const {
    return h == 0 ? v < Un : (v >= 1 && v <= Un);
  }
  // byte offset of the cell at step v from the row pair's base (kOob stays kOob)
  __device__ __forceinline__ int at(int vb, int v) const {
    return vb == kOob ? kOob : (flip ? vb - v * us : vb + v * us);
  }
};

template <typename T, int SMAX, int UC, int KS>
__global__ void __launch_bounds__(64) jeanie3_fwd_kernel(JeanieArgs<T> a) {
  constexpr int SPR = UC + 1;
  const int b = blockIdx.x;
  const int lane = threadIdx.x, h = lane >> 5, n = lane & 31;
  const int K = a.K, Tn = a.Tn, Un = a.Un;
  const bool vn = n < K;
  const int n1 = vn ? n / a.K2 : 0, n2 = vn ? n - n1 * a.K2 : 0;
  const T INF = inf_v<T>();
  const int plane = Tn * Un, nrp = (Tn + 1) / 2, hl = (Tn - 1) & 1;

  J3Win w;
  w.init(lane, n1, n2, a.K1, a.K2, a.s1, a.s2);
  J3Lane<T> g;
  g.init(n, h, a, false);
  Buf bC, bR;
  bC.init(a.C + (size_t)b * K * plane, (long long)K * plane);
  bR.init(a.Rw + (size_t)b * K * plane, (long long)K * plane);

  // Rw of the row above a row pair, by column, in registers (half 0 reads
  // column v + 1 at step v before it overwrites column v - 1 with the row
  // below, which half 1 produced a step earlier; entries of columns >= U stay
  // +inf). Half 1 keeps a copy it never reads.
  T ub[SPR];
#pragma unroll
  for (int v = 0; v < SPR; ++v) ub[v] = INF;

  // register ring: the cost of one row pair, loaded during the previous one
  T cr[SPR];
  {
    const int vb = g.base(0);
#pragma unroll
    for (int v = 0; v < SPR; ++v) cr[v] = bC.ld<T>(g.at(vb, v), 0);
  }
  T left = INF, pup = INF, xch = INF, lup = INF, rlast = INF;
  for (int r = 0; r < nrp; ++r) {
    const int vb = g.base(r), vbn = g.base(r + 1);
#pragma unroll
    for (int v = 0; v < SPR; ++v) {
      const bool valid = vb != kOob && g.col_ok(v);
      const T ch = cr[v] * a.k;
      // temporal predecessors: up (t-1, u), left (t, u-1), diagonal (t-1, u-1)
      const T up = h ? xch : lup;
      const T dg = v == 0 ? ((r == 0 && h == 0) ? (T)0 : INF) : pup;
      lup = ub[v < UC ? v + 1 : 0];   // half 0's next "up"
      T rh = ch + softmin3h(up, left, dg);
      rh = valid ? rh : INF;
      const T s2h = win2<T, SMAX>(rh, w, a.s2);
      T rw = win1<T, SMAX, KS>(s2h, w, a.s1);
      rw = valid ? rw : INF;
      bR.st(rh * a.inv_k, valid ? g.at(vb, v) : kOob, 0);
      if (r == nrp - 1 && v == Un - 1 + hl) rlast = rh;   // cell (T-1, U-1) in half hl
      left = rw;
      pup = up;
      xch = swap_halves(rw);
      // half 0 keeps the row below it (half 1's Rw at column v - 1) for the next row pair
      if (v >= 1) ub[v - 1] = xch;
      cr[v] = bC.ld<T>(g.at(vbn, v), 0);
    }
  }
  // out = softmin over the viewpoints of R[., T-1, U-1] (half hl holds the cell)
  T m = vn ? rlast : INF;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) m = fmin(m, __shfl_xor(m, o));
  T s = (vn && m < INF) ? ex2(m - rlast) : (T)0;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o);
  if (h == hl && n == 0) a.out[b] = (m - lg2(s)) * a.inv_k;
}

template <typename T>
struct alignas(2 * sizeof(T)) FG {
  T f, g;   // F = Rh - Ch and G = Rbar of a cell
};

// PS: dC in aligned pairs of row neighbours: the pair of steps v - 1 and v
// at step v (half 0: v odd, half 1: v even, v >= 2).
template <typename T, int SMAX, int UC, int KS, bool PS>
__global__ void __launch_bounds__(64) jeanie3_bwd_kernel(JeanieArgs<T> a) {
  constexpr int SPR = UC + 1;
  const int b = blockIdx.x;
  const int lane = threadIdx.x, h = lane >> 5, n = lane & 31;
  const int K = a.K, Tn = a.Tn, Un = a.Un;
  const bool vn = n < K;
  const int n1 = vn ? n / a.K2 : 0, n2 = vn ? n - n1 * a.K2 : 0;
  const T INF = inf_v<T>();
  const int plane = Tn * Un, nrp = (Tn + 1) / 2;
  const T gout = a.gout[b];
  const bool has_gr = a.gR != nullptr;

  J3Win w;
  w.init(lane, n1, n2, a.K1, a.K2, a.s1, a.s2);
  J3Lane<T> g;
  g.init(n, h, a, true);
  const size_t pb = (size_t)b * K * plane;
  Buf bC, bR, bG, bD;
  bC.init(a.C + pb, (long long)K * plane);
  bR.init(a.R + pb, (long long)K * plane);
  bG.init(has_gr ? a.gR + pb : a.C, has_gr ? (long long)K * plane : 0);   // empty: loads read 0
  bD.init(a.dC + pb, (long long)K * plane);

  // (F, G) of the row below a row pair (the row above in the flipped grid;
  // columns >= U stay (-inf, 0)), by column, in registers, as in the forward
  FG<T> ub[SPR];
#pragma unroll
  for (int v = 0; v < SPR; ++v) ub[v] = {-INF, (T)0};

  T rr[SPR], rc[SPR], rg[SPR];
  {
    const int vb = g.base(0);
#pragma unroll
    for (int v = 0; v < SPR; ++v) {
      const int o = g.at(vb, v);
      rr[v] = bR.ld<T>(o, 0);
      rc[v] = bC.ld<T>(o, 0);
      rg[v] = bG.ld<T>(o, 0);
    }
  }
  const FG<T> none = {-INF, (T)0};
  FG<T> left = none, pup = none, xch = none, lup = none;
  for (int r = 0; r < nrp; ++r) {
    const int vb = g.base(r), vbn = g.base(r + 1);
#pragma unroll
    for (int v = 0; v < SPR; ++v) {
      const bool valid = vb != kOob && g.col_ok(v);
      const T rh = valid ? rr[v] * a.k : INF;
      const T ch = rc[v] * a.k;
      // successors (t+1, u), (t, u+1), (t+1, u+1) of the cell
      const FG<T> up = h ? xch : lup;
      const FG<T> dg = v == 0 ? none : pup;
      lup = ub[v < UC ? v + 1 : 0];
      const T s2h = win2<T, SMAX>(rh, w, a.s2);
      const T rwh = win1<T, SMAX, KS>(s2h, w, a.s1);
      T wbar = up.g * ex2(up.f - rwh) + left.g * ex2(left.f - rwh) + dg.g * ex2(dg.f - rwh);
      wbar = valid ? wbar : (T)0;
      const T s2bar = win1_adj<T, SMAX, KS>(wbar, valid ? rwh : (T)0, s2h, w, a.s1);
      T rbar = win2_adj<T, SMAX>(valid ? s2bar : (T)0, valid ? s2h : (T)0, rh, w, a.s2);
      if (v == 0 && r == 0) {
        // the last cell (T-1, U-1) (half 0): seed with grad_out * softmax_n(-R/g)
        T m = valid ? rh : INF;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) m = fmin(m, __shfl_xor(m, o));
        T s = valid ? ex2(m - rh) : (T)0;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o);
        rbar += gout * ex2(m - lg2(s) - rh);
      }
      if (has_gr) rbar += rg[v];
      rbar = valid ? rbar : (T)0;
      const FG<T> cur = {valid ? rh - ch : -INF, rbar};
      if constexpr (PS) {
        const bool pair = ((h + v) & 1) && v >= 1 + h;
        st_pair<T>(bD, (valid && pair) ? g.at(vb, v) : kOob, rbar, left.g);
      } else {
        bD.st(rbar, valid ? g.at(vb, v) : kOob, 0);
      }
      left = cur;
      pup = up;
      xch = {swap_halves(cur.f), swap_halves(cur.g)};
      if (v >= 1) ub[v - 1] = xch;
      const int o = g.at(vbn, v);
      rr[v] = bR.ld<T>(o, 0);
      rc[v] = bC.ld<T>(o, 0);
      rg[v] = bG.ld<T>(o, 0);
    }
  }
}

// ------------------------------------------------- padded-lane kernels
//
// For windows of at most one viewpoint each way (s1, s2 <= 1) the lanes of a
// half hold the viewpoints with one unused lane after each axis-2 row
// (lane n1 P + n2, P = K2 + s2, K1 P < 32). Every window neighbour a cell
// has then sits in its own viewpoint row or in an unused lane, and the
// kernels need no per-neighbour masks:
//  * in the forward direction cells outside the grid, and unused lanes, hold
//    the finite sentinel BIG = 2^100 (scaled domain) both before and after
//    the axis-2 window: 2^(x - BIG) underflows
//    to exactly 0 for every value x a cell in the grid takes, so a softmin
//    with such neighbours equals the softmin without them, and a softmin of
//    sentinels stays finite (no inf - inf);
//  * in the adjoint direction they hold a zero adjoint, so their terms
//    vanish;
//  * lanes shifted in from outside a 32-lane half receive BIG (values) or 0
//    (adjoints) from the shift itself (DPP old value / bound_ctrl fill, and
//    v_permlane16_swap against a fill register).
// The arithmetic of a cell is that of the general kernels above.

template <typename T>
__device__ __forceinline__ T big_v() {
  return (T)0x1p100;
}

// Lane l - 1 / l + 1 across the wavefront (DPP wave shifts); the lane without
// a source takes `fill`, or 0 for the zero-filled form.
__device__ __forceinline__ unsigned wsh(unsigned v, bool up, unsigned fill) {
  return up ? __builtin_amdgcn_update_dpp(fill, v, 0x130, 0xf, 0xf, false)    // wave_shl:1
            : __builtin_amdgcn_update_dpp(fill, v, 0x138, 0xf, 0xf, false);   // wave_shr:1
}
__device__ __forceinline__ unsigned wsh0(unsigned v, bool up) {
  return up ? __builtin_amdgcn_update_dpp(0u, v, 0x130, 0xf, 0xf, true)
            : __builtin_amdgcn_update_dpp(0u, v, 0x138, 0xf, 0xf, true);
}
// Lane l - K / l + K (0 < K < 16) within each 32-lane half: a DPP row shift for
// the lanes whose source is in their own 16-lane row, whose old value is
// the complementary row shift of the neighbouring row, brought over by
// v_permlane16_swap against a register of `fill` (which the lanes whose
// source lies outside the half keep).
template <int K>
__device__ __forceinline__ unsigned rsh(unsigned v, bool up, unsigned fill) {
  static_assert(K > 0 && K < 16, "row shifts reach 15 lanes");
  if (up) {
    const unsigned c = __builtin_amdgcn_update_dpp(0u, v, 0x110 + 16 - K, 0xf, 0xf, true);
    const auto r = __builtin_amdgcn_permlane16_swap(c, fill, false, false);
    // r[1]: rows 0, 2 <- rows 1, 3 of c; rows 1, 3 keep fill
    return __builtin_amdgcn_update_dpp(r[1], v, 0x100 + K, 0xf, 0xf, false);   // row_shl:K
  }
  const unsigned b = __builtin_amdgcn_update_dpp(0u, v, 0x100 + 16 - K, 0xf, 0xf, true);
  const auto r = __builtin_amdgcn_permlane16_swap(fill, b, false, false);
  // r[0]: rows 1, 3 <- rows 0, 2 of b; rows 0, 2 keep fill
  return __builtin_amdgcn_update_dpp(r[0], v, 0x110 + K, 0xf, 0xf, false);     // row_shr:K
}

// Neighbour across an axis in the padded layout: stride 1 (axis 2, or axis 1
// when P = 1) or P (axis 1), with the fill of a value (BIG) or of an adjoint
// (0).
template <int STRIDE>
__device__ __forceinline__ unsigned pshift(unsigned v, bool up, unsigned fill, bool zero) {
  if constexpr (STRIDE == 1) return zero ? wsh0(v, up) : wsh(v, up, fill);
  else return rsh<STRIDE>(v, up, zero ? 0u : fill);
}
template <int STRIDE>
__device__ __forceinline__ float pnb(float v, bool up, bool zero) {
  const unsigned f = __float_as_uint(big_v<float>());
  return __uint_as_float(pshift<STRIDE>(__float_as_uint(v), up, f, zero));
}
template <int STRIDE>
__device__ __forceinline__ double pnb(double v, bool up, bool zero) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const unsigned long long f = (unsigned long long)__double_as_longlong(big_v<double>());
  const unsigned lo = pshift<STRIDE>((unsigned)b, up, (unsigned)f, zero);
  const unsigned hi = pshift<STRIDE>((unsigned)(b >> 32), up, (unsigned)(f >> 32), zero);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// softmin of the window of one neighbour each way (values; no masks)
template <int STRIDE, typename T>
__device__ __forceinline__ T pwin(T v) {
  return softmin3h(pnb<STRIDE>(v, false, false), v, pnb<STRIDE>(v, true, false));
}
// its adjoint: g 2^(hq - x) summed over the window's lanes (adjoints; no masks)
template <int STRIDE, typename T>
__device__ __forceinline__ T pwin_adj(T g, T hq, T x) {
  const T gl = pnb<STRIDE>(g, false, true), hl = pnb<STRIDE>(hq, false, true);
  const T gr = pnb<STRIDE>(g, true, true), hr = pnb<STRIDE>(hq, true, true);
  return g * ex2(hq - x) + gl * ex2(hl - x) + gr * ex2(hr - x);
}

// Viewpoint of a lane of a half in the padded layout, and whether it is one.
__device__ __forceinline__ int pview(int n, int P, int K1, int K2, bool* ok) {
  const int n1 = n / P, n2 = n - n1 * P;
  *ok = n1 < K1 && n2 < K2;
  return *ok ? n1 * K2 + n2 : 0;
}

// A lane's row of UC elements at byte offset o (kOob: zeros) into registers,
// in column order, by 16-byte loads.
template <typename T, int UC>
__device__ __forceinline__ void j3_ld_row(const Buf& b, int o, T (&x)[UC]) {
  constexpr int EV = 16 / (int)sizeof(T);
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int q = 0; q < UC / EV; ++q) {
    const u4 w = __builtin_amdgcn_raw_buffer_load_b128(b.r, o == kOob ? kOob : o + 16 * q, 0, 0);
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[q * 4 + e] = __uint_as_float(w[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 2; ++e)
        x[q * 2 + e] =
            __longlong_as_double((long long)(((unsigned long long)w[2 * e + 1] << 32) | w[2 * e]));
    }
  }
}

// A lane's row of UC elements (column order) stored at byte offset o (kOob:
// dropped) by 16-byte stores.
template <typename T, int UC>
__device__ __forceinline__ void j3_st_row(const Buf& b, int o, const T (&x)[UC]) {
  constexpr int EV = 16 / (int)sizeof(T);
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int q = 0; q < UC / EV; ++q) {
    u4 w;
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = __float_as_uint(x[q * 4 + e]);
    } else {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const unsigned long long z = (unsigned long long)__double_as_longlong(x[q * 2 + e]);
        w[2 * e] = (unsigned)z;
        w[2 * e + 1] = (unsigned)(z >> 32);
      }
    }
    __builtin_amdgcn_raw_buffer_store_b128(w, b.r, o == kOob ? kOob : o + 16 * q, 0, 0);
  }
}

// x0 on half 0's lanes, x1 on half 1's, as a select (the empty asm keeps a
// select of two register-array entries whose indices differ by the half
// from being folded into a run-time index into the array).
template <typename T>
__device__ __forceinline__ T j3_by_half(int h, T x0, T x1) {
  asm volatile("" : "+v"(x0), "+v"(x1));
  return h ? x1 : x0;
}

// RS: rows of exactly UC columns (U = UC), not transposed, R 16-byte
// aligned: each lane keeps its row of R through the row pair and stores it
// whole at the end in 16-byte pieces (a quarter of the store instructions;
// the halves' adjacent rows fill whole cache lines).
template <typename T, int UC, int P, bool RS>
__global__ void __launch_bounds__(64) jeanie3p_fwd_kernel(JeanieArgs<T> a) {
  constexpr int SPR = UC + 1;
  const int b = blockIdx.x;
  const int lane = threadIdx.x, h = lane >> 5;
  const int Tn = a.Tn, Un = a.Un, K = a.K;
  bool vn;
  const int n = pview(lane & 31, P, a.K1, a.K2, &vn);
  const T BIG = big_v<T>(), INF = inf_v<T>();
  const int plane = Tn * Un, nrp = (Tn + 1) / 2, hl = (Tn - 1) & 1;
  const bool w1 = a.s1 > 0, w2 = a.s2 > 0;

  J3Lane<T> g;
  g.init(n, h, a, false);
  g.vn = vn;
  Buf bC, bR;
  bC.init(a.C + (size_t)b * K * plane, (long long)K * plane);
  bR.init(a.Rw + (size_t)b * K * plane, (long long)K * plane);

  T ub[SPR];
#pragma unroll
  for (int v = 0; v < SPR; ++v) ub[v] = BIG;
  // cost of the row pair by step: RS loads the next row pair's rows whole
  // (column u is step u + h) at the start of each row pair, else one
  // element per step
  T cr[SPR], cnext[UC];
  auto c_steps = [&](const T (&row)[UC]) {
#pragma unroll
    for (int v = 0; v < SPR; ++v)
      cr[v] = j3_by_half(h, row[v < UC ? v : 0], row[v > 0 ? v - 1 : 0]);
  };
  if constexpr (RS) {
    const int vb = g.base(0);
    j3_ld_row<T, UC>(bC, vb == kOob ? kOob : g.at(vb, h), cnext);
    c_steps(cnext);
  } else {
    const int vb = g.base(0);
#pragma unroll
    for (int v = 0; v < SPR; ++v) cr[v] = bC.ld<T>(g.at(vb, v), 0);
  }
  T left = BIG, pup = BIG, xch = BIG, lup = BIG, rlast = BIG;
  T rrow[SPR];   // RS: the row pair's R, by step
  for (int r = 0; r < nrp; ++r) {
    const int vb = g.base(r), vbn = g.base(r + 1);
    if constexpr (RS) j3_ld_row<T, UC>(bC, vbn == kOob ? kOob : g.at(vbn, h), cnext);
#pragma unroll
    for (int v = 0; v < SPR; ++v) {
      const bool valid = vb != kOob && g.col_ok(v);
      const T ch = cr[v] * a.k;
      const T up = h ? xch : lup;
      const T dg = v == 0 ? ((r == 0 && h == 0) ? (T)0 : BIG) : pup;
      lup = ub[v < UC ? v + 1 : 0];
      T rh = ch + softmin3h(up, left, dg);
      rh = valid ? rh : BIG;
      // (the stride-1 shifts cross between the halves: unused lane 31 would
      // take lane 32's value into its window, and axis 1 reads lane 31)
      const T s2h = w2 ? (valid ? pwin<1>(rh) : BIG) : rh;
      const T rw = w1 ? pwin<P>(s2h) : s2h;
      if constexpr (RS)
        rrow[v] = rh * a.inv_k;
      else
        bR.st(rh * a.inv_k, valid ? g.at(vb, v) : kOob, 0);
      if (r == nrp - 1 && v == Un - 1 + hl) rlast = rh;
      left = rw;
      pup = up;
      xch = swap_halves(rw);
      if (v >= 1) ub[v - 1] = xch;
      if constexpr (!RS) cr[v] = bC.ld<T>(g.at(vbn, v), 0);
    }
    if constexpr (RS) {
      c_steps(cnext);
      // column u was step u + h
      constexpr int EV = 16 / (int)sizeof(T);
      typedef unsigned int u4 __attribute__((ext_vector_type(4)));
      const int o0 = vb == kOob ? kOob : g.at(vb, h);
#pragma unroll
      for (int q = 0; q < UC / EV; ++q) {
        T x[EV];
#pragma unroll
        for (int e = 0; e < EV; ++e) {
          // (kept a select: folded into an index h + const it would become a
          // run-time index into rrow)
          const int u = q * EV + e;
          T x0 = rrow[u], x1 = rrow[u + 1];
          asm volatile("" : "+v"(x0), "+v"(x1));
          x[e] = h ? x1 : x0;
        }
        u4 w;
        if constexpr (sizeof(T) == 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = __float_as_uint(x[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const unsigned long long z = (unsigned long long)__double_as_longlong(x[e]);
            w[2 * e] = (unsigned)z;
            w[2 * e + 1] = (unsigned)(z >> 32);
          }
        }
        __builtin_amdgcn_raw_buffer_store_b128(w, bR.r, o0 == kOob ? kOob : o0 + 16 * q, 0, 0);
      }
    }
  }
  T m = vn ? rlast : INF;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) m = fmin(m, __shfl_xor(m, o));
  T s = (vn && m < INF) ? ex2(m - rlast) : (T)0;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o);
  if (h == hl && lane % 32 == 0) a.out[b] = (m - lg2(s)) * a.inv_k;
}

// PS: rows of exactly UC columns (U = UC), not transposed, dC 16-byte
// aligned: each lane keeps its row's dC in registers through the row pair
// and stores the whole row at its end in 16-byte pieces. The halves' rows
// 2r and 2r + 1 are adjacent, so a store instruction writes whole cache
// lines (scattered single or pair stores, each a few bytes of a line, had
// cost about 30% more HBM writes than dC's bytes).
template <typename T, int UC, int P, bool PS>
__global__ void __launch_bounds__(64) jeanie3p_bwd_kernel(JeanieArgs<T> a) {
  constexpr int SPR = UC + 1;
  const int b = blockIdx.x;
  const int lane = threadIdx.x, h = lane >> 5;
  const int Tn = a.Tn, K = a.K;
  bool vn;
  const int n = pview(lane & 31, P, a.K1, a.K2, &vn);
  const T BIG = big_v<T>(), INF = inf_v<T>();
  const int plane = Tn * a.Un, nrp = (Tn + 1) / 2;
  const T gout = a.gout[b];
  const bool has_gr = a.gR != nullptr;
  const bool w1 = a.s1 > 0, w2 = a.s2 > 0;

  J3Lane<T> g;
  g.init(n, h, a, true);
  g.vn = vn;
  const size_t pb = (size_t)b * K * plane;
  Buf bC, bR, bG, bD;
  bC.init(a.C + pb, (long long)K * plane);
  bR.init(a.R + pb, (long long)K * plane);
  bG.init(has_gr ? a.gR + pb : a.C, has_gr ? (long long)K * plane : 0);
  bD.init(a.dC + pb, (long long)K * plane);

  const FG<T> none = {-INF, (T)0};
  FG<T> ub[SPR];
#pragma unroll
  for (int v = 0; v < SPR; ++v) ub[v] = none;
  // R, C (and grad_R) of the row pair by step: PS loads the next row pair's
  // rows whole (column u is step UC - 1 + h - u) at the start of each row
  // pair, else one element per step
  T rr[SPR], rc[SPR], rg[SPR], nR[UC], nC[UC], nG[UC];
  auto to_steps = [&](const T (&row)[UC], T (&st)[SPR]) {
#pragma unroll
    for (int v = 0; v < SPR; ++v)
      st[v] = j3_by_half(h, row[v < UC ? UC - 1 - v : 0], row[v > 0 ? UC - v : 0]);
  };
  auto ld_rows = [&](int vbr) {
    const int o = vbr == kOob ? kOob : g.at(vbr, UC - 1 + h);
    j3_ld_row<T, UC>(bR, o, nR);
    j3_ld_row<T, UC>(bC, o, nC);
    if (has_gr) j3_ld_row<T, UC>(bG, o, nG);
  };
  auto rows_to_steps = [&]() {
    to_steps(nR, rr);
    to_steps(nC, rc);
    if (has_gr) to_steps(nG, rg);
  };
  if constexpr (PS) {
#pragma unroll
    for (int v = 0; v < SPR; ++v) rg[v] = (T)0;
    ld_rows(g.base(0));
    rows_to_steps();
  } else {
    const int vb = g.base(0);
#pragma unroll
    for (int v = 0; v < SPR; ++v) {
      const int o = g.at(vb, v);
      rr[v] = bR.ld<T>(o, 0);
      rc[v] = bC.ld<T>(o, 0);
      rg[v] = bG.ld<T>(o, 0);
    }
  }
  FG<T> left = none, pup = none, xch = none, lup = none;
  T drow[SPR];   // PS: the row pair's dC, by step
  for (int r = 0; r < nrp; ++r) {
    const int vb = g.base(r), vbn = g.base(r + 1);
    if constexpr (PS) ld_rows(vbn);
#pragma unroll
    for (int v = 0; v < SPR; ++v) {
      const bool valid = vb != kOob && g.col_ok(v);
      const T rh = valid ? rr[v] * a.k : BIG;
      const T ch = rc[v] * a.k;
      const FG<T> up = h ? xch : lup;
      const FG<T> dg = v == 0 ? none : pup;
      lup = ub[v < UC ? v + 1 : 0];
      const T s2h = w2 ? (valid ? pwin<1>(rh) : BIG) : rh;
      const T rwh = w1 ? pwin<P>(s2h) : s2h;
      const T wbar = up.g * ex2(up.f - rwh) + left.g * ex2(left.f - rwh) + dg.g * ex2(dg.f - rwh);
      const T s2bar = w1 ? pwin_adj<P>(wbar, valid ? rwh : (T)0, s2h) : wbar;
      T rbar = w2 ? pwin_adj<1>(s2bar, valid ? s2h : (T)0, rh) : s2bar;
      if (v == 0 && r == 0) {
        // the last cell (T-1, U-1) (half 0): seed with grad_out * softmax_n(-R/g)
        T m = valid ? rh : INF;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) m = fmin(m, __shfl_xor(m, o));
        T s = valid ? ex2(m - rh) : (T)0;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o);
        rbar += valid ? gout * ex2(m - lg2(s) - rh) : (T)0;
      }
      if (has_gr) rbar += rg[v];
      const FG<T> cur = {valid ? rh - ch : -INF, rbar};
      if constexpr (PS) {
        drow[v] = rbar;
      } else {
        bD.st(rbar, valid ? g.at(vb, v) : kOob, 0);
      }
      left = cur;
      pup = up;
      xch = {swap_halves(cur.f), swap_halves(cur.g)};
      if (v >= 1) ub[v - 1] = xch;
      if constexpr (!PS) {
        const int o = g.at(vbn, v);
        rr[v] = bR.ld<T>(o, 0);
        rc[v] = bC.ld<T>(o, 0);
        rg[v] = bG.ld<T>(o, 0);
      }
    }
    if constexpr (PS) {
      rows_to_steps();
      // the lane's whole row (column u was step UC - 1 + h - u), from
      // column 0 up in 16-byte stores: the two halves' rows 2r and 2r + 1
      // are adjacent, so each store instruction writes whole cache lines
      constexpr int EV = 16 / (int)sizeof(T);
      typedef unsigned int u4 __attribute__((ext_vector_type(4)));
      const int o0 = vb == kOob ? kOob : g.at(vb, UC - 1 + h);
#pragma unroll
      for (int q = 0; q < UC / EV; ++q) {
        T x[EV];
#pragma unroll
        for (int e = 0; e < EV; ++e) {
          // (the empty asm keeps the select a select: folded into an index
          // h + const, it became a run-time index into drow, one compare
          // and select per element)
          const int u = q * EV + e;
          T x0 = drow[UC - 1 - u], x1 = drow[UC - u];
          asm volatile("" : "+v"(x0), "+v"(x1));
          x[e] = h ? x1 : x0;
        }
        u4 w;
        if constexpr (sizeof(T) == 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = __float_as_uint(x[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const unsigned long long z = (unsigned long long)__double_as_longlong(x[e]);
            w[2 * e] = (unsigned)z;
            w[2 * e + 1] = (unsigned)(z >> 32);
          }
        }
        __builtin_amdgcn_raw_buffer_store_b128(w, bD.r, o0 == kOob ? kOob : o0 + 16 * q, 0, 0);
      }
    }
  }
}

// ------------------------------------ several wavefronts per pair
//
// The padded-lane sweeps with the row pairs of a pair spread over the W
// wavefronts of a workgroup: wavefront w walks row pairs w, w + W, ..., and
// row pair r runs L = 2 steps behind row pair r - 1. Half 0's "up" (the row
// above the pair) is the previous wavefront's half 1, which writes each
// column to an LDS slot one step after computing it; the lag leaves one
// step between the write and the read. Every wavefront takes the same
// number of steps, each ending in a workgroup barrier (LDS operations
// complete, then s_barrier; global stores are not waited for), so a pair
// takes L (W - 1) + ceil(nrp / W) max(U + 1, L W) steps instead of
// nrp (U + 1): with one wavefront per SIMD the single-wavefront sweep is
// bound by the latency of its dependent chain, and several wavefronts
// per SIMD fill each other's waits. The arithmetic of a cell is that of the
// padded kernels; only the source of half 0's "up" changes.
constexpr int kJ3mLag = 2;     // steps between consecutive row pairs
constexpr int kJ3mWaves = 8;   // wavefronts per workgroup at most

__device__ __forceinline__ void j3_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// RS: whole-row loads of C and stores of R (as jeanie3p_fwd_kernel).
template <typename T, int UC, int P, bool RS>
__global__ void __launch_bounds__(64 * kJ3mWaves) jeanie3m_fwd_kernel(JeanieArgs<T> a) {
  constexpr int SPR = UC + 1, L = kJ3mLag;
  extern __shared__ __align__(16) unsigned char j3m_lds[];
  const int b = blockIdx.x;
  const int W = (int)blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int Tn = a.Tn, Un = a.Un, K = a.K;
  bool vn;
  const int n = pview(l32, P, a.K1, a.K2, &vn);
  const T BIG = big_v<T>(), INF = inf_v<T>();
  const int plane = Tn * Un, nrp = (Tn + 1) / 2, hl = (Tn - 1) & 1;
  const bool w1 = a.s1 > 0, w2 = a.s2 > 0;
  const int KR = (nrp + W - 1) / W, PER = SPR > L * W ? SPR : L * W;

  // LDS: [W][SPR][32] slots (wavefront w reads block w, written by w - 1),
  // then 64 slots that take half 0's stores
  T* const hand = reinterpret_cast<T*>(j3m_lds);
  T* const in_slot = hand + (size_t)wave * SPR * 32 + l32;
  T* const out_slot = h ? hand + (size_t)(wave + 1 == W ? 0 : wave + 1) * SPR * 32 + l32
                        : hand + (size_t)W * SPR * 32 + lane;

  J3Lane<T> g;
  g.init(n, h, a, false);
  g.vn = vn;
  Buf bC, bR;
  bC.init(a.C + (size_t)b * K * plane, (long long)K * plane);
  bR.init(a.Rw + (size_t)b * K * plane, (long long)K * plane);

  T cr[SPR], cnext[UC], rrow[SPR];
  auto c_steps = [&](const T (&row)[UC]) {
#pragma unroll
    for (int v = 0; v < SPR; ++v)
      cr[v] = j3_by_half(h, row[v < UC ? v : 0], row[v > 0 ? v - 1 : 0]);
  };
  if constexpr (RS) {
    const int vb = g.base(wave);
    j3_ld_row<T, UC>(bC, vb == kOob ? kOob : g.at(vb, h), cnext);
    c_steps(cnext);
  } else {
    const int vb = g.base(wave);
#pragma unroll
    for (int v = 0; v < SPR; ++v) cr[v] = bC.ld<T>(g.at(vb, v), 0);
  }
  T rlast = BIG;
  for (int i = 0; i < L * wave; ++i) j3_barrier();
  for (int k = 0; k < KR; ++k) {
    const int r = wave + k * W;
    const int vb = g.base(r), vbn = g.base(r + W);
    if constexpr (RS) j3_ld_row<T, UC>(bC, vbn == kOob ? kOob : g.at(vbn, h), cnext);
    T left = BIG, pup = BIG, xch = BIG;
#pragma unroll
    for (int v = 0; v < SPR; ++v) {
      const bool valid = vb != kOob && g.col_ok(v);
      const T ch = cr[v] * a.k;
      // half 0: the row above at column v (none above row 0, nor at column
      // UC, outside every row)
      const T up = h ? xch : ((r == 0 || v == UC) ? BIG : in_slot[v * 32]);
      const T dg = v == 0 ? ((r == 0 && h == 0) ? (T)0 : BIG) : pup;
      T rh = ch + softmin3h(up, left, dg);
      rh = valid ? rh : BIG;
      const T s2h = w2 ? (valid ? pwin<1>(rh) : BIG) : rh;
      const T rw = w1 ? pwin<P>(s2h) : s2h;
      if constexpr (RS)
        rrow[v] = rh * a.inv_k;
      else
        bR.st(rh * a.inv_k, valid ? g.at(vb, v) : kOob, 0);
      if (r == nrp - 1 && v == Un - 1 + hl) rlast = rh;
      left = rw;
      pup = up;
      xch = swap_halves(rw);
      // half 1: column v - 1 of its row, for the next row pair's half 0
      if (v >= 1) *(h ? out_slot + (v - 1) * 32 : out_slot) = rw;
      if constexpr (!RS) cr[v] = bC.ld<T>(g.at(vbn, v), 0);
      j3_barrier();
    }
    if constexpr (RS) {
      c_steps(cnext);
      T row[UC];   // column u was step u + h
#pragma unroll
      for (int u = 0; u < UC; ++u) row[u] = j3_by_half(h, rrow[u], rrow[u + 1]);
      j3_st_row<T, UC>(bR, vb == kOob ? kOob : g.at(vb, h), row);
    }
    for (int i = SPR; i < PER; ++i) j3_barrier();
  }
  for (int i = 0; i < L * (W - 1 - wave); ++i) j3_barrier();
  if (wave != (nrp - 1) % W) return;
  T m = vn ? rlast : INF;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) m = fmin(m, __shfl_xor(m, o));
  T s = (vn && m < INF) ? ex2(m - rlast) : (T)0;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o);
  if (h == hl && lane % 32 == 0) a.out[b] = (m - lg2(s)) * a.inv_k;
}

template <typename T, int UC, int P, bool PS>
__global__ void __launch_bounds__(64 * kJ3mWaves) jeanie3m_bwd_kernel(JeanieArgs<T> a) {
  constexpr int SPR = UC + 1, L = kJ3mLag;
  extern __shared__ __align__(16) unsigned char j3m_lds[];
  const int b = blockIdx.x;
  const int W = (int)blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int Tn = a.Tn, K = a.K;
  bool vn;
  const int n = pview(l32, P, a.K1, a.K2, &vn);
  const T BIG = big_v<T>(), INF = inf_v<T>();
  const int plane = Tn * a.Un, nrp = (Tn + 1) / 2;
  const T gout = a.gout[b];
  const bool has_gr = a.gR != nullptr;
  const bool w1 = a.s1 > 0, w2 = a.s2 > 0;
  const int KR = (nrp + W - 1) / W, PER = SPR > L * W ? SPR : L * W;

  FG<T>* const hand = reinterpret_cast<FG<T>*>(j3m_lds);
  FG<T>* const in_slot = hand + (size_t)wave * SPR * 32 + l32;
  FG<T>* const out_slot = h ? hand + (size_t)(wave + 1 == W ? 0 : wave + 1) * SPR * 32 + l32
                            : hand + (size_t)W * SPR * 32 + lane;

  J3Lane<T> g;
  g.init(n, h, a, true);
  g.vn = vn;
  const size_t pb = (size_t)b * K * plane;
  Buf bC, bR, bG, bD;
  bC.init(a.C + pb, (long long)K * plane);
  bR.init(a.R + pb, (long long)K * plane);
  bG.init(has_gr ? a.gR + pb : a.C, has_gr ? (long long)K * plane : 0);
  bD.init(a.dC + pb, (long long)K * plane);

  const FG<T> none = {-INF, (T)0};
  T rr[SPR], rc[SPR], rg[SPR], nR[UC], nC[UC], nG[UC], drow[SPR];
  auto to_steps = [&](const T (&row)[UC], T (&st)[SPR]) {
#pragma unroll
    for (int v = 0; v < SPR; ++v)
      st[v] = j3_by_half(h, row[v < UC ? UC - 1 - v : 0], row[v > 0 ? UC - v : 0]);
  };
  auto ld_rows = [&](int vbr) {
    const int o = vbr == kOob ? kOob : g.at(vbr, UC - 1 + h);
    j3_ld_row<T, UC>(bR, o, nR);
    j3_ld_row<T, UC>(bC, o, nC);
    if (has_gr) j3_ld_row<T, UC>(bG, o, nG);
  };
  auto rows_to_steps = [&]() {
    to_steps(nR, rr);
    to_steps(nC, rc);
    if (has_gr) to_steps(nG, rg);
  };
  if constexpr (PS) {
#pragma unroll
    for (int v = 0; v < SPR; ++v) rg[v] = (T)0;
    ld_rows(g.base(wave));
    rows_to_steps();
  } else {
    const int vb = g.base(wave);
#pragma unroll
    for (int v = 0; v < SPR; ++v) {
      const int o = g.at(vb, v);
      rr[v] = bR.ld<T>(o, 0);
      rc[v] = bC.ld<T>(o, 0);
      rg[v] = bG.ld<T>(o, 0);
    }
  }
  for (int i = 0; i < L * wave; ++i) j3_barrier();
  for (int k = 0; k < KR; ++k) {
    const int r = wave + k * W;
    const int vb = g.base(r), vbn = g.base(r + W);
    if constexpr (PS) ld_rows(vbn);
    FG<T> left = none, pup = none, xch = none;
#pragma unroll
    for (int v = 0; v < SPR; ++v) {
      const bool valid = vb != kOob && g.col_ok(v);
      const T rh = valid ? rr[v] * a.k : BIG;
      const T ch = rc[v] * a.k;
      // (selected by component: a select of the structs would take their
      // addresses and put xch in scratch memory)
      FG<T> lu = none;
      if (r != 0 && v != UC) lu = in_slot[v * 32];
      const FG<T> up = {h ? xch.f : lu.f, h ? xch.g : lu.g};
      const FG<T> dg = v == 0 ? none : pup;
      const T s2h = w2 ? (valid ? pwin<1>(rh) : BIG) : rh;
      const T rwh = w1 ? pwin<P>(s2h) : s2h;
      const T wbar = up.g * ex2(up.f - rwh) + left.g * ex2(left.f - rwh) + dg.g * ex2(dg.f - rwh);
      const T s2bar = w1 ? pwin_adj<P>(wbar, valid ? rwh : (T)0, s2h) : wbar;
      T rbar = w2 ? pwin_adj<1>(s2bar, valid ? s2h : (T)0, rh) : s2bar;
      if (v == 0 && r == 0) {
        // the last cell (T-1, U-1) (half 0): seed with grad_out * softmax_n(-R/g)
        T m = valid ? rh : INF;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) m = fmin(m, __shfl_xor(m, o));
        T s = valid ? ex2(m - rh) : (T)0;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o);
        rbar += valid ? gout * ex2(m - lg2(s) - rh) : (T)0;
      }
      if (has_gr) rbar += rg[v];
      const FG<T> cur = {valid ? rh - ch : -INF, rbar};
      if constexpr (PS)
        drow[v] = rbar;
      else
        bD.st(rbar, valid ? g.at(vb, v) : kOob, 0);
      left = cur;
      pup = up;
      xch = {swap_halves(cur.f), swap_halves(cur.g)};
      if (v >= 1) *(h ? out_slot + (v - 1) * 32 : out_slot) = cur;
      if constexpr (!PS) {
        const int o = g.at(vbn, v);
        rr[v] = bR.ld<T>(o, 0);
        rc[v] = bC.ld<T>(o, 0);
        rg[v] = bG.ld<T>(o, 0);
      }
      j3_barrier();
    }
    if constexpr (PS) {
      rows_to_steps();
      T row[UC];   // column u was step UC - 1 + h - u
#pragma unroll
      for (int u = 0; u < UC; ++u) row[u] = j3_by_half(h, drow[UC - 1 - u], drow[UC - u]);
      j3_st_row<T, UC>(bD, vb == kOob ? kOob : g.at(vb, UC - 1 + h), row);
    }
    for (int i = SPR; i < PER; ++i) j3_barrier();
  }
  for (int i = 0; i < L * (W - 1 - wave); ++i) j3_barrier();
}

// Row length the kernels are compiled for: the smallest of 8, 16, 32 that
// holds U (16 in float64), 0 beyond. Longer rows would not unroll into
// registers; they use the workgroup-per-pair kernels.
template <typename T>
static int j3_uc(int Un) {
  constexpr int umax = sizeof(T) == 4 ? 32 : 16;
  return Un <= 8 ? 8 : (Un <= 16 ? 16 : (Un <= umax ? umax : 0));
}

template <typename T, int SMAX, int UC, int KS>
static void j3_launch(bool bwd, const JeanieArgs<T>& a, int B, hipStream_t s) {
  // pair stores of dC: full rows, not transposed, even element index at dC
  const bool ps = a.Un == UC && !a.swap && (((size_t)a.dC / sizeof(T)) & 1) == 0;
  if (bwd && ps)
    hipLaunchKernelGGL((jeanie3_bwd_kernel<T, SMAX, UC, KS, true>), dim3(B), dim3(64), 0, s, a);
  else if (bwd)
    hipLaunchKernelGGL((jeanie3_bwd_kernel<T, SMAX, UC, KS, false>), dim3(B), dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL((jeanie3_fwd_kernel<T, SMAX, UC, KS>), dim3(B), dim3(64), 0, s, a);
}

template <typename T, int SMAX, int KS>
static void j3_launch_uc(bool bwd, int uc, const JeanieArgs<T>& a, int B, hipStream_t s) {
  switch (uc) {
    case 8: j3_launch<T, SMAX, 8, KS>(bwd, a, B, s); break;
    case 16: j3_launch<T, SMAX, 16, KS>(bwd, a, B, s); break;
    default:
      if constexpr (sizeof(T) == 4) j3_launch<T, SMAX, 32, KS>(bwd, a, B, s);
      break;
  }
}

// Axis-1 strides with LDS-free neighbour moves: 1 (one viewpoint axis) and 5
// (5 x 5 viewpoints); other strides exchange through ds_bpermute.
template <typename T, int SMAX>
static void j3_launch_ks(bool bwd, int uc, const JeanieArgs<T>& a, int B, hipStream_t s) {
  if (a.K2 == 1)
    j3_launch_uc<T, SMAX, 1>(bwd, uc, a, B, s);
  else if (a.K2 == 5)
    j3_launch_uc<T, SMAX, 5>(bwd, uc, a, B, s);
  else
    j3_launch_uc<T, SMAX, 0>(bwd, uc, a, B, s);
}

template <typename T, int P>
static void j3p_launch_uc(bool bwd, int uc, const JeanieArgs<T>& a, int B, hipStream_t s) {
  // whole-row loads and stores: full rows, not transposed, 16-byte aligned
  auto al16 = [](const void* p) { return ((size_t)p & 15) == 0; };
  const bool rows = a.Un == uc && !a.swap;
  const bool ps = rows && al16(a.dC) && al16(a.C) && al16(a.R) && al16(a.gR);
  const bool rs = rows && al16(a.Rw) && al16(a.C);
#define TW_J3P(UC_)                                                                              \
  do {                                                                                           \
    if (bwd && ps)                                                                               \
      hipLaunchKernelGGL((jeanie3p_bwd_kernel<T, UC_, P, true>), dim3(B), dim3(64), 0, s, a);    \
    else if (bwd)                                                                                \
      hipLaunchKernelGGL((jeanie3p_bwd_kernel<T, UC_, P, false>), dim3(B), dim3(64), 0, s, a);   \
    else if (rs)                                                                                 \
      hipLaunchKernelGGL((jeanie3p_fwd_kernel<T, UC_, P, true>), dim3(B), dim3(64), 0, s, a);    \
    else                                                                                         \
      hipLaunchKernelGGL((jeanie3p_fwd_kernel<T, UC_, P, false>), dim3(B), dim3(64), 0, s, a);   \
  } while (0)
  switch (uc) {
    case 8: TW_J3P(8); break;
    case 16: TW_J3P(16); break;
    default:
      if constexpr (sizeof(T) == 4) TW_J3P(32);
      break;
  }
#undef TW_J3P
}

// Several wavefronts per pair (W of them, 2 <= W <= kJ3mWaves).
template <typename T, int P>
static void j3m_launch_uc(bool bwd, int uc, int W, const JeanieArgs<T>& a, int B, hipStream_t s) {
  // whole-row loads and stores: full rows, not transposed, 16-byte aligned,
  // of at most 64 bytes (longer rows' registers would spill under the
  // 512-thread launch bound)
  auto al16 = [](const void* p) { return ((size_t)p & 15) == 0; };
  const bool rows = a.Un == uc && !a.swap && uc * sizeof(T) <= 64;
  const bool ps = rows && al16(a.dC) && al16(a.C) && al16(a.R) && al16(a.gR);
  const bool rs = rows && al16(a.Rw) && al16(a.C);
  const size_t elem = bwd ? 2 * sizeof(T) : sizeof(T);
  const size_t lds = ((size_t)W * (uc + 1) * 32 + 64) * elem;
  const dim3 grid((unsigned)B), block((unsigned)(64 * W));
#define TW_J3M(UC_)                                                                              \
  do {                                                                                           \
    if (bwd && ps)                                                                               \
      hipLaunchKernelGGL((jeanie3m_bwd_kernel<T, UC_, P, true>), grid, block, lds, s, a);        \
    else if (bwd)                                                                                \
      hipLaunchKernelGGL((jeanie3m_bwd_kernel<T, UC_, P, false>), grid, block, lds, s, a);       \
    else if (rs)                                                                                 \
      hipLaunchKernelGGL((jeanie3m_fwd_kernel<T, UC_, P, true>), grid, block, lds, s, a);        \
    else                                                                                         \
      hipLaunchKernelGGL((jeanie3m_fwd_kernel<T, UC_, P, false>), grid, block, lds, s, a);       \
  } while (0)
  switch (uc) {
    case 8: TW_J3M(8); break;
    case 16: TW_J3M(16); break;
    default:
      if constexpr (sizeof(T) == 4) TW_J3M(32);
      break;
  }
#undef TW_J3M
}

// TORCHWARP_JEANIE_MW: 0 keeps one wavefront per pair in the padded-lane
// sweeps; otherwise (unset) pairs of two row pairs or more take several.
static int j3m_mode() {
  static const int mode = [] {
    const char* e = getenv("TORCHWARP_JEANIE_MW");
    return e ? atoi(e) : -1;
  }();
  return mode;
}

template <typename T>
static int j3_run(bool bwd, const JeanieArgs<T>& a, int B, hipStream_t s, const char* what) {
  const int uc = j3_uc<T>(a.Un);
  if (a.K > 32 || uc == 0 || a.s1 > 2 || a.s2 > 2) return kJ3Unsupported;
  if (B == 0) return TW_OK;
  // padded lanes: windows of one neighbour each way, one unused lane after
  // each axis-2 row when that axis has a window, and lane 31 of each half
  // unused (the stride-1 wave shifts cross from one half into the other);
  // strides 1 and 6 built (one viewpoint axis, and 5 x 5 viewpoints)
  const int P = a.K2 + (a.s2 > 0 ? 1 : 0);
  if (a.s1 <= 1 && a.s2 <= 1 && a.K1 * P < 32 && (P == 1 || P == 6)) {
    // Wavefronts per pair: one while the batch fills half the SIMDs with a
    // wavefront per pair (lockstep wavefronts sharing SIMDs with other
    // workgroups' measured slower than one wavefront walking the whole pair:
    // cfg5a, 1024 pairs, W = 2: backward 50.9 -> 55.7 us); below that about
    // two per SIMD over the batch, at most one per row pair (cfg4, 400 pairs,
    // W = 4: 0.066 -> 0.059 ms per step).
    const int nrp = (a.Tn + 1) / 2;
    const long long simds = 4LL * num_cus();
    int W = 1;
    if (2LL * B <= simds) {
      const long long w = (2 * simds + B - 1) / (B > 0 ? B : 1);
      W = (int)(w < nrp ? w : nrp);
      W = W < kJ3mWaves ? W : kJ3mWaves;
    }
    if (W >= 2 && j3m_mode() != 0) {
      if (P == 1)
        j3m_launch_uc<T, 1>(bwd, uc, W, a, B, s);
      else
        j3m_launch_uc<T, 6>(bwd, uc, W, a, B, s);
    } else if (P == 1) {
      j3p_launch_uc<T, 1>(bwd, uc, a, B, s);
    } else {
      j3p_launch_uc<T, 6>(bwd, uc, a, B, s);
    }
    return check_launch(what);
  }
  if (a.s1 > 1 || a.s2 > 1)
    j3_launch_ks<T, 2>(bwd, uc, a, B, s);
  else
    j3_launch_ks<T, 1>(bwd, uc, a, B, s);
  return check_launch(what);
}

template <typename T>
int jeanie3_fwd(const JeanieArgs<T>& a, int B, hipStream_t s, const char* what) {
  return j3_run<T>(false, a, B, s, what);
}

template <typename T>
int jeanie3_bwd(const JeanieArgs<T>& a, int B, hipStream_t s, const char* what) {
  return j3_run<T>(true, a, B, s, what);
}

template int jeanie3_fwd<float>(const JeanieArgs<float>&, int, hipStream_t, const char*);
template int jeanie3_fwd<double>(const JeanieArgs<double>&, int, hipStream_t, const char*);
template int jeanie3_bwd<float>(const JeanieArgs<float>&, int, hipStream_t, const char*);
template int jeanie3_bwd<double>(const JeanieArgs<double>&, int, hipStream_t, const char*);

}  // namespace tw
