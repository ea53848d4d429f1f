// uDTW / soft-DTW dynamic program for gfx950: forward and fused backward.
//
// One workgroup per sequence pair. Thread t owns the ROWS contiguous grid
// rows t*ROWS .. t*ROWS+ROWS-1 and sweeps the anti-diagonals d = i + j with
// its rows' two previous diagonals held in registers. The only cross-thread
// value per diagonal is the last owned row of the previous thread (forward)
// or the first owned row of the next thread (backward): a DPP wave shift
// inside a wavefront, an LDS mailbox between wavefronts. Wavefronts meet at
// an LDS-only barrier once per diagonal.
//
// Forward (reference: udtw_cuda.cu:57-164 and :298-422, udtw/_torch_dp.py:14-42):
//   R[i,j] = C[i,j] + softmin_g(R[i-1,j-1], R[i-1,j], R[i,j-1])
//   P[i,j] = Q[i,j] + sum_k softmax(-R_k/g)_k P_k
// with R[-1,-1] = 0 and +inf elsewhere on the border, R = +inf / P = 0 for
// unreachable cells and outside the Sakoe-Chiba band |i-j| <= band.
// R is stored scaled (Rh = R log2(e)/g) in a diagonal-major layout (the
// cells of diagonal d contiguous, by row), P unscaled in the same layout;
// both are internal tensors carried from the forward to the backward.
//
// Backward (udtw_cuda.cu:166-278, :424-582; udtw/_torch_dp.py:45-75), for
// L = gR R[N-1,M-1] + gP P[N-1,M-1] and successors s of cell k:
//   w = 2^(Eh_s - Rh_k),  Eh = Rh - Ch
//   Rbar_k = sum_s w (Rbar_s - Pbar_s (P_k - A_s) / g),  A = P - Q
//   Pbar_k = sum_s w Pbar_s.
//
// Cost sources (template SRC):
//   SRC_COST  C, Q given as [B,N,M]                   -> writes dC, dQ
//   SRC_SQ    raw squared distance S = x2+y2-2x.y [B,N,M] and variances
//             vx [B,N], vy [B,M]: C = max(S,0)/max((vx+vy)/2,eps),
//             Q = beta ln max(...)                      -> writes dS, dvx, dvy
//   SRC_FEAT1 one feature per step, x [B,N], y [B,M] and variances,
//             C from (x-y)^2 in registers               -> writes dx, dy, dvx, dvy
// Column sums (dy, dvy) accumulate in LDS: on one diagonal every column is
// touched by exactly one cell, so the adds never collide and their order is
// fixed by the diagonal index (bitwise deterministic).

#include "tw_capi.hpp"
#include "tw_common.hpp"
#include "../../include/torchwarp_hip.h"

namespace tw {

enum { SRC_COST = 0, SRC_SQ = 1, SRC_FEAT1 = 2 };

template <typename T>
struct UdtwArgs {
  const T* C;    // SRC_COST cost / SRC_SQ raw squared distance, [B,N,M]
  const T* Q;    // SRC_COST penalty [B,N,M] (PEN)
  const T* X;    // SRC_FEAT1 [B,N]
  const T* Y;    // SRC_FEAT1 [B,M]
  const T* VX;   // SRC_SQ / SRC_FEAT1 [B,N]
  const T* VY;   // [B,M]
  T* R;          // [B, N*M] diagonal-major, scaled
  T* P;          // [B, N*M] diagonal-major (PEN)
  T* out_r;      // [B]
  T* out_p;      // [B]
  const T* gr;   // [B]
  const T* gp;   // [B] (PEN)
  T* dC;         // SRC_COST d cost / SRC_SQ d squared distance, [B,N,M]
  T* dQ;         // SRC_COST d penalty (may be null)
  T* dX;         // SRC_FEAT1 [B,N]
  T* dY;         // SRC_FEAT1 [B,M]
  T* dVX;        // SRC_SQ / SRC_FEAT1 [B,N] (may be null: no variance gradient)
  T* dVY;        // [B,M]
  int N, M;
  T k;           // log2(e) / gamma
  T inv_k;       // gamma ln 2
  T inv_gamma;   // 1 / gamma
  T beta;
  T beta_ln2;    // beta ln 2
  T eps;
  T band;        // <= 0: no band
};

// Cell cost in the scaled domain plus the pieces the chain rule needs.
template <typename T>
struct CellCost {
  T ch;       // scaled cost  C * log2(e)/g
  T q;        // penalty
  T c;        // unscaled cost (SRC_SQ / SRC_FEAT1)
  T rv;       // 1 / var
  T sq_raw;   // squared distance before the clamp
  T var_raw;  // variance before the clamp
};

template <typename T, int SRC, bool PEN>
__device__ __forceinline__ CellCost<T> cell_cost(const UdtwArgs<T>& a, T cin, T qin, T x, T vx,
                                                 T y, T vy) {
  CellCost<T> o;
  if (SRC == SRC_COST) {
    o.c = cin;
    o.ch = cin * a.k;
    o.q = PEN ? qin : (T)0;
    o.rv = (T)1;
    o.sq_raw = (T)0;
    o.var_raw = (T)1;
  } else {
    T sq_raw;
    if (SRC == SRC_FEAT1) {
      const T df = x - y;
      sq_raw = df * df;
    } else {
      sq_raw = cin;
    }
    const T sq = sq_raw > (T)0 ? sq_raw : (T)0;
    const T var_raw = (T)0.5 * (vx + vy);
    const T var = var_raw > a.eps ? var_raw : a.eps;
    o.rv = rcp(var);
    o.c = sq * o.rv;
    o.ch = o.c * a.k;
    o.q = PEN ? a.beta_ln2 * lg2(var) : (T)0;
    o.sq_raw = sq_raw;
    o.var_raw = var_raw;
  }
  return o;
}

template <typename T, int ROWS, int SRC, bool PEN>
__global__ void __launch_bounds__(1024) udtw_fwd_kernel(UdtwArgs<T> a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* sm = reinterpret_cast<T*>(smem_raw);
  const int N = a.N, M = a.M;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const T INF = inf_v<T>();
  const size_t NM = (size_t)N * M;

  T* mbr = sm;                 // mailbox R [2][nw]
  T* mbp = sm + 2 * nw;        // mailbox P [2][nw]
  T* ys = sm + 4 * nw;         // y  [M]  (SRC_FEAT1)
  T* vys = ys + (SRC == SRC_FEAT1 ? M : 0);  // vy [M] (SRC_SQ, SRC_FEAT1)

  if (SRC == SRC_FEAT1)
    for (int t = tid; t < M; t += blockDim.x) ys[t] = a.Y[(size_t)b * M + t];
  if (SRC != SRC_COST)
    for (int t = tid; t < M; t += blockDim.x) vys[t] = a.VY[(size_t)b * M + t];
  for (int t = tid; t < 2 * nw; t += blockDim.x) {
    mbr[t] = INF;
    mbp[t] = (T)0;
  }

  const int row0 = tid * ROWS;
  T xr[ROWS], vxr[ROWS];
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    const int i = row0 + k;
    xr[k] = (SRC == SRC_FEAT1 && i < N) ? a.X[(size_t)b * N + i] : (T)0;
    vxr[k] = (SRC != SRC_COST && i < N) ? a.VX[(size_t)b * N + i] : (T)1;
  }
  T r1[ROWS], r2[ROWS], p1[ROWS], p2[ROWS];
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    r1[k] = INF;
    r2[k] = INF;
    p1[k] = (T)0;
    p2[k] = (T)0;
  }
  // Neighbour row (previous thread's last row) at diagonals d-1 and d-2.
  // Thread 0's "neighbour" is the border; its value 0 at the origin makes
  // the generic update give R[0,0] = C[0,0], P[0,0] = Q[0,0].
  T nr1 = (tid == 0) ? (T)0 : INF, nr2 = INF, np1 = (T)0, np2 = (T)0;

  const T* Cb = a.C ? a.C + b * NM : nullptr;
  const T* Qb = a.Q ? a.Q + b * NM : nullptr;
  T* Rb = a.R + b * NM;
  T* Pb = PEN ? a.P + b * NM : nullptr;

  T pc[ROWS], pq[ROWS];
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    pc[k] = (T)0;
    pq[k] = (T)0;
  }
  auto fetch = [&](int d) {
    if (SRC == SRC_FEAT1) return;
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const int i = row0 + k, j = d - i;
      if (i < N && j >= 0 && j < M) {
        const size_t o = (size_t)i * M + j;
        pc[k] = Cb[o];
        if (SRC == SRC_COST && PEN) pq[k] = Qb[o];
      }
    }
  };
  fetch(0);
  __syncthreads();

  const int Dn = N + M - 1;
  long long off = 0;
  for (int d = 0; d < Dn; ++d) {
    const int lo = max(0, d - M + 1), hi = min(N - 1, d);
    T cc[ROWS], cq[ROWS];
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      cc[k] = pc[k];
      cq[k] = pq[k];
    }
    if (d + 1 < Dn) fetch(d + 1);

    nr2 = nr1;
    np2 = np1;
    {
      T sr = from_prev_lane(r1[ROWS - 1], INF);
      T sp = PEN ? from_prev_lane(p1[ROWS - 1], (T)0) : (T)0;
      if (lane == 0) {
        if (wave == 0) {
          sr = INF;
          sp = (T)0;
        } else {
          const int par = (d - 1) & 1;
          sr = mbr[par * nw + wave - 1];
          if (PEN) sp = mbp[par * nw + wave - 1];
        }
      }
      nr1 = sr;
      np1 = sp;
    }

    T nr[ROWS], np[ROWS];
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const int i = row0 + k, j = d - i;
      const bool valid = (i < N) & (j >= 0) & (j < M);
      const int jc = j < 0 ? 0 : (j >= M ? M - 1 : j);
      const T up = k ? r1[k - 1] : nr1;
      const T dg = k ? r2[k - 1] : nr2;
      const T lf = r1[k];
      T y = (T)0, vy = (T)1;
      if (SRC == SRC_FEAT1) y = ys[jc];
      if (SRC != SRC_COST) vy = vys[jc];
      const CellCost<T> cv = cell_cost<T, SRC, PEN>(a, cc[k], cq[k], xr[k], vxr[k], y, vy);
      const T m = min3(dg, up, lf);
      const T ed = ex2(m - dg), eu = ex2(m - up), el = ex2(m - lf);
      const T s = ed + eu + el;
      const T rv = cv.ch + m - lg2(s);
      bool ok = valid && (m < INF);
      if (a.band > (T)0) ok = ok && (fabs((T)(i - j)) <= a.band);
      nr[k] = ok ? rv : INF;
      if (PEN) {
        const T pup = k ? p1[k - 1] : np1;
        const T pdg = k ? p2[k - 1] : np2;
        const T pv = cv.q + (ed * pdg + eu * pup + el * p1[k]) * rcp(s);
        np[k] = ok ? pv : (T)0;
      } else {
        np[k] = (T)0;
      }
      if (valid) {
        const long long o = off + (i - lo);
        Rb[o] = nr[k];
        if (PEN) Pb[o] = np[k];
      }
    }
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      r2[k] = r1[k];
      r1[k] = nr[k];
      p2[k] = p1[k];
      p1[k] = np[k];
    }
    if (nw > 1) {
      const int par = d & 1;
      if (lane == 63) {
        mbr[par * nw + wave] = r1[ROWS - 1];
        if (PEN) mbp[par * nw + wave] = p1[ROWS - 1];
      }
      lds_barrier();
    }
    off += hi - lo + 1;
  }
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    if (row0 + k == N - 1) {
      a.out_r[b] = r1[k] < INF ? r1[k] * a.inv_k : INF;
      a.out_p[b] = PEN ? p1[k] : (T)0;
    }
  }
}

template <typename T, int ROWS, int SRC, bool PEN>
__global__ void __launch_bounds__(1024) udtw_bwd_kernel(UdtwArgs<T> a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* sm = reinterpret_cast<T*>(smem_raw);
  const int N = a.N, M = a.M;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const T INF = inf_v<T>();
  const size_t NM = (size_t)N * M;
  const bool vgrad = SRC != SRC_COST && a.dVX != nullptr;

  T* mbe = sm;                 // mailboxes [2][nw] each: E, G(Rbar), H(Pbar), A
  T* mbg = sm + 2 * nw;
  T* mbh = sm + 4 * nw;
  T* mba = sm + 6 * nw;
  T* ys = sm + 8 * nw;                              // y   [M] (FEAT1)
  T* vys = ys + (SRC == SRC_FEAT1 ? M : 0);         // vy  [M] (SQ, FEAT1)
  T* dys = vys + (SRC != SRC_COST ? M : 0);         // dy  [M] (FEAT1)
  T* dvys = dys + (SRC == SRC_FEAT1 ? M : 0);       // dvy [M] (SQ, FEAT1)

  for (int t = tid; t < M; t += blockDim.x) {
    if (SRC == SRC_FEAT1) {
      ys[t] = a.Y[(size_t)b * M + t];
      dys[t] = (T)0;
    }
    if (SRC != SRC_COST) {
      vys[t] = a.VY[(size_t)b * M + t];
      dvys[t] = (T)0;
    }
  }
  for (int t = tid; t < 2 * nw; t += blockDim.x) {
    mbe[t] = -INF;
    mbg[t] = (T)0;
    mbh[t] = (T)0;
    mba[t] = (T)0;
  }

  const int row0 = tid * ROWS;
  T xr[ROWS], vxr[ROWS], dxr[ROWS], dvr[ROWS];
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    const int i = row0 + k;
    xr[k] = (SRC == SRC_FEAT1 && i < N) ? a.X[(size_t)b * N + i] : (T)0;
    vxr[k] = (SRC != SRC_COST && i < N) ? a.VX[(size_t)b * N + i] : (T)1;
    dxr[k] = (T)0;
    dvr[k] = (T)0;
  }
  // Own rows at diagonals d+1 (…1) and d+2 (…2).
  T e1[ROWS], e2[ROWS], g1[ROWS], g2[ROWS], h1[ROWS], h2[ROWS], a1[ROWS], a2[ROWS];
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    e1[k] = e2[k] = -INF;
    g1[k] = g2[k] = h1[k] = h2[k] = a1[k] = a2[k] = (T)0;
  }
  // Next thread's first row at d+1 / d+2.
  T ne1 = -INF, ne2 = -INF, ng1 = 0, ng2 = 0, nh1 = 0, nh2 = 0, na1 = 0, na2 = 0;

  const T* Cb = a.C ? a.C + b * NM : nullptr;
  const T* Qb = a.Q ? a.Q + b * NM : nullptr;
  const T* Rb = a.R + b * NM;
  const T* Pb = PEN ? a.P + b * NM : nullptr;
  T* dCb = a.dC ? a.dC + b * NM : nullptr;
  T* dQb = a.dQ ? a.dQ + b * NM : nullptr;
  const T gr = a.gr[b];
  const T gp = PEN ? a.gp[b] : (T)0;

  const int Dn = N + M - 1;
  T pr[ROWS], pp[ROWS], pc[ROWS], pq[ROWS];
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    pr[k] = INF;
    pp[k] = pc[k] = pq[k] = (T)0;
  }
  auto fetch = [&](int d, long long off) {
    const int lo = max(0, d - M + 1);
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const int i = row0 + k, j = d - i;
      if (i < N && j >= 0 && j < M) {
        const long long od = off + (i - lo);
        pr[k] = Rb[od];
        if (PEN) pp[k] = Pb[od];
        if (SRC != SRC_FEAT1) {
          const size_t o = (size_t)i * M + j;
          pc[k] = Cb[o];
          if (SRC == SRC_COST && PEN) pq[k] = Qb[o];
        }
      }
    }
  };
  long long off = (long long)NM - 1;
  fetch(Dn - 1, off);
  __syncthreads();

  for (int d = Dn - 1; d >= 0; --d) {
    const int lo = max(0, d - M + 1);
    T cr[ROWS], cp[ROWS], cc[ROWS], cq[ROWS];
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      cr[k] = pr[k];
      cp[k] = pp[k];
      cc[k] = pc[k];
      cq[k] = pq[k];
    }
    long long off1 = off;
    if (d > 0) {
      const int lo1 = max(0, d - 1 - M + 1), hi1 = min(N - 1, d - 1);
      off1 = off - (hi1 - lo1 + 1);
      fetch(d - 1, off1);
    }

    ne2 = ne1;
    ng2 = ng1;
    nh2 = nh1;
    na2 = na1;
    {
      T se = from_next_lane(e1[0], -INF);
      T sg = from_next_lane(g1[0], (T)0);
      T sh = PEN ? from_next_lane(h1[0], (T)0) : (T)0;
      T sa = PEN ? from_next_lane(a1[0], (T)0) : (T)0;
      if (lane == 63) {
        if (wave == nw - 1) {
          se = -INF;
          sg = sh = sa = (T)0;
        } else {
          const int par = (d + 1) & 1;
          se = mbe[par * nw + wave + 1];
          sg = mbg[par * nw + wave + 1];
          if (PEN) {
            sh = mbh[par * nw + wave + 1];
            sa = mba[par * nw + wave + 1];
          }
        }
      }
      ne1 = se;
      ng1 = sg;
      nh1 = sh;
      na1 = sa;
    }

    T xe[ROWS], xg[ROWS], xh[ROWS], xa[ROWS];
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const int i = row0 + k, j = d - i;
      const bool valid = (i < N) & (j >= 0) & (j < M);
      const int jc = j < 0 ? 0 : (j >= M ? M - 1 : j);
      const T rk = valid ? cr[k] : INF;
      const T pk = cp[k];
      T y = (T)0, vy = (T)1;
      if (SRC == SRC_FEAT1) y = ys[jc];
      if (SRC != SRC_COST) vy = vys[jc];
      const CellCost<T> cv = cell_cost<T, SRC, PEN>(a, cc[k], cq[k], xr[k], vxr[k], y, vy);
      // successors: down (i+1, j) and right (i, j+1) on d+1, diagonal (i+1, j+1) on d+2
      const T edn = (k + 1 < ROWS) ? e1[k + 1] : ne1;
      const T gdn = (k + 1 < ROWS) ? g1[k + 1] : ng1;
      const T edg = (k + 1 < ROWS) ? e2[k + 1] : ne2;
      const T gdg = (k + 1 < ROWS) ? g2[k + 1] : ng2;
      const T ert = e1[k], grt = g1[k];
      T g, h = (T)0;
      if (d == Dn - 1) {
        g = gr;
        h = gp;
      } else {
        const T wdn = ex2(edn - rk), wrt = ex2(ert - rk), wdg = ex2(edg - rk);
        g = wdn * gdn + wrt * grt + wdg * gdg;
        if (PEN) {
          const T hdn = (k + 1 < ROWS) ? h1[k + 1] : nh1;
          const T adn = (k + 1 < ROWS) ? a1[k + 1] : na1;
          const T hdg = (k + 1 < ROWS) ? h2[k + 1] : nh2;
          const T adg = (k + 1 < ROWS) ? a2[k + 1] : na2;
          const T hrt = h1[k], art = a1[k];
          const T wh_dn = wdn * hdn, wh_rt = wrt * hrt, wh_dg = wdg * hdg;
          g -= (wh_dn * (pk - adn) + wh_rt * (pk - art) + wh_dg * (pk - adg)) * a.inv_gamma;
          h = wh_dn + wh_rt + wh_dg;
        }
        if (!(rk < INF)) {
          g = (T)0;
          h = (T)0;
        }
      }
      if (!valid) {
        g = (T)0;
        h = (T)0;
      }
      xe[k] = (valid && rk < INF) ? rk - cv.ch : -INF;
      xg[k] = g;
      xh[k] = h;
      xa[k] = valid ? pk - cv.q : (T)0;

      if (valid) {
        if (SRC == SRC_COST) {
          const size_t o = (size_t)i * M + j;
          dCb[o] = g;
          if (dQb) dQb[o] = h;
        } else {
          const T dsq = cv.sq_raw > (T)0 ? g * cv.rv : (T)0;
          if (SRC == SRC_SQ) dCb[(size_t)i * M + j] = dsq;
          if (SRC == SRC_FEAT1) {
            const T df = (T)2 * dsq * (xr[k] - y);
            dxr[k] += df;
            atomicAdd(&dys[j], -df);
          }
          if (vgrad) {
            const T dvar = cv.var_raw > a.eps ? (a.beta * h - g * cv.c) * cv.rv : (T)0;
            dvr[k] += (T)0.5 * dvar;
            atomicAdd(&dvys[j], (T)0.5 * dvar);
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      e2[k] = e1[k];
      e1[k] = xe[k];
      g2[k] = g1[k];
      g1[k] = xg[k];
      h2[k] = h1[k];
      h1[k] = xh[k];
      a2[k] = a1[k];
      a1[k] = xa[k];
    }
    if (nw > 1) {
      const int par = d & 1;
      if (lane == 0) {
        mbe[par * nw + wave] = e1[0];
        mbg[par * nw + wave] = g1[0];
        if (PEN) {
          mbh[par * nw + wave] = h1[0];
          mba[par * nw + wave] = a1[0];
        }
      }
      lds_barrier();
    }
    off = off1;
  }

#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    const int i = row0 + k;
    if (i < N) {
      if (SRC == SRC_FEAT1) a.dX[(size_t)b * N + i] = dxr[k];
      if (vgrad) a.dVX[(size_t)b * N + i] = dvr[k];
    }
  }
  if (SRC != SRC_COST) {
    __syncthreads();
    for (int t = tid; t < M; t += blockDim.x) {
      if (SRC == SRC_FEAT1) a.dY[(size_t)b * M + t] = dys[t];
      if (vgrad) a.dVY[(size_t)b * M + t] = dvys[t];
    }
  }
}

// ---------------------------------------------------------------- launching

struct Shape {
  int rows;
  int threads;
};

// Rows per thread and threads per pair for a grid with N rows (N <= M).
// Up to 4 wavefronts (one per SIMD of a CU), more rows per thread beyond.
static Shape pick_shape(int N) {
  int rows = 1;
  while (rows < 16 && (N + rows - 1) / rows > 256) rows *= 2;
  int threads = (N + rows - 1) / rows;
  if (threads > 1024) return {0, 0};
  threads = ((threads + 63) / 64) * 64;
  return {rows, threads};
}

template <typename T, int SRC, bool PEN>
static size_t fwd_lds(int nw, int M) {
  size_t n = 4 * (size_t)nw;
  if (SRC == SRC_FEAT1) n += 2 * (size_t)M;
  if (SRC == SRC_SQ) n += (size_t)M;
  return n * sizeof(T);
}

template <typename T, int SRC, bool PEN>
static size_t bwd_lds(int nw, int M) {
  size_t n = 8 * (size_t)nw;
  if (SRC == SRC_FEAT1) n += 4 * (size_t)M;
  if (SRC == SRC_SQ) n += 2 * (size_t)M;
  return n * sizeof(T);
}

template <typename T, int SRC, bool PEN>
static int launch_udtw(bool backward, const UdtwArgs<T>& a, int B, hipStream_t stream,
                       const char* what) {
  if (B == 0) return TW_OK;
  const Shape sh = pick_shape(a.N);
  if (sh.rows == 0) {
    return fail(TW_ESIZE, "%s: the shorter sequence has %d steps; this build handles up to 16384",
                what, a.N);
  }
  const int nw = sh.threads / 64;
  const size_t lds = backward ? bwd_lds<T, SRC, PEN>(nw, a.M) : fwd_lds<T, SRC, PEN>(nw, a.M);
  if (lds > (size_t)max_lds_bytes()) {
    return fail(TW_ESIZE, "%s: %zu bytes of LDS needed (M = %d), %d available", what, lds, a.M,
                max_lds_bytes());
  }
  dim3 grid(B), block(sh.threads);
#define TW_UDTW_CASE(R_)                                                                   \
  case R_:                                                                                 \
    if (backward)                                                                          \
      hipLaunchKernelGGL((udtw_bwd_kernel<T, R_, SRC, PEN>), grid, block, lds, stream, a); \
    else                                                                                   \
      hipLaunchKernelGGL((udtw_fwd_kernel<T, R_, SRC, PEN>), grid, block, lds, stream, a); \
    break;
  switch (sh.rows) {
    TW_UDTW_CASE(1)
    TW_UDTW_CASE(2)
    TW_UDTW_CASE(4)
    TW_UDTW_CASE(8)
    TW_UDTW_CASE(16)
    default:
      return fail(TW_EINVAL, "%s: internal: bad row count", what);
  }
#undef TW_UDTW_CASE
  return check_launch(what);
}

template <typename T, int SRC>
static int launch_pen(bool pen, bool backward, const UdtwArgs<T>& a, int B, hipStream_t s,
                      const char* what) {
  return pen ? launch_udtw<T, SRC, true>(backward, a, B, s, what)
             : launch_udtw<T, SRC, false>(backward, a, B, s, what);
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
                    int B, int N, int M, double gamma, T* dC, T* dQ, hipStream_t s,
                    const char* what) {
  if (int e = check_dims(what, B, N, M, gamma)) return e;
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
  set_hyper(a, gamma, 0.0, 1.0, 0.0);
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
  return cost_bwd<T>(C, Q, R, P, gr, gp, B, N, M, gamma, dC, dQ, s, what);
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
                         float gamma, float* d_cost, float* d_pen, hipStream_t stream) {
  return cost_bwd<float>(cost, pen, R, P, grad_dist, grad_pen, B, N, M, gamma, d_cost, d_pen,
                         stream, "tw_udtw_cost_bwd_f32");
}

int tw_udtw_cost_bwd_f64(const double* cost, const double* pen, const double* R,
                         const double* P, const double* grad_dist, const double* grad_pen, int B,
                         int N, int M, double gamma, double* d_cost, double* d_pen,
                         hipStream_t stream) {
  return cost_bwd<double>(cost, pen, R, P, grad_dist, grad_pen, B, N, M, gamma, d_cost, d_pen,
                          stream, "tw_udtw_cost_bwd_f64");
}

}  // extern "C"

// Features path: defined with the pairwise-distance kernels it uses for D > 1.
namespace tw {

template <typename T>
int sqdist_raw(const T* X, const T* Y, int P, int R, int C, int D, T* out, hipStream_t s,
               const char* what);
template <typename T>
int sqdist_raw_bwd(const T* X, const T* Y, const T* dS, int P, int R, int C, int D, T* dX, T* dY,
                   hipStream_t s, const char* what);

template <typename T>
static int feat_fwd(const T* X, const T* Y, const T* vx, const T* vy, int B, int N, int M, int D,
                    double gamma, double beta, double eps, double band, T* R, T* P, T* out_r,
                    T* out_p, T* ws, size_t ws_bytes, hipStream_t s, const char* what) {
  if (int e = check_dims(what, B, N, M, gamma)) return e;
  if (D <= 0) return fail(TW_EINVAL, "%s: D must be > 0", what);
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
                    double beta, double eps, T* dX, T* dY, T* dvx, T* dvy, T* ws,
                    size_t ws_bytes, hipStream_t s, const char* what) {
  if (int e = check_dims(what, B, N, M, gamma)) return e;
  if (D <= 0) return fail(TW_EINVAL, "%s: D must be > 0", what);
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
  set_hyper(a, gamma, beta, eps, 0.0);
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
  // recompute the raw squared distances, then overwrite them in place with
  // their adjoint (each cell is read and written by the same thread)
  if (int e = sqdist_raw<T>(X, Y, B, N, M, D, ws, s, what)) return e;
  a.C = ws;
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
                         float bandwidth, float* R, float* P, float* out_dist, float* out_pen,
                         float* workspace, size_t workspace_bytes, hipStream_t stream) {
  return feat_fwd<float>(X, Y, vx, vy, B, N, M, D, gamma, beta, eps, bandwidth, R, P, out_dist,
                         out_pen, workspace, workspace_bytes, stream, "tw_udtw_feat_fwd_f32");
}

int tw_udtw_feat_fwd_f64(const double* X, const double* Y, const double* vx, const double* vy,
                         int B, int N, int M, int D, double gamma, double beta, double eps,
                         double bandwidth, double* R, double* P, double* out_dist,
                         double* out_pen, double* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  return feat_fwd<double>(X, Y, vx, vy, B, N, M, D, gamma, beta, eps, bandwidth, R, P, out_dist,
                          out_pen, workspace, workspace_bytes, stream, "tw_udtw_feat_fwd_f64");
}

int tw_udtw_feat_bwd_f32(const float* X, const float* Y, const float* vx, const float* vy,
                         const float* R, const float* P, const float* grad_dist,
                         const float* grad_pen, int B, int N, int M, int D, float gamma,
                         float beta, float eps, float* dX, float* dY, float* dvx, float* dvy,
                         float* workspace, size_t workspace_bytes, hipStream_t stream) {
  return feat_bwd<float>(X, Y, vx, vy, R, P, grad_dist, grad_pen, B, N, M, D, gamma, beta, eps,
                         dX, dY, dvx, dvy, workspace, workspace_bytes, stream,
                         "tw_udtw_feat_bwd_f32");
}

int tw_udtw_feat_bwd_f64(const double* X, const double* Y, const double* vx, const double* vy,
                         const double* R, const double* P, const double* grad_dist,
                         const double* grad_pen, int B, int N, int M, int D, double gamma,
                         double beta, double eps, double* dX, double* dY, double* dvx,
                         double* dvy, double* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  return feat_bwd<double>(X, Y, vx, vy, R, P, grad_dist, grad_pen, B, N, M, D, gamma, beta, eps,
                          dX, dY, dvx, dvy, workspace, workspace_bytes, stream,
                          "tw_udtw_feat_bwd_f64");
}

}  // extern "C"
