// uDTW / soft-DTW dynamic program for gfx950: forward and fused backward.
//
// One workgroup per sequence pair. Thread t owns the ROWS contiguous grid
// rows t*ROWS .. t*ROWS+ROWS-1 and sweeps the anti-diagonals d = i + j with
// its rows' two previous diagonals held in registers. The only cross-thread
// value per diagonal is the last owned row of the previous thread (forward)
// or the first owned row of the next thread (backward): a DPP wave shift
// inside a wavefront, an LDS mailbox between wavefronts. Wavefronts meet at
// an LDS-only barrier once per block of four diagonals.
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
// Column sums (dy, dvy) travel up the rows with their column and are stored
// when the column leaves the sweep, so their order of summation is fixed
// (bitwise deterministic).

#include <limits.h>
#include <type_traits>
#include <stdlib.h>

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
  int sigma;     // VX / VY hold standard deviations: variances are their squares
  T hv1, hv0;    // half variance of an input v: v (hv1 v + hv0)
  int gstride;   // element stride of gr / gp (0: one value for every pair)
};

// Half of a variance input: 0.5 v, or 0.5 v^2 when the input is a standard
// deviation, as v (hv1 v + hv0) with (hv1, hv0) = (0, 0.5) or (0.5, 0).
template <typename T>
__device__ __forceinline__ T half_var(const UdtwArgs<T>& a, T v) {
  return v * (a.hv1 * v + a.hv0);
}

// ------------------------------------------------------------- pipeline
//
// The steps of a sweep are grouped in blocks of kSlots = 4; the wavefronts of
// a workgroup meet at one barrier per block. Wavefront w runs kLag = 4
// diagonals behind wavefront w-1 (forward; behind w+1 in the backward), so
// at step tau it needs its neighbour's boundary record of step tau - 5.
// Every wavefront stores its boundary record of step tau into slot tau % 4 of
// half (tau / 4) % 2 of its neighbour's mailbox. After the barrier that ends
// block k (every LDS operation complete), the neighbour reads the four
// records of block k: steps 4k+5, 4k+6, 4k+7 of block k+1 use the first
// three, the fourth is kept in a register for step 4k+8, the first step of
// block k+2. A half is rewritten two blocks later, after the barrier that
// follows those reads, so no record is overwritten before it is read and the
// reads are issued a whole step before their first use. The store is one
// instruction for the whole wavefront: the lane holding the boundary row
// writes the mailbox slot, the other lanes a private dump area, so no
// exec-mask branch is needed. The edge wavefront makes its own records (the
// border row and the column entering the sweep). A loop trip is one block,
// so mailbox slots, prefetch registers and buffer offsets of a step are
// compile-time constants.
//
// Column values (y and hy = half the column variance) travel with the sweep:
// row i on diagonal d uses column j = d - i, which row i-1 used on diagonal
// d-1, so a row takes its column operands from the row above (forward) or
// below (backward) with the DPP shift that moves R. The backward's column
// gradient sums ride along the same way and are stored when their column
// leaves the sweep at row 0, summed over rows in a fixed order.
//
// Global accesses are raw buffer operations with a lane-constant voffset and
// a wave-uniform, non-negative soffset. The hardware range check covers the
// voffset only; lanes outside the grid pass an out-of-range voffset, so their
// loads return 0 and their stores are dropped without branching. The
// soffsets of 64 consecutive steps are computed once, one step per lane, and
// each step takes its own with v_readlane: no per-step scalar arithmetic.

constexpr int kLag = 4;
constexpr int kSlots = 4;            // steps per block (and per loop trip)
constexpr int kBox = 2 * kSlots;     // mailbox slots per wavefront boundary
constexpr int kDump = 64 + kBox;
constexpr int kWindow = 64;          // steps per soffset window (one per lane)

// Barrier at the end of a block: every LDS operation of this wavefront is
// complete (the block's mailbox stores and the reads of the previous block's
// records), then the workgroup barrier. Outstanding global stores are not
// waited for.
__device__ __forceinline__ void block_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <typename T>
struct alignas(4 * sizeof(T)) Rec4 {
  T x, y, z, w;
};
template <typename T>
struct alignas(4 * sizeof(T)) Rec8 {
  Rec4<T> a, b;
};

// soff(d) = (index of the first cell of diagonal d) - (row of that cell) in
// the diagonal-major layout of an N x M grid, N <= M: cell (i, d - i) is
// element soff(d) + i. Clamped to diagonal 0 below and Dn - 1 above.
__device__ __forceinline__ int diag_soff(int d, int N, int M) {
  d = d < 0 ? 0 : (d > N + M - 2 ? N + M - 2 : d);
  const int lo = d - M + 1 > 0 ? d - M + 1 : 0;
  return (int)(diag_offset(d, N, M) - lo);
}

template <int ROWS>
struct MaxThreads {
  static constexpr int value = ROWS >= 16 ? 1024 : 256;
};

template <typename T, int ROWS, int SRC, bool PEN, bool BAND, int PF>
__global__ void __launch_bounds__(MaxThreads<ROWS>::value) udtw_fwd_kernel(UdtwArgs<T> a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int ES = sizeof(T);
  constexpr bool COLS = SRC != SRC_COST;
  const int N = a.N, M = a.M;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const T INF = inf_v<T>();
  const long long NM = (long long)N * M;
  const int Dn = N + M - 1;

  // box[v * kBox + slot]: wavefront v's inbox (the row above its first
  // row; box[nw] is the last wavefront's unread outbox), then the dump area.
  Rec4<T>* box = reinterpret_cast<Rec4<T>*>(smem_raw);
  Rec4<T>* dump = box + (nw + 1) * kBox;
  const Rec4<T> rec0 = {INF, (T)0, (T)0, (T)0.5};   // the record before the sweep
  for (int t = tid; t < (nw + 1) * kBox; t += blockDim.x) box[t] = rec0;

  Buf bR, bP, bC, bQ, bY, bVY;
  bR.init(a.R + b * NM, NM);
  if (PEN) bP.init(a.P + b * NM, NM);
  if (SRC != SRC_FEAT1) bC.init(a.C + b * NM, NM);
  if (SRC == SRC_COST && PEN) bQ.init(a.Q + b * NM, NM);
  if (SRC == SRC_FEAT1) bY.init(a.Y + (size_t)b * M, M);
  if (COLS) bVY.init(a.VY + (size_t)b * M, M);
  // column operands of the edge wavefront: loads at byte offset vcol (lane
  // uniform); columns past the end fail the range check and read 0
  auto col_y = [&](int vcol) -> T { return SRC == SRC_FEAT1 ? bY.ld<T>(vcol, 0) : (T)0; };
  auto col_vy = [&](int vcol) -> T { return COLS ? bVY.ld<T>(vcol, 0) : (T)1; };

  Rec4<T>* const inbox = box + wave * kBox;
  Rec4<T>* const outbox = box + (wave + 1) * kBox;
  // the mailbox store of a step: lane 63 to the slot, the others to the dump
  Rec4<T>* const my_out = lane == 63 ? outbox : dump + lane;
  __syncthreads();

  const int row0 = tid * ROWS;
  T xr[ROWS], hxr[ROWS], r1[ROWS], r2[ROWS], p1[ROWS], p2[ROWS], yc[ROWS], hyc[ROWS];
  int vst[ROWS], vnat[ROWS], jb[ROWS];
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    const int i = row0 + k;
    xr[k] = (SRC == SRC_FEAT1 && i < N) ? a.X[(size_t)b * N + i] : (T)0;
    hxr[k] = (COLS && i < N) ? half_var(a, a.VX[(size_t)b * N + i]) : (T)0.5;
    r1[k] = r2[k] = INF;
    p1[k] = p2[k] = (T)0;
    yc[k] = (T)0;
    hyc[k] = (T)0.5;
    vst[k] = i * ES;                          // row offset within a diagonal
    vnat[k] = i < N ? i * (M - 1) * ES : 0;   // [N, M] offset of (i, d - i) minus d
    jb[k] = i < N ? -i : INT_MIN / 2;         // column of row i on diagonal d is d + jb
  }
  T nr1 = (tid == 0) ? (T)0 : INF, nr2 = INF, np1 = (T)0, np2 = (T)0;

  const int d_first = -kLag * wave;
  const int steps = (Dn + kLag * (nw - 1) + kSlots - 1) / kSlots * kSlots;

  T rc[PF][ROWS], rq[PF][ROWS];
  // C (and Q) of diagonal d at byte soffset so = max(d, 0) * ES
  auto fetch = [&](int d, int so, T* c, T* q) {
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const int vo = (unsigned)(d + jb[k]) < (unsigned)M ? vnat[k] : kOob;
      c[k] = bC.ld<T>(vo, so);
      if (SRC == SRC_COST && PEN) q[k] = bQ.ld<T>(vo, so);
    }
  };
  if (SRC != SRC_FEAT1) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int d = d_first + u;
      fetch(d, (d > 0 ? d : 0) * ES, rc[u], rq[u]);
    }
  }

  // The sweep, instantiated for the edge wavefront (0: its row above is the
  // border, its entering column comes from a register ring of column loads)
  // and for the others (row above and columns from the mailbox).
  auto sweep = [&](auto edge_tag) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    T ey_ring[kSlots], evy_ring[kSlots];   // EDGE: column d of ring slot d % kSlots
    int vcol = 0;                          // EDGE: byte offset of column t0
    if (EDGE && COLS) {
#pragma unroll
      for (int u = 0; u < kSlots; ++u) {
        ey_ring[u] = col_y(u * ES);
        evy_ring[u] = col_vy(u * ES);
      }
    }
    Rec4<T> carry = rec0;   // the record used by the first step of the next block
    // Drain the set-up loads here: the compiler derives each in-loop wait on
    // a ring register from every path into the loop, and the entry path
    // would otherwise force a near-full vmcnt wait on every trip.
    __builtin_amdgcn_s_waitcnt(0);
    for (int tw = 0; tw < steps; tw += kWindow) {
      // lane l: byte soffsets of step tw + l (R / P store, C / Q fetch)
      const int dl = d_first + tw + lane;
      const int so_st = diag_soff(dl, N, M) * ES;
      const int so_ld = SRC != SRC_FEAT1 ? (dl + PF > 0 ? dl + PF : 0) * ES : 0;
      const int tn = min(kWindow, steps - tw);
    for (int t0 = 0; t0 < tn; t0 += kSlots) {
      const int half = (t0 / kSlots) & 1;   // mailbox half of this block
      Rec4<T> rec[kSlots];
      if (!EDGE) {
        const Rec4<T>* prev = inbox + (half ^ 1) * kSlots;
        rec[0] = carry;
#pragma unroll
        for (int u = 1; u < kSlots; ++u) rec[u] = prev[u - 1];
        carry = prev[kSlots - 1];
      }
      Rec4<T>* const out = my_out + half * kSlots;
#pragma unroll
      for (int u = 0; u < kSlots; ++u) {
        const int d = d_first + tw + t0 + u;
        T cc[ROWS], cq[ROWS];
#pragma unroll
        for (int k = 0; k < ROWS; ++k) {
          cc[k] = rc[u % PF][k];
          cq[k] = rq[u % PF][k];
        }
        // the row above the first row on diagonal d-1, and the column
        // entering the first row on diagonal d
        Rec4<T> e;
        if (EDGE)
          e = {INF, (T)0, ey_ring[u], COLS ? half_var(a, evy_ring[u]) : (T)0.5};
        else
          e = rec[u];

        nr2 = nr1;
        np2 = np1;
        nr1 = shift_prev(r1[ROWS - 1], e.x);
        if (PEN) np1 = EDGE ? shift_prev0(p1[ROWS - 1]) : shift_prev(p1[ROWS - 1], e.y);
        if (COLS) {
          // the edge wavefront's column operands are wave-uniform: passing
          // them through readfirstlane gives each shift a fresh copy, so the
          // ring registers are never tied to (and overwritten by) a shift
          const T ny = SRC != SRC_FEAT1 ? (T)0
                       : shift_prev(yc[ROWS - 1], EDGE ? uniform(e.z) : e.z);
          const T nhy = shift_prev(hyc[ROWS - 1], EDGE ? uniform(e.w) : e.w);
#pragma unroll
          for (int k = ROWS - 1; k > 0; --k) {
            yc[k] = yc[k - 1];
            hyc[k] = hyc[k - 1];
          }
          yc[0] = ny;
          hyc[0] = nhy;
        }

        const int so = __builtin_amdgcn_readlane(so_st, t0 + u);
        T nr[ROWS], np[ROWS];
#pragma unroll
        for (int k = 0; k < ROWS; ++k) {
          const int j = d + jb[k];
          const bool valid = (unsigned)j < (unsigned)M;
          const T up = k ? r1[k - 1] : nr1;
          const T dg = k ? r2[k - 1] : nr2;
          const T lf = r1[k];
          T ch, q = (T)0;
          if (SRC == SRC_COST) {
            ch = cc[k] * a.k;
            if (PEN) q = cq[k];
          } else {
            T sq;
            if (SRC == SRC_FEAT1) {
              const T df = xr[k] - yc[k];
              sq = df * df;
            } else {
              sq = cc[k] > (T)0 ? cc[k] : (T)0;
            }
            const T var = fmax(hxr[k] + hyc[k], a.eps);   // max((vx + vy) / 2, eps)
            ch = sq * (rcp(var) * a.k);
            if (PEN) q = a.beta_ln2 * lg2(var);
          }
          const T m = min3(dg, up, lf);
          const T ed = ex2(m - dg), eu = ex2(m - up), el = ex2(m - lf);
          const T s = ed + eu + el;
          const T rv = ch + m - lg2(s);
          bool ok = valid;
          if (BAND) ok = ok && (m < INF) && (fabs((T)(2 * (row0 + k) - d)) <= a.band);
          nr[k] = ok ? rv : INF;
          if (PEN) {
            const T pup = k ? p1[k - 1] : np1;
            const T pdg = k ? p2[k - 1] : np2;
            const T pv = q + (ed * pdg + eu * pup + el * p1[k]) * rcp(s);
            np[k] = ok ? pv : (T)0;
          } else {
            np[k] = (T)0;
          }
          const int vo = valid ? vst[k] : kOob;
          bR.st(nr[k], vo, so);
          if (PEN) bP.st(np[k], vo, so);
        }
#pragma unroll
        for (int k = 0; k < ROWS; ++k) {
          r2[k] = r1[k];
          r1[k] = nr[k];
          p2[k] = p1[k];
          p1[k] = np[k];
        }
        // The ring reloads are issued after the last use of the slot they
        // refill, so the slot's register is reused in place and the loop back
        // edge needs no copies (nor the waits they imply).
        __builtin_amdgcn_sched_barrier(0);
        if (SRC != SRC_FEAT1)
          fetch(d + PF, __builtin_amdgcn_readlane(so_ld, t0 + u), rc[u % PF], rq[u % PF]);
        if (EDGE && COLS) {
          ey_ring[u] = col_y(vcol + (u + kSlots) * ES);
          evy_ring[u] = col_vy(vcol + (u + kSlots) * ES);
        }
        out[u] = {r1[ROWS - 1], p1[ROWS - 1], yc[ROWS - 1], hyc[ROWS - 1]};
      }
      block_barrier();
      vcol += kSlots * ES;
    }
    }
  };
  if (wave == 0)
    sweep(std::true_type{});
  else
    sweep(std::false_type{});
  // cell (N-1, M-1) is the last element of the diagonal-major R / P; the
  // thread that stored it reads it back
  if (row0 <= N - 1 && N - 1 < row0 + ROWS) {
    const int so = (int)(NM - 1) * ES;
    const T rl = bR.ld<T>(0, so);
    a.out_r[b] = rl < INF ? rl * a.inv_k : INF;
    a.out_p[b] = PEN ? bP.ld<T>(0, so) : (T)0;
  }
}

template <typename T, int ROWS, int SRC, bool PEN, bool BAND, int PF>
__global__ void __launch_bounds__(MaxThreads<ROWS>::value) udtw_bwd_kernel(UdtwArgs<T> a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int ES = sizeof(T);
  constexpr bool COLS = SRC != SRC_COST;
  const int N = a.N, M = a.M;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const T INF = inf_v<T>();
  const long long NM = (long long)N * M;
  const bool vgrad = COLS && a.dVX != nullptr;
  const int Dn = N + M - 1;

  // Rows are bottom-aligned: row N-1 is the last row of the last wavefront,
  // where every column enters the backward sweep.
  const int row0 = tid * ROWS - ((int)blockDim.x * ROWS - N);

  // box[(v + 1) * kBox + slot]: wavefront v's inbox, the row below its last
  // row: (E, G, H, A) and (y, hy, dy sum, dvy sum); box[0..kBox) is
  // wavefront 0's unread outbox. Then the dump area.
  Rec8<T>* box = reinterpret_cast<Rec8<T>*>(smem_raw);
  Rec8<T>* dump = box + (nw + 1) * kBox;
  const Rec8<T> rec0 = {{-INF, (T)0, (T)0, (T)0}, {(T)0, (T)0.5, (T)0, (T)0}};
  for (int t = tid; t < (nw + 1) * kBox; t += blockDim.x) box[t] = rec0;

  Buf bR, bP, bC, bQ, bdC, bdQ, bY, bVY, bdY, bdVY;
  bR.init(a.R + b * NM, NM);
  if (PEN) bP.init(a.P + b * NM, NM);
  if (SRC != SRC_FEAT1) {
    bC.init(a.C + b * NM, NM);
    bdC.init(a.dC + b * NM, NM);
  }
  const bool want_dq = SRC == SRC_COST && PEN && a.dQ != nullptr;
  if (SRC == SRC_COST && PEN) {
    bQ.init(a.Q + b * NM, NM);
    // no penalty gradient wanted: its stores go to an empty buffer (dropped)
    bdQ.init(want_dq ? a.dQ + b * NM : a.Q, want_dq ? NM : 0);
  }
  if (SRC == SRC_FEAT1) {
    bY.init(a.Y + (size_t)b * M, M);
    bdY.init(a.dY + (size_t)b * M, M);
  }
  if (COLS) bVY.init(a.VY + (size_t)b * M, M);
  // without variance gradients the column sums are still formed (no branch in
  // the sweep) and their stores go to an empty buffer, which drops them
  if (COLS) bdVY.init(vgrad ? a.dVY + (size_t)b * M : a.VY, vgrad ? M : 0);
  // column operands of the edge wavefront at byte offset vcol (lane uniform);
  // columns before the first fail the range check and read 0
  auto col_y = [&](int vcol) -> T { return SRC == SRC_FEAT1 ? bY.ld<T>(vcol, 0) : (T)0; };
  auto col_vy = [&](int vcol) -> T { return COLS ? bVY.ld<T>(vcol, 0) : (T)1; };

  const bool last_wave = wave == nw - 1;
  Rec8<T>* const inbox = box + (wave + 1) * kBox;
  Rec8<T>* const outbox = box + wave * kBox;
  Rec8<T>* const my_out = lane == 0 ? outbox : dump + lane;
  __syncthreads();

  T xr[ROWS], hxr[ROWS], dxr[ROWS], dvr[ROWS];
  T e1[ROWS], e2[ROWS], g1[ROWS], g2[ROWS], h1[ROWS], h2[ROWS], a1[ROWS], a2[ROWS];
  T yc[ROWS], hyc[ROWS], cy[ROWS], cvy[ROWS];
  int vst[ROWS], vnat[ROWS], jb[ROWS], vrow0[ROWS];
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    const int i = row0 + k;
    const bool in = i >= 0 && i < N;
    xr[k] = (SRC == SRC_FEAT1 && in) ? a.X[(size_t)b * N + i] : (T)0;
    hxr[k] = (COLS && in) ? half_var(a, a.VX[(size_t)b * N + i]) : (T)0.5;
    dxr[k] = dvr[k] = (T)0;
    e1[k] = e2[k] = -INF;
    g1[k] = g2[k] = h1[k] = h2[k] = a1[k] = a2[k] = (T)0;
    yc[k] = cy[k] = cvy[k] = (T)0;
    hyc[k] = (T)0.5;
    vst[k] = in ? i * ES : 0;
    vnat[k] = in ? i * (M - 1) * ES : 0;
    jb[k] = in ? -i : INT_MIN / 2;
    vrow0[k] = i == 0 ? 0 : kOob;   // the row that stores finished columns
  }
  // Row below the last row on the two previous diagonals. The virtual cell
  // (N, M) on diagonal Dn+1 is given E = Rh(N-1, M-1), A = P(N-1, M-1) and the
  // incoming gradients, so the recursion yields grad_dist / grad_pen at
  // (N-1, M-1) without a special case.
  T ne1 = -INF, ne2 = -INF, ng1 = 0, ng2 = 0, nh1 = 0, nh2 = 0, na1 = 0, na2 = 0;
  if (last_wave && lane == 63) {
    const int so = (int)(NM - 1) * ES;
    ne1 = bR.ld<T>(0, so);
    ng1 = a.gr[(size_t)b * a.gstride];
    if (PEN) {
      nh1 = a.gp[(size_t)b * a.gstride];
      na1 = bP.ld<T>(0, so);
    }
  }

  const int d_first = Dn - 1 + kLag * (nw - 1 - wave);
  const int steps = (Dn + kLag * (nw - 1) + kSlots - 1) / kSlots * kSlots;

  T rr[PF][ROWS], rp[PF][ROWS], rc[PF][ROWS], rq[PF][ROWS];
  // R, P of diagonal d at byte soffset so_d = soff(d) * ES (diagonal-major),
  // C, Q at so_n = max(d, 0) * ES ([N, M])
  auto fetch = [&](int d, int so_d, int so_n, T* r, T* p, T* c, T* q) {
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const bool v = (unsigned)(d + jb[k]) < (unsigned)M;
      const int vd = v ? vst[k] : kOob;
      r[k] = bR.ld<T>(vd, so_d);
      if (PEN) p[k] = bP.ld<T>(vd, so_d);
      if (SRC != SRC_FEAT1) {
        const int vn = v ? vnat[k] : kOob;
        c[k] = bC.ld<T>(vn, so_n);
        if (SRC == SRC_COST && PEN) q[k] = bQ.ld<T>(vn, so_n);
      }
    }
  };
#pragma unroll
  for (int u = 0; u < PF; ++u) {
    const int d = d_first - u;
    fetch(d, diag_soff(d, N, M) * ES, (d > 0 ? d : 0) * ES, rr[u], rp[u], rc[u], rq[u]);
  }

  // The sweep, instantiated for the edge wavefront (the last: its row below
  // is the virtual row N, its entering column comes from a register ring of
  // column loads) and for the others (row below and columns from the mailbox).
  auto sweep = [&](auto edge_tag) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    // EDGE: ring slot u of a trip holds column M-1-t0-u, the one entering row
    // N-1 on that step's diagonal
    T ey_ring[kSlots], evy_ring[kSlots];
    int vcol = (M - 1) * ES;   // EDGE: byte offset of column M-1-t0
    if (EDGE && COLS) {
#pragma unroll
      for (int u = 0; u < kSlots; ++u) {
        ey_ring[u] = col_y(vcol - u * ES);
        evy_ring[u] = col_vy(vcol - u * ES);
      }
    }
    Rec8<T> carry = rec0;   // the record used by the first step of the next block
    __builtin_amdgcn_s_waitcnt(0);   // drain the set-up loads (as in the forward)
    for (int tw = 0; tw < steps; tw += kWindow) {
      // lane l: byte soffsets of step tw + l (fetch of R / P and C / Q, and
      // the stores of the step's own diagonal)
      const int dl = d_first - tw - lane;
      const int so_fd = diag_soff(dl - PF, N, M) * ES;
      const int so_fn = SRC != SRC_FEAT1 ? (dl - PF > 0 ? dl - PF : 0) * ES : 0;
      const int so_st = (dl > 0 ? dl : 0) * ES;
      const int tn = min(kWindow, steps - tw);
    for (int t0 = 0; t0 < tn; t0 += kSlots) {
      const int half = (t0 / kSlots) & 1;   // mailbox half of this block
      Rec8<T> rec[kSlots];
      if (!EDGE) {
        const Rec8<T>* prev = inbox + (half ^ 1) * kSlots;
        rec[0] = carry;
#pragma unroll
        for (int u = 1; u < kSlots; ++u) {
          rec[u].a = prev[u - 1].a;
          if (COLS) rec[u].b = prev[u - 1].b;
        }
        carry.a = prev[kSlots - 1].a;
        if (COLS) carry.b = prev[kSlots - 1].b;
      }
      Rec8<T>* const out = my_out + half * kSlots;
#pragma unroll
      for (int u = 0; u < kSlots; ++u) {
        const int d = d_first - tw - t0 - u;
        T cr[ROWS], cp[ROWS], cc[ROWS], cq[ROWS];
  #pragma unroll
        for (int k = 0; k < ROWS; ++k) {
          cr[k] = rr[u % PF][k];
          cp[k] = rp[u % PF][k];
          cc[k] = rc[u % PF][k];
          cq[k] = rq[u % PF][k];
        }
        // the row below the last row on diagonal d+1, and the column entering
        // the last row on diagonal d
        Rec8<T> ex;
        if (EDGE)
          ex = {{-INF, (T)0, (T)0, (T)0},
                {ey_ring[u], COLS ? half_var(a, evy_ring[u]) : (T)0.5, (T)0, (T)0}};
        else
          ex = rec[u];

        ne2 = ne1;
        ng2 = ng1;
        nh2 = nh1;
        na2 = na1;
        ne1 = shift_next(e1[0], ex.a.x);
        ng1 = EDGE ? shift_next0(g1[0]) : shift_next(g1[0], ex.a.y);
        if (PEN) {
          nh1 = EDGE ? shift_next0(h1[0]) : shift_next(h1[0], ex.a.z);
          na1 = EDGE ? shift_next0(a1[0]) : shift_next(a1[0], ex.a.w);
        }
        if (COLS) {
          const T fy = SRC != SRC_FEAT1 ? (T)0
                       : shift_next(yc[0], EDGE ? uniform(ex.b.x) : ex.b.x);
          const T fhy = shift_next(hyc[0], EDGE ? uniform(ex.b.y) : ex.b.y);
          const T fcy = SRC != SRC_FEAT1 ? (T)0 : EDGE ? shift_next0(cy[0]) : shift_next(cy[0], ex.b.z);
          const T fcvy = EDGE ? shift_next0(cvy[0]) : shift_next(cvy[0], ex.b.w);
  #pragma unroll
          for (int k = 0; k + 1 < ROWS; ++k) {
            yc[k] = yc[k + 1];
            hyc[k] = hyc[k + 1];
            cy[k] = cy[k + 1];
            cvy[k] = cvy[k + 1];
          }
          yc[ROWS - 1] = fy;
          hyc[ROWS - 1] = fhy;
          cy[ROWS - 1] = fcy;
          cvy[ROWS - 1] = fcvy;
        }

        const int so_n = __builtin_amdgcn_readlane(so_st, t0 + u);
        T xe[ROWS], xg[ROWS], xh[ROWS], xa[ROWS];
  #pragma unroll
        for (int k = 0; k < ROWS; ++k) {
          const bool valid = (unsigned)(d + jb[k]) < (unsigned)M;
          const T rk = valid ? cr[k] : INF;
          const T pk = cp[k];
          T ch, q = (T)0, c = (T)0, rv = (T)1, sq_raw = (T)0, var_raw = (T)1;
          if (SRC == SRC_COST) {
            ch = cc[k] * a.k;
            if (PEN) q = cq[k];
          } else {
            if (SRC == SRC_FEAT1) {
              const T df = xr[k] - yc[k];
              sq_raw = df * df;
            } else {
              sq_raw = cc[k];
            }
            const T sq = sq_raw > (T)0 ? sq_raw : (T)0;
            var_raw = hxr[k] + hyc[k];
            const T var = fmax(var_raw, a.eps);
            rv = rcp(var);
            c = sq * rv;
            ch = c * a.k;
            if (PEN) q = a.beta_ln2 * lg2(var);
          }
          // successors: down (i+1, j) and right (i, j+1) on d+1, diagonal (i+1, j+1) on d+2
          const T edn = (k + 1 < ROWS) ? e1[k + 1] : ne1;
          const T gdn = (k + 1 < ROWS) ? g1[k + 1] : ng1;
          const T edg = (k + 1 < ROWS) ? e2[k + 1] : ne2;
          const T gdg = (k + 1 < ROWS) ? g2[k + 1] : ng2;
          const T wdn = ex2(edn - rk), wrt = ex2(e1[k] - rk), wdg = ex2(edg - rk);
          T g = wdn * gdn + wrt * g1[k] + wdg * gdg;
          T h = (T)0;
          if (PEN) {
            const T hdn = (k + 1 < ROWS) ? h1[k + 1] : nh1;
            const T adn = (k + 1 < ROWS) ? a1[k + 1] : na1;
            const T hdg = (k + 1 < ROWS) ? h2[k + 1] : nh2;
            const T adg = (k + 1 < ROWS) ? a2[k + 1] : na2;
            const T wh_dn = wdn * hdn, wh_rt = wrt * h1[k], wh_dg = wdg * hdg;
            g -= (wh_dn * (pk - adn) + wh_rt * (pk - a1[k]) + wh_dg * (pk - adg)) * a.inv_gamma;
            h = wh_dn + wh_rt + wh_dg;
          }
          // outside the grid, and (band) at unreachable cells, nothing flows
          bool live = valid;
          if (BAND) live = live && rk < INF;
          g = live ? g : (T)0;
          h = live ? h : (T)0;
          xe[k] = live ? rk - ch : -INF;
          xg[k] = g;
          xh[k] = h;
          xa[k] = valid ? pk - q : (T)0;

          const int vn = valid ? vnat[k] : kOob;
          if (SRC == SRC_COST) {
            bdC.st(g, vn, so_n);
            if (PEN) bdQ.st(h, vn, so_n);
          } else {
            const T dsq = sq_raw > (T)0 ? g * rv : (T)0;
            if (SRC == SRC_SQ) bdC.st(dsq, vn, so_n);
            if (SRC == SRC_FEAT1) {
              const T df = valid ? (T)2 * dsq * (xr[k] - yc[k]) : (T)0;
              dxr[k] += df;
              cy[k] -= df;
            }
            {
              T dvar = var_raw > a.eps ? (T)0.5 * (a.beta * h - g * c) * rv : (T)0;
              dvar = valid ? dvar : (T)0;
              dvr[k] += dvar;
              cvy[k] += dvar;
            }
            // column d leaves the sweep at row 0: store its sums
            const int vc = ((unsigned)d < (unsigned)M) ? vrow0[k] : kOob;
            if (SRC == SRC_FEAT1) bdY.st(cy[k], vc, so_n);
            bdVY.st(cvy[k], vc, so_n);
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
        // ring reloads only now (see the forward)
        __builtin_amdgcn_sched_barrier(0);
        fetch(d - PF, __builtin_amdgcn_readlane(so_fd, t0 + u),
              __builtin_amdgcn_readlane(so_fn, t0 + u), rr[u % PF], rp[u % PF], rc[u % PF],
              rq[u % PF]);
        if (EDGE && COLS) {
          ey_ring[u] = col_y(vcol - (u + kSlots) * ES);
          evy_ring[u] = col_vy(vcol - (u + kSlots) * ES);
        }
        if (COLS) {
          out[u] = {{e1[0], g1[0], h1[0], a1[0]}, {yc[0], hyc[0], cy[0], cvy[0]}};
        } else {
          out[u].a = {e1[0], g1[0], h1[0], a1[0]};
        }
      }
      block_barrier();
      vcol -= kSlots * ES;
    }
    }
  };
  if (last_wave)
    sweep(std::true_type{});
  else
    sweep(std::false_type{});
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    const int i = row0 + k;
    if (i >= 0 && i < N) {
      if (SRC == SRC_FEAT1) a.dX[(size_t)b * N + i] = dxr[k];
      if (vgrad) a.dVX[(size_t)b * N + i] = dvr[k];
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
  // tuning override: TORCHWARP_UDTW_ROWS = 1, 2, 4, 8 or 16 rows per thread,
  // taken when the kernel's thread limit for that row count allows it
  static const int forced = [] {
    const char* e = getenv("TORCHWARP_UDTW_ROWS");
    return e ? atoi(e) : 0;
  }();
  if ((forced == 1 || forced == 2 || forced == 4 || forced == 8 || forced == 16) &&
      (N + forced - 1) / forced <= (forced >= 16 ? 1024 : 256))
    rows = forced;
  int threads = (N + rows - 1) / rows;
  if (threads > 1024) return {0, 0};
  threads = ((threads + 63) / 64) * 64;
  return {rows, threads};
}

// LDS of one workgroup: the mailbox rings and the dump area of the
// mailbox stores (records of 4 values forward, 8 backward).
template <typename T>
static size_t udtw_lds(bool backward, int nw) {
  return (size_t)((nw + 1) * kBox + kDump) * (backward ? 8 : 4) * sizeof(T);
}

// Prefetch depth (diagonals) of the register ring for a row count.
template <int ROWS>
struct PrefetchDepth {
  static constexpr int value = ROWS == 1 ? 4 : (ROWS == 2 ? 2 : 1);
};

template <typename T, int SRC, bool PEN, bool BAND>
static int launch_udtw(bool backward, const UdtwArgs<T>& a, int B, hipStream_t stream,
                       const char* what) {
  if (B == 0) return TW_OK;
  const Shape sh = pick_shape(a.N);
  if (sh.rows == 0) {
    return fail(TW_ESIZE, "%s: the shorter sequence has %d steps; this build handles up to 16384",
                what, a.N);
  }
  if ((long long)a.N * a.M * (long long)sizeof(T) >= (1LL << 31)) {
    return fail(TW_ESIZE, "%s: one pair's N*M matrix must stay below 2 GiB", what);
  }
  const int nw = sh.threads / 64;
  const size_t lds = udtw_lds<T>(backward, nw);
  if (lds > (size_t)max_lds_bytes()) {
    return fail(TW_ESIZE, "%s: %zu bytes of LDS needed, %d available", what, lds,
                max_lds_bytes());
  }
  dim3 grid(B), block(sh.threads);
#define TW_UDTW_CASE(R_)                                                                     \
  case R_:                                                                                   \
    if (backward)                                                                            \
      hipLaunchKernelGGL(                                                                    \
          (udtw_bwd_kernel<T, R_, SRC, PEN, BAND, PrefetchDepth<R_>::value>), grid, block,   \
          lds, stream, a);                                                                   \
    else                                                                                     \
      hipLaunchKernelGGL(                                                                    \
          (udtw_fwd_kernel<T, R_, SRC, PEN, BAND, PrefetchDepth<R_>::value>), grid, block,   \
          lds, stream, a);                                                                   \
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
  const bool band = a.band > (T)0;
  if (pen)
    return band ? launch_udtw<T, SRC, true, true>(backward, a, B, s, what)
                : launch_udtw<T, SRC, true, false>(backward, a, B, s, what);
  return band ? launch_udtw<T, SRC, false, true>(backward, a, B, s, what)
              : launch_udtw<T, SRC, false, false>(backward, a, B, s, what);
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
                    double gamma, double beta, double eps, double band, int sigma, T* R, T* P,
                    T* out_r, T* out_p, T* ws, size_t ws_bytes, hipStream_t s,
                    const char* what) {
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

// d sigma = 2 sigma d var, in place over the variance gradients of both sides
template <typename T>
__global__ void __launch_bounds__(256) sigma_grad_kernel(const T* __restrict__ sx,
                                                         const T* __restrict__ sy, T* dsx, T* dsy,
                                                         long long nx, long long ny) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < nx)
    dsx[i] *= (T)2 * sx[i];
  else if (i < nx + ny)
    dsy[i - nx] *= (T)2 * sy[i - nx];
}

template <typename T>
static int sigma_grads(const T* sx, const T* sy, T* dsx, T* dsy, long long nx, long long ny,
                       hipStream_t s, const char* what) {
  const long long n = nx + ny;
  hipLaunchKernelGGL((sigma_grad_kernel<T>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     sx, sy, dsx, dsy, nx, ny);
  return check_launch(what);
}

template <typename T>
static int feat_bwd(const T* X, const T* Y, const T* vx, const T* vy, const T* R, const T* P,
                    const T* gr, const T* gp, int B, int N, int M, int D, double gamma,
                    double beta, double eps, double band, int sigma, int gstride, T* dX, T* dY,
                    T* dvx, T* dvy, T* ws, size_t ws_bytes, hipStream_t s, const char* what) {
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
  if (gstride != 0 && gstride != 1) return fail(TW_EINVAL, "%s: grad_stride must be 0 or 1", what);
  a.gstride = gstride;
  set_hyper(a, gamma, beta, eps, band);
  set_sigma(a, sigma);
  const bool sig_grads = sigma && dvx != nullptr;
  if (D == 1) {
    a.X = X;
    a.Y = Y;
    a.dX = dX;
    a.dY = dY;
    if (int e = launch_pen<T, SRC_FEAT1>(pen, true, a, B, s, what)) return e;
    return sig_grads ? sigma_grads<T>(vx, vy, dvx, dvy, (long long)B * N, (long long)B * M, s, what)
                     : TW_OK;
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
  if (int e = sqdist_raw_bwd<T>(X, Y, ws, B, N, M, D, dX, dY, s, what)) return e;
  return sig_grads ? sigma_grads<T>(vx, vy, dvx, dvy, (long long)B * N, (long long)B * M, s, what)
                   : TW_OK;
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
                         float* dX, float* dY, float* dvx, float* dvy, float* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  return feat_bwd<float>(X, Y, vx, vy, R, P, grad_dist, grad_pen, B, N, M, D, gamma, beta, eps,
                         bandwidth, sigma, grad_stride, dX, dY, dvx, dvy, workspace,
                         workspace_bytes, stream, "tw_udtw_feat_bwd_f32");
}

int tw_udtw_feat_bwd_f64(const double* X, const double* Y, const double* vx, const double* vy,
                         const double* R, const double* P, const double* grad_dist,
                         const double* grad_pen, int B, int N, int M, int D, double gamma,
                         double beta, double eps, double bandwidth, int sigma, int grad_stride,
                         double* dX, double* dY, double* dvx, double* dvy, double* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  return feat_bwd<double>(X, Y, vx, vy, R, P, grad_dist, grad_pen, B, N, M, D, gamma, beta, eps,
                          bandwidth, sigma, grad_stride, dX, dY, dvx, dvy, workspace,
                          workspace_bytes, stream, "tw_udtw_feat_bwd_f64");
}

}  // extern "C"
