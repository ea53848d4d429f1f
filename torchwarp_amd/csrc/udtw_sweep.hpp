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
//   SRC_SQ    raw squared distance S = x2+y2-2x.y [B, N*M] diagonal-major
//             (as R, so every diagonal's access is coalesced) and variances
//             vx [B,N], vy [B,M]: C = max(S,0)/max((vx+vy)/2,eps),
//             Q = beta ln max(...)                      -> writes dS (same layout), dvx, dvy
//   SRC_FEAT1 one feature per step, x [B,N], y [B,M] and variances,
//             C from (x-y)^2 in registers               -> writes dx, dy, dvx, dvy
// Column sums (dy, dvy) travel up the rows with their column and are stored
// when the column leaves the sweep, so their order of summation is fixed
// (bitwise deterministic).

#pragma once

#include <limits.h>
#include <stdlib.h>
#include <type_traits>

#include "tw_capi.hpp"
#include "tw_common.hpp"

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
  int groups;    // forward with MW: row groups (workgroups) per pair
  unsigned int* status;   // MW: per-device status word (TW_STATUS_WAIT_GAVE_UP)
  int spins;              // MW: poll rounds of a boundary-row wait (a test's limit)
  unsigned long long wait_ticks;   // MW: time limit of a wait, device real-time ticks
  int drop_handoff;       // MW test hook: boundary rows are never handed over
  int rd;                 // float: carry R in double precision (the RD kernels)
  unsigned long long* hand;   // backward with MW: boundary hand-off records
};

// Half of a variance input: 0.5 v, or 0.5 v^2 when the input is a standard
// deviation, as v (hv1 v + hv0) with (hv1, hv0) = (0, 0.5) or (0.5, 0).
template <typename T>
__device__ __forceinline__ T half_var(const UdtwArgs<T>& a, T v) {
  return v * fma(a.hv1, v, a.hv0);
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

// Several workgroups per pair (MW, forward only): workgroup g of a pair owns
// rows [256 g, 256 g + 256), four wavefronts of one row per thread, one
// wavefront per SIMD where the batch leaves CUs idle. Its first wavefront
// takes the row above (row 256 g - 1, the previous workgroup's last) from
// the R / P planes: a fill kernel first writes the sentinel into those rows,
// the producing lane stores each cell a second time with an agent-scope
// relaxed atomic store, and at the start of every 64-step window lane l of
// the consumer polls the cell of step l with agent-scope atomic loads until
// no valid lane holds the sentinel. Each cell is its own flag, so no fence
// or cache write-back is needed, on any XCD. Workgroup g runs kGroupLag
// diagonals behind g - 1's first wavefront: its last wavefront's lag plus a
// window and the HBM round trip, so the polls rarely wait once the pipeline
// of a pair's groups has filled (a group whose rows have no cells yet on a
// diagonal steps through it quickly and then waits for the groups below it:
// the first wait of the last of G groups lasts about G times a few hundred
// steps). The waited-on workgroup always has the lower index, so in-order
// dispatch guarantees progress, and every wait is bounded in time by the
// device's real-time counter (kMwWaitSeconds; a test can bound it by a few
// poll rounds instead). A wait that runs out sets TW_STATUS_WAIT_GAVE_UP in
// the device's status word and lets the sentinel (a NaN) flow on into the
// pair's outputs, so the kernel still exits and tw_async_status reports it.
constexpr int kMwRows = 256;
constexpr int kGroupLag = kLag * (kMwRows / 64) + kWindow + 16;
constexpr int kMwSpins = 0x7FFFFFFF;
constexpr double kMwWaitSeconds = 2.0;
// True when a wait that began at tick t0 has polled `spin + 1` rounds out of
// a.spins, or has lasted longer than a.wait_ticks (wave-uniform).
template <typename T>
__device__ __forceinline__ bool wait_ran_out(const UdtwArgs<T>& a, int spin,
                                             unsigned long long t0) {
  return spin + 1 >= a.spins || __builtin_amdgcn_s_memrealtime() - t0 > a.wait_ticks;
}
__host__ __device__ constexpr unsigned long long mw_sentinel_bits(int es) {
  return es == 4 ? 0x7FC0DEADull : 0x7FF8DEADDEADDEADull;
}
// Lane l's value of v, wave-uniform.
__device__ __forceinline__ float lane_val(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double lane_val(double v, int l) {
  const long long x = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)x, l);
  const int hi = __builtin_amdgcn_readlane((int)(x >> 32), l);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
template <typename T>
__device__ __forceinline__ bool mw_is_sentinel(T v) {
  if constexpr (sizeof(T) == 4)
    return __float_as_uint(v) == (unsigned)mw_sentinel_bits(4);
  else
    return (unsigned long long)__double_as_longlong(v) == mw_sentinel_bits(8);
}

// Backward hand-off records (MW): the top row of a row group hands the group
// above its (E, Rbar, Pbar, A) and the column gradient sums (dy, dvy) of
// every diagonal, as 64-bit words stored with agent-scope atomics into a
// caller workspace pre-filled with kHandSentinel (never a value a record
// holds: two NaNs with a fixed payload). Floats are packed two per word;
// with R in double (RD) E takes a word of its own. Per cell
// hand_words(element size) words are reserved (4 for float, 6 for double).
constexpr unsigned long long kHandSentinel = 0x7FF8DEAD7FC0DEADull;
__host__ __device__ constexpr int hand_words(int es) { return es == 4 ? 4 : 6; }
__device__ __forceinline__ unsigned long long pack_ff(float lo, float hi) {
  return (unsigned long long)__float_as_uint(lo) | ((unsigned long long)__float_as_uint(hi) << 32);
}
__device__ __forceinline__ float word_lo(unsigned long long w) { return __uint_as_float((unsigned)w); }
__device__ __forceinline__ float word_hi(unsigned long long w) {
  return __uint_as_float((unsigned)(w >> 32));
}
__device__ __forceinline__ unsigned long long word_d(double v) {
  return (unsigned long long)__double_as_longlong(v);
}
__device__ __forceinline__ double word_to_d(unsigned long long w) {
  return __longlong_as_double((long long)w);
}
// Words in use per record for T (float / double) and RD.
template <typename T, bool RD>
struct HandRec {
  static constexpr int words = sizeof(T) == 8 ? 6 : (RD ? 4 : 3);
};

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
// Records of the RD kernels (float values; R / E and P / A in double).
struct alignas(8) RecD4 {   // forward: R (double), P, y, hy
  double x;
  float y, z, w;
};
struct alignas(8) RecDA {   // backward: E (double), Rbar, Pbar, A
  double x;
  float y, z, w;
};
struct alignas(16) RecD8 {
  RecDA a;
  Rec4<float> b;
};
// Mailbox record types of a forward / backward sweep.
template <typename T, bool RD>
using FwdRec = std::conditional_t<RD, RecD4, Rec4<T>>;
template <typename T, bool RD>
using BwdRec = std::conditional_t<RD, RecD8, Rec8<T>>;

// soff(d) = (index of the first cell of diagonal d) - (row of that cell) in
// the diagonal-major layout of an N x M grid, N <= M: cell (i, d - i) is
// element soff(d) + i. Clamped to diagonal 0 below and Dn - 1 above.
__device__ __forceinline__ int diag_soff(int d, int N, int M) {
  d = d < 0 ? 0 : (d > N + M - 2 ? N + M - 2 : d);
  const int lo = d - M + 1 > 0 ? d - M + 1 : 0;
  return (int)(diag_offset(d, N, M) - lo);
}

// Column operands staged in LDS (one row per thread, up to 256 rows): entry
// kColPad + j holds column j's (y, hy), and the kColPad entries on either
// side hold (0, 0.5), so every row reads its own column on every diagonal
// of the sweep (columns -kColPad .. M + kColPad - 1) without a bounds check.
template <typename T>
struct alignas(2 * sizeof(T)) ColRec {
  T y, hy;
};
__host__ __device__ __forceinline__ int col_pad(int N, int nw) {
  return 64 * nw + N + kLag * nw + 8;
}

// Threads per workgroup a kernel is compiled for. One row per thread with
// the columns travelling by DPP (no LDS columns) serves long sequences with
// up to 16 wavefronts (8 in float64, whose backward needs ~180 VGPRs), so a
// SIMD holds several of the pair's wavefronts and hides their waits: at
// N = M = 1024 the sweeps take 0.93 / 1.76 ms against 1.28 / 2.24 ms with
// 4 rows per thread and one wavefront per SIMD.
template <typename T, int ROWS, bool LC, bool BWD, bool MW = false>
struct MaxThreads {
  static constexpr int value =
      MW ? 256 : ROWS >= 16 ? 1024 : ((ROWS == 1 && !LC) ? (sizeof(T) == 4 ? 1024 : 512) : 256);
};

// LC (one row per thread): the column operands come from LDS (ColRec);
// otherwise they travel down the rows with the DPP shifts that move R.
template <typename T, int ROWS, int SRC, bool PEN, bool BAND, int PF, bool LC, bool MW = false,
          bool RD = false>
__global__ void __launch_bounds__((MaxThreads<T, ROWS, LC, false, MW>::value)) udtw_fwd_kernel(UdtwArgs<T> a) {
  // Products and sums are fused only where written as fma: the edge and the
  // other wavefronts, and every launch layout, then evaluate a cell alike.
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int ES = sizeof(T);
  // RT: the type R is carried in (registers, mailboxes, the R plane)
  using RT = std::conditional_t<RD, double, T>;
  constexpr int RES = sizeof(RT);
  static_assert(!RD || (sizeof(T) == 4 && ROWS == 1), "RD: float, one row per thread");
  const RT RINF = inf_v<RT>();
  constexpr bool COLS = SRC != SRC_COST;
  constexpr bool FLOW = COLS && !LC;
  static_assert(!LC || (COLS && ROWS == 1), "LDS columns need one row per thread");
  static_assert(!MW || (ROWS == 1 && !LC), "MW: one row per thread");
  const int N = a.N, M = a.M;
  // MW: pair b, row group grp of G, rows from rbase
  const int G = MW ? a.groups : 1;
  const int b = MW ? (int)blockIdx.x / G : (int)blockIdx.x;
  const int grp = MW ? (int)blockIdx.x % G : 0;
  const int rbase = grp * kMwRows;
  const int tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const T INF = inf_v<T>();
  const long long NM = (long long)N * M;
  const int Dn = N + M - 1;
  // MW: this workgroup's last wavefront publishes its last row (not the last group's)
  const bool publish = MW && grp < G - 1 && wave == nw - 1;
  // MW test hook: the published row is not stored at all (its wait gives up)
  const bool drop_row = publish && lane == 63 && a.drop_handoff;

  // box[v * kBox + slot]: wavefront v's inbox (the row above its first
  // row; box[nw] is the last wavefront's unread outbox), then the dump area.
  using Rec = FwdRec<T, RD>;
  Rec* box = reinterpret_cast<Rec*>(smem_raw);
  Rec* dump = box + (nw + 1) * kBox;
  const Rec rec0 = {RINF, (T)0, (T)0, (T)0.5};   // the record before the sweep
  for (int t = tid; t < (nw + 1) * kBox; t += blockDim.x) box[t] = rec0;
  ColRec<T>* cols = reinterpret_cast<ColRec<T>*>(dump + kDump);
  const int cpad = col_pad(N, nw);
  if (LC) {
    for (int t = tid; t < M + 2 * cpad; t += blockDim.x) {
      const int j = t - cpad;
      ColRec<T> c = {(T)0, (T)0.5};
      if (j >= 0 && j < M) {
        if (SRC == SRC_FEAT1) c.y = a.Y[(size_t)b * M + j];
        c.hy = half_var(a, a.VY[(size_t)b * M + j]);
      }
      cols[t] = c;
    }
  }

  Buf bR, bP, bC, bQ, bY, bVY;
  RT* const Rpl = reinterpret_cast<RT*>(a.R);   // the R planes ([B, N*M] of RT)
  bR.init(Rpl + b * NM, NM);
  if (PEN) bP.init(a.P + b * NM, NM);
  if (SRC != SRC_FEAT1) bC.init(a.C + b * NM, NM);
  if (SRC == SRC_COST && PEN) bQ.init(a.Q + b * NM, NM);
  if (SRC == SRC_FEAT1 && FLOW) bY.init(a.Y + (size_t)b * M, M);
  if (FLOW) bVY.init(a.VY + (size_t)b * M, M);
  // column operands of the edge wavefront: loads at byte offset vcol (lane
  // uniform); columns past the end fail the range check and read 0
  auto col_y = [&](int vcol) -> T { return SRC == SRC_FEAT1 ? bY.ld<T>(vcol, 0) : (T)0; };
  auto col_vy = [&](int vcol) -> T { return FLOW ? bVY.ld<T>(vcol, 0) : (T)1; };

  Rec* const inbox = box + wave * kBox;
  Rec* const outbox = box + (wave + 1) * kBox;
  // the mailbox store of a step: lane 63 to the slot, the others to the dump
  Rec* const my_out = lane == 63 ? outbox : dump + lane;
  __syncthreads();

  const int row0 = rbase + tid * ROWS;
  T xr[ROWS], hxr[ROWS], p1[ROWS], p2[ROWS], yc[ROWS], hyc[ROWS];
  RT r1[ROWS], r2[ROWS];
  int vst[ROWS], vsr[ROWS], vnat[ROWS], jb[ROWS];
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    const int i = row0 + k;
    xr[k] = (SRC == SRC_FEAT1 && i < N) ? a.X[(size_t)b * N + i] : (T)0;
    hxr[k] = (COLS && i < N) ? half_var(a, a.VX[(size_t)b * N + i]) : (T)0.5;
    r1[k] = r2[k] = RINF;
    p1[k] = p2[k] = (T)0;
    yc[k] = (T)0;
    hyc[k] = (T)0.5;
    vst[k] = i * ES;                          // row offset within a diagonal
    vsr[k] = i * RES;                         // the same in the R plane
    vnat[k] = i < N ? i * (M - 1) * ES : 0;   // [N, M] offset of (i, d - i) minus d
    jb[k] = i < N ? -i : INT_MIN / 2;         // column of row i on diagonal d is d + jb
  }
  RT nr1 = (row0 == 0) ? (RT)0 : RINF, nr2 = RINF;
  T np1 = (T)0, np2 = (T)0;

  const int d_first = -kLag * wave - (MW ? kGroupLag * grp : 0);
  const int steps =
      (Dn + kLag * (nw - 1) + (MW ? kGroupLag * (G - 1) : 0) + kSlots - 1) / kSlots * kSlots;

  T rc[PF][ROWS], rq[PF][ROWS];
  // C (and Q) of diagonal d at byte soffset so: max(d, 0) * ES in the [N, M]
  // layout, soff(d) * ES in the diagonal-major one (SRC_SQ)
  constexpr bool DG = SRC == SRC_SQ;
  auto fetch_so = [&](int d) { return DG ? diag_soff(d, N, M) * ES : (d > 0 ? d : 0) * ES; };
  auto fetch = [&](int d, int so, T* c, T* q) {
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const int vo = (unsigned)(d + jb[k]) < (unsigned)M ? (DG ? vst[k] : vnat[k]) : kOob;
      c[k] = bC.ld<T>(vo, so);
      if (SRC == SRC_COST && PEN) q[k] = bQ.ld<T>(vo, so);
    }
  };
  // VEC (cost in the [N, M] layout): a row's cells on the kSlots diagonals
  // of a block are consecutive in memory, so each lane loads them with one
  // 16-byte load per plane, a block ahead (into cn / qn, copied into the
  // ring at the block's start), instead of one 4-byte load per step: the
  // lanes' rows are M apart, so every load touches one cache line per lane.
  // Cells off the row read another row's or no data; the sweep masks them.
  constexpr bool VEC = SRC == SRC_COST && PF == kSlots;
  T cn[kSlots][ROWS], qn[kSlots][ROWS];
  auto fetch4 = [&](int d, T (*c)[ROWS], T (*q)[ROWS]) {
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const int vo = vnat[k] + d * ES;   // cell (i, d - i) and the next three
#pragma unroll
      for (int h = 0; h < (int)sizeof(T) / 4; ++h) {
        const unsigned int __attribute__((ext_vector_type(4))) w =
            __builtin_amdgcn_raw_buffer_load_b128(bC.r, vo + 16 * h, 0, 0);
        unsigned int __attribute__((ext_vector_type(4))) z = {0, 0, 0, 0};
        if (PEN) z = __builtin_amdgcn_raw_buffer_load_b128(bQ.r, vo + 16 * h, 0, 0);
        if constexpr (sizeof(T) == 4) {
          c[0][k] = __uint_as_float(w.x); c[1][k] = __uint_as_float(w.y);
          c[2][k] = __uint_as_float(w.z); c[3][k] = __uint_as_float(w.w);
          q[0][k] = __uint_as_float(z.x); q[1][k] = __uint_as_float(z.y);
          q[2][k] = __uint_as_float(z.z); q[3][k] = __uint_as_float(z.w);
        } else {
          auto dbl = [](unsigned lo, unsigned hi) {
            return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
          };
          c[2 * h][k] = dbl(w.x, w.y); c[2 * h + 1][k] = dbl(w.z, w.w);
          q[2 * h][k] = dbl(z.x, z.y); q[2 * h + 1][k] = dbl(z.z, z.w);
        }
      }
    }
  };
  if (VEC) {
    fetch4(d_first, cn, qn);
  } else if (SRC != SRC_FEAT1) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int d = d_first + u;
      fetch(d, fetch_so(d), rc[u], rq[u]);
    }
  }

  // The sweep, instantiated for the edge wavefront (0: its row above is the
  // border, its entering column comes from a register ring of column loads)
  // and for the others (row above and columns from the mailbox).
  auto sweep = [&](auto edge_tag) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    T ey_ring[kSlots], evy_ring[kSlots];   // EDGE: column d of ring slot d % kSlots
    // EDGE: byte offset of the column entering row rbase on the block's first
    // diagonal (negative before the grid: those loads fail the range check)
    int vcol = (d_first - rbase) * ES;
    if (EDGE && FLOW) {
#pragma unroll
      for (int u = 0; u < kSlots; ++u) {
        ey_ring[u] = col_y(vcol + u * ES);
        evy_ring[u] = col_vy(vcol + u * ES);
      }
    }
    // LC: this row's column entry on diagonal d is crow[d]; step u of a block
    // uses creg[u % 2] and reads the next step's into the other one
    const ColRec<T>* const crow = cols + cpad - row0;
    ColRec<T> creg[2];
    if (LC) creg[0] = crow[d_first];
    Rec carry = rec0;   // the record used by the first step of the next block
    // Drain the set-up loads here: the compiler derives each in-loop wait on
    // a ring register from every path into the loop, and the entry path
    // would otherwise force a near-full vmcnt wait on every trip.
    __builtin_amdgcn_s_waitcnt(0);
    for (int tw = 0; tw < steps; tw += kWindow) {
      // lane l: byte soffsets of step tw + l (R / P store, C / Q fetch)
      const int dl = d_first + tw + lane;
      const int so_st = diag_soff(dl, N, M) * ES;
      const int so_ld = SRC != SRC_FEAT1 ? fetch_so(dl + PF) : 0;
      const int tn = min(kWindow, steps - tw);
      // MW, edge wavefront of a later group: lane l holds the row above on
      // step l of the window, (R, P) of cell (rbase - 1, dl - rbase)
      RT win_r = RINF;
      T win_p = (T)0;
      if (MW && EDGE && grp > 0) {
        const int j = dl - rbase;
        const bool v = (unsigned)j < (unsigned)M;
        const size_t cell = (size_t)b * NM + diag_soff(dl - 1, N, M) + (rbase - 1);
        RT* const pr = Rpl + cell;
        T* const pp = PEN ? a.P + cell : a.P;
        RT vr = RINF;
        T vp = (T)0;
        bool gave_up = false;
        const unsigned long long t0w = __builtin_amdgcn_s_memrealtime();
        for (int spin = 0;; ++spin) {
          if (v) {
            vr = __hip_atomic_load(pr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (PEN) vp = __hip_atomic_load(pp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          const bool pend = v && (mw_is_sentinel(vr) || (PEN && mw_is_sentinel(vp)));
          if (__ballot(pend) == 0) break;
          if (wait_ran_out(a, spin, t0w)) {
            gave_up = true;
            break;
          }
          __builtin_amdgcn_s_sleep(4);
        }
        // The wait ran out: report it (the sentinel, a NaN, then flows into
        // this pair's outputs) and go on, so the kernel still exits.
        if (gave_up && lane == 0)
          __hip_atomic_fetch_or(a.status, TW_STATUS_WAIT_GAVE_UP, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
        win_r = v ? vr : RINF;
        win_p = v ? vp : (T)0;
      }
    for (int t0 = 0; t0 < tn; t0 += kSlots) {
      const int half = (t0 / kSlots) & 1;   // mailbox half of this block
      Rec rec[kSlots];
      if (!EDGE) {
        const Rec* prev = inbox + (half ^ 1) * kSlots;
        rec[0] = carry;
#pragma unroll
        for (int u = 1; u < kSlots; ++u) rec[u] = prev[u - 1];
        carry = prev[kSlots - 1];
      }
      Rec* const out = my_out + half * kSlots;
      const ColRec<T>* const cblk = crow + (d_first + tw + t0);
      if (VEC) {
#pragma unroll
        for (int u = 0; u < kSlots; ++u)
#pragma unroll
          for (int k = 0; k < ROWS; ++k) {
            rc[u][k] = cn[u][k];
            rq[u][k] = qn[u][k];
          }
        fetch4(d_first + tw + t0 + kSlots, cn, qn);
      }
      // band: every row of this wavefront is outside |2i - d| <= band on all
      // of the block's diagonals, so its cells are INF / 0 without arithmetic
      bool skip = false;
      if (BAND) {
        const int dlo = d_first + tw + t0, wlo = rbase + wave * 64 * ROWS;
        skip = (T)(2 * wlo - (dlo + kSlots - 1)) > a.band ||
               (T)(dlo - 2 * (wlo + 64 * ROWS - 1)) > a.band;
      }
#pragma unroll
      for (int u = 0; u < kSlots; ++u) {
        const int d = d_first + tw + t0 + u;
        if (LC) creg[(u + 1) & 1] = cblk[u + 1];
        T cc[ROWS], cq[ROWS];
#pragma unroll
        for (int k = 0; k < ROWS; ++k) {
          cc[k] = rc[u % PF][k];
          cq[k] = rq[u % PF][k];
        }
        // the row above the first row on diagonal d-1, and the column
        // entering the first row on diagonal d
        Rec e;
        if (EDGE && MW)
          e = {lane_val(win_r, t0 + u), lane_val(win_p, t0 + u), ey_ring[u],
               COLS ? half_var(a, evy_ring[u]) : (T)0.5};
        else if (EDGE)
          e = {RINF, (T)0, ey_ring[u], COLS ? half_var(a, evy_ring[u]) : (T)0.5};
        else
          e = rec[u];

        nr2 = nr1;
        np2 = np1;
        nr1 = shift_prev(r1[ROWS - 1], e.x);
        if (PEN)
          np1 = (EDGE && !MW) ? shift_prev0(p1[ROWS - 1]) : shift_prev(p1[ROWS - 1], (T)e.y);
        if (LC) {
          yc[0] = creg[u & 1].y;
          hyc[0] = creg[u & 1].hy;
        } else if (COLS) {
          // the edge wavefront's column operands are wave-uniform: passing
          // them through readfirstlane gives each shift a fresh copy, so the
          // ring registers are never tied to (and overwritten by) a shift
          const T ny = SRC != SRC_FEAT1 ? (T)0
                       : shift_prev(yc[ROWS - 1], EDGE ? uniform((T)e.z) : (T)e.z);
          const T nhy = shift_prev(hyc[ROWS - 1], EDGE ? uniform((T)e.w) : (T)e.w);
#pragma unroll
          for (int k = ROWS - 1; k > 0; --k) {
            yc[k] = yc[k - 1];
            hyc[k] = hyc[k - 1];
          }
          yc[0] = ny;
          hyc[0] = nhy;
        }

        const int so = __builtin_amdgcn_readlane(so_st, t0 + u);
        const int so_r = so * (RES / ES);   // the same diagonal in the R plane
        RT nr[ROWS];
        T np[ROWS];
#pragma unroll
        for (int k = 0; k < ROWS; ++k) {
          const int j = d + jb[k];
          const bool valid = (unsigned)j < (unsigned)M;
          if (BAND && skip) {
            nr[k] = RINF;
            np[k] = (T)0;
          } else {
          const RT up = k ? r1[k - 1] : nr1;
          const RT dg = k ? r2[k - 1] : nr2;
          const RT lf = r1[k];
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
          // the differences of neighbours are taken in RT, the exponentials
          // in T (with RD: float exp2 / log2 of double-exact differences)
          const RT m = min3(dg, up, lf);
          const T ed = ex2((T)(m - dg)), eu = ex2((T)(m - up)), el = ex2((T)(m - lf));
          const T s = ed + eu + el;
          const RT rv = (RT)ch + m - (RT)lg2(s);
          bool ok = valid;
          if (BAND) ok = ok && (m < RINF) && (fabs((T)(2 * (row0 + k) - d)) <= a.band);
          nr[k] = ok ? rv : RINF;
          if (PEN) {
            const T pup = k ? p1[k - 1] : np1;
            const T pdg = k ? p2[k - 1] : np2;
            const T ps = fma(el, p1[k], fma(eu, pup, ed * pdg));
            const T pv = fma(ps, rcp(s), q);
            np[k] = ok ? pv : (T)0;
          } else {
            np[k] = (T)0;
          }
          }
          const bool stv = valid && !(MW && drop_row);
          bR.st(nr[k], stv ? vsr[k] : kOob, so_r);
          if (PEN) bP.st(np[k], stv ? vst[k] : kOob, so);
          if (MW && publish && lane == 63 && valid && !drop_row) {
            // the next group's row above: a second, agent-coherent store
            const size_t c = (size_t)b * NM + (size_t)((so + vst[k]) / ES);
            __hip_atomic_store(Rpl + c, nr[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (PEN)
              __hip_atomic_store(a.P + c, np[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
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
        if (SRC != SRC_FEAT1 && !VEC)
          fetch(d + PF, __builtin_amdgcn_readlane(so_ld, t0 + u), rc[u % PF], rq[u % PF]);
        if (EDGE && FLOW) {
          ey_ring[u] = col_y(vcol + (u + kSlots) * ES);
          evy_ring[u] = col_vy(vcol + (u + kSlots) * ES);
        }
        if (FLOW) {
          out[u] = {r1[ROWS - 1], p1[ROWS - 1], yc[ROWS - 1], hyc[ROWS - 1]};
        } else {
          out[u].x = r1[ROWS - 1];
          out[u].y = p1[ROWS - 1];
        }
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
    const RT rl = bR.ld<RT>(0, (int)(NM - 1) * RES);
    a.out_r[b] = (T)(rl * (RT)a.inv_k);   // INF (unreachable) and NaN pass through
    a.out_p[b] = PEN ? bP.ld<T>(0, so) : (T)0;
  }
}

// LC (one row per thread): the column operands come from LDS (ColRec) and
// the column gradient sums are accumulated per wavefront in LDS: a row reads
// its column's running sums at the start of a step and stores them updated
// at its end; the row above reads them on the next step. The wavefront's LDS
// operations execute in order, so each row sees the store of the row below
// (a wavefront-scope fence keeps the compiler from reordering them), and the
// rows add in sweep order, bottom row first. The wavefronts' sums are added
// in a fixed order at the end. Otherwise both travel along the rows with DPP
// shifts.
template <typename T, int ROWS, int SRC, bool PEN, bool BAND, int PF, bool LC, bool RD = false,
          bool MW = false>
__global__ void __launch_bounds__((MaxThreads<T, ROWS, LC, true, MW>::value)) udtw_bwd_kernel(UdtwArgs<T> a) {
  // (fused only where written as fma, as in the forward)
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int ES = sizeof(T);
  // RT: the type R and E = R - C are carried in (as the forward's R plane)
  using RT = std::conditional_t<RD, double, T>;
  constexpr int RES = sizeof(RT);
  static_assert(!RD || (sizeof(T) == 4 && ROWS == 1), "RD: float, one row per thread");
  const RT RINF = inf_v<RT>();
  constexpr bool COLS = SRC != SRC_COST;
  constexpr bool FLOW = COLS && !LC;
  static_assert(!LC || (COLS && ROWS == 1), "LDS columns need one row per thread");
  static_assert(!MW || (ROWS == 1 && !LC), "MW: one row per thread");
  const int N = a.N, M = a.M;
  // MW: G groups of kMwRows rows per pair, aligned to the bottom (the last
  // ends at row N-1, the first may be partial); group grp has gsh groups
  // below it. The group below runs first, so it has the lower index.
  const int G = MW ? a.groups : 1;
  const int b = MW ? (int)blockIdx.x / G : (int)blockIdx.x;
  const int gsh = MW ? (int)blockIdx.x % G : 0;
  const int grp = G - 1 - gsh;
  const int rbot = N - 1 - kMwRows * gsh;   // MW: this group's last row
  const int tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const T INF = inf_v<T>();
  const long long NM = (long long)N * M;
  const bool vgrad = COLS && a.dVX != nullptr;
  const int Dn = N + M - 1;

  // Rows are bottom-aligned: row N-1 is the last row of the last wavefront,
  // where every column enters the backward sweep.
  const int row0 = tid * ROWS - ((int)blockDim.x * ROWS - N) - (MW ? kMwRows * gsh : 0);

  // box[(v + 1) * kBox + slot]: wavefront v's inbox, the row below its last
  // row: (E, G, H, A) and (y, hy, dy sum, dvy sum); box[0..kBox) is
  // wavefront 0's unread outbox. Then the dump area.
  using Rec = BwdRec<T, RD>;
  Rec* box = reinterpret_cast<Rec*>(smem_raw);
  Rec* dump = box + (nw + 1) * kBox;
  const Rec rec0 = {{-RINF, (T)0, (T)0, (T)0}, {(T)0, (T)0.5, (T)0, (T)0}};
  for (int t = tid; t < (nw + 1) * kBox; t += blockDim.x) box[t] = rec0;
  // LC: column operands, then per wavefront the (dy, dvy) sums (same indexing)
  const int cpad = col_pad(N, nw), ncol = M + 2 * cpad;
  ColRec<T>* cols = reinterpret_cast<ColRec<T>*>(dump + kDump);
  ColRec<T>* acc = cols + ncol;
  if (LC) {
    for (int t = tid; t < ncol; t += blockDim.x) {
      const int j = t - cpad;
      ColRec<T> c = {(T)0, (T)0.5};
      if (j >= 0 && j < M) {
        if (SRC == SRC_FEAT1) c.y = a.Y[(size_t)b * M + j];
        c.hy = half_var(a, a.VY[(size_t)b * M + j]);
      }
      cols[t] = c;
    }
    for (int t = tid; t < nw * ncol; t += blockDim.x) acc[t] = {(T)0, (T)0};
  }

  Buf bR, bP, bC, bQ, bdC, bdQ, bY, bVY, bdY, bdVY;
  bR.init(reinterpret_cast<const RT*>(a.R) + b * NM, NM);
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
  if (SRC == SRC_FEAT1 && FLOW) {
    bY.init(a.Y + (size_t)b * M, M);
    bdY.init(a.dY + (size_t)b * M, M);
  }
  if (FLOW) bVY.init(a.VY + (size_t)b * M, M);
  // without variance gradients the column sums are still formed (no branch in
  // the sweep) and their stores go to an empty buffer, which drops them
  if (FLOW) bdVY.init(vgrad ? a.dVY + (size_t)b * M : a.VY, vgrad ? M : 0);
  // column operands of the edge wavefront at byte offset vcol (lane uniform);
  // columns before the first fail the range check and read 0
  auto col_y = [&](int vcol) -> T { return SRC == SRC_FEAT1 ? bY.ld<T>(vcol, 0) : (T)0; };
  auto col_vy = [&](int vcol) -> T { return COLS ? bVY.ld<T>(vcol, 0) : (T)1; };

  const bool last_wave = wave == nw - 1;
  Rec* const inbox = box + (wave + 1) * kBox;
  Rec* const outbox = box + wave * kBox;
  Rec* const my_out = lane == 0 ? outbox : dump + lane;
  __syncthreads();

  T xr[ROWS], hxr[ROWS], dxr[ROWS], dvr[ROWS];
  RT e1[ROWS], e2[ROWS];
  T g1[ROWS], g2[ROWS], h1[ROWS], h2[ROWS], a1[ROWS], a2[ROWS];
  T yc[ROWS], hyc[ROWS], cy[ROWS], cvy[ROWS];
  int vst[ROWS], vsr[ROWS], vnat[ROWS], jb[ROWS], vrow0[ROWS];
  // SRC_COST: parity of the element index of (i, d - i) in dC / dQ, less d
  // (the gradients leave in aligned pairs of row neighbours)
  int cpar[ROWS], qpar[ROWS];
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    const int i = row0 + k;
    const bool in = i >= 0 && i < N;
    if (SRC == SRC_COST) {
      const size_t rowc = (size_t)b * NM + (size_t)(in ? i : 0) * (M - 1);
      cpar[k] = (int)((((size_t)a.dC / ES) + rowc) & 1);
      qpar[k] = want_dq ? (int)((((size_t)a.dQ / ES) + rowc) & 1) : 0;
    }
    xr[k] = (SRC == SRC_FEAT1 && in) ? a.X[(size_t)b * N + i] : (T)0;
    hxr[k] = (COLS && in) ? half_var(a, a.VX[(size_t)b * N + i]) : (T)0.5;
    dxr[k] = dvr[k] = (T)0;
    e1[k] = e2[k] = -RINF;
    g1[k] = g2[k] = h1[k] = h2[k] = a1[k] = a2[k] = (T)0;
    yc[k] = cy[k] = cvy[k] = (T)0;
    hyc[k] = (T)0.5;
    vst[k] = in ? i * ES : 0;
    vsr[k] = in ? i * RES : 0;
    vnat[k] = in ? i * (M - 1) * ES : 0;
    jb[k] = in ? -i : INT_MIN / 2;
    // the row that stores finished columns (MW: in the top group only; the
    // other groups hand their column sums up with the boundary records)
    vrow0[k] = (i == 0 && (!MW || grp == 0)) ? 0 : kOob;
  }
  // Row below the last row on the two previous diagonals. The virtual cell
  // (N, M) on diagonal Dn+1 is given E = Rh(N-1, M-1), A = P(N-1, M-1) and the
  // incoming gradients, so the recursion yields grad_dist / grad_pen at
  // (N-1, M-1) without a special case.
  RT ne1 = -RINF, ne2 = -RINF;
  T ng1 = 0, ng2 = 0, nh1 = 0, nh2 = 0, na1 = 0, na2 = 0;
  if (last_wave && lane == 63 && gsh == 0) {
    const int so = (int)(NM - 1) * ES;
    ne1 = bR.ld<RT>(0, (int)(NM - 1) * RES);
    ng1 = a.gr[(size_t)b * a.gstride];
    if (PEN) {
      nh1 = a.gp[(size_t)b * a.gstride];
      na1 = bP.ld<T>(0, so);
    }
  }

  const int d_first = Dn - 1 + kLag * (nw - 1 - wave) + (MW ? kGroupLag * gsh : 0);
  const int steps =
      (Dn + kLag * (nw - 1) + (MW ? kGroupLag * (G - 1) : 0) + kSlots - 1) / kSlots * kSlots;
  // MW: the top row of a group above the bottom one publishes its records
  const bool publish = MW && grp > 0 && wave == 0 && !a.drop_handoff;
  constexpr int HW = HandRec<T, RD>::words;
  constexpr int HWS = hand_words(ES);

  RT rr[PF][ROWS];
  T rp[PF][ROWS], rc[PF][ROWS], rq[PF][ROWS];
  constexpr bool VEC = SRC == SRC_COST && PF == kSlots;   // block-wide C / Q loads
  // R, P of diagonal d at byte soffset so_d = soff(d) * ES (diagonal-major;
  // R at the same cell of its RES-byte plane), C, Q at so_n = max(d, 0) * ES
  // ([N, M])
  auto fetch = [&](int d, int so_d, int so_n, RT* r, T* p, T* c, T* q) {
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const bool v = (unsigned)(d + jb[k]) < (unsigned)M;
      const int vd = v ? vst[k] : kOob;
      r[k] = bR.ld<RT>(v ? vsr[k] : kOob, so_d * (RES / ES));
      if (PEN) p[k] = bP.ld<T>(vd, so_d);
      if (SRC == SRC_SQ) {
        c[k] = bC.ld<T>(vd, so_d);   // diagonal-major, as R
      } else if (SRC != SRC_FEAT1 && !VEC) {
        const int vn = v ? vnat[k] : kOob;
        c[k] = bC.ld<T>(vn, so_n);
        if (SRC == SRC_COST && PEN) q[k] = bQ.ld<T>(vn, so_n);
      }
    }
  };
  // VEC: as in the forward, a row's C / Q cells of a block come from one
  // 16-byte load per plane, a block ahead. The block's diagonals run down
  // from dh, so cell (i, dh - u - i) of step u is component 3 - u of the
  // load at (i, dh - 3 - i).
  T cn[kSlots][ROWS], qn[kSlots][ROWS];
  auto fetch4 = [&](int dh, T (*c)[ROWS], T (*q)[ROWS]) {
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const int vo = vnat[k] + (dh - (kSlots - 1)) * ES;
#pragma unroll
      for (int h = 0; h < (int)sizeof(T) / 4; ++h) {
        const unsigned int __attribute__((ext_vector_type(4))) w =
            __builtin_amdgcn_raw_buffer_load_b128(bC.r, vo + 16 * h, 0, 0);
        unsigned int __attribute__((ext_vector_type(4))) z = {0, 0, 0, 0};
        if (PEN) z = __builtin_amdgcn_raw_buffer_load_b128(bQ.r, vo + 16 * h, 0, 0);
        if constexpr (sizeof(T) == 4) {
          c[3][k] = __uint_as_float(w.x); c[2][k] = __uint_as_float(w.y);
          c[1][k] = __uint_as_float(w.z); c[0][k] = __uint_as_float(w.w);
          q[3][k] = __uint_as_float(z.x); q[2][k] = __uint_as_float(z.y);
          q[1][k] = __uint_as_float(z.z); q[0][k] = __uint_as_float(z.w);
        } else {
          auto dbl = [](unsigned lo, unsigned hi) {
            return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
          };
          c[3 - 2 * h][k] = dbl(w.x, w.y); c[2 - 2 * h][k] = dbl(w.z, w.w);
          q[3 - 2 * h][k] = dbl(z.x, z.y); q[2 - 2 * h][k] = dbl(z.z, z.w);
        }
      }
      // At the plane's start (row 0, the last blocks) the load begins before
      // the plane: a negative voffset fails the range check as a whole, so
      // those lanes take the block's cells one by one (negative ones read 0).
      if (__ballot(vo < 0) != 0 && vo < 0) {
#pragma unroll
        for (int u = 0; u < kSlots; ++u) {
          const int vu = vnat[k] + (dh - u) * ES;
          c[u][k] = bC.ld<T>(vu, 0);
          q[u][k] = PEN ? bQ.ld<T>(vu, 0) : (T)0;
        }
      }
    }
  };
#pragma unroll
  for (int u = 0; u < PF; ++u) {
    const int d = d_first - u;
    fetch(d, diag_soff(d, N, M) * ES, (d > 0 ? d : 0) * ES, rr[u], rp[u], rc[u], rq[u]);
  }
  if (VEC) fetch4(d_first, cn, qn);

  // The sweep, instantiated for the edge wavefront (the last: its row below
  // is the virtual row N, its entering column comes from a register ring of
  // column loads) and for the others (row below and columns from the mailbox).
  auto sweep = [&](auto edge_tag) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    // EDGE: ring slot u of a trip holds column M-1-t0-u, the one entering row
    // N-1 on that step's diagonal
    T ey_ring[kSlots], evy_ring[kSlots];
    // EDGE: byte offset of column M-1-t0 (MW: the column entering row rbot
    // on the group's first diagonal)
    int vcol = (M - 1 + (MW ? (kGroupLag + kMwRows) * gsh : 0)) * ES;
    if (EDGE && FLOW) {
#pragma unroll
      for (int u = 0; u < kSlots; ++u) {
        ey_ring[u] = col_y(vcol - u * ES);
        evy_ring[u] = col_vy(vcol - u * ES);
      }
    }
    // LC: this row's entries on diagonal d are crow[d] and arow[d]; step u
    // of a block uses creg[u % 2] and reads the next step's into the other
    const ColRec<T>* const crow = cols + cpad - row0;
    ColRec<T>* const arow = acc + wave * ncol + cpad - row0;
    ColRec<T> creg[2];
    if (LC) creg[0] = crow[d_first];
    Rec carry = rec0;   // the record used by the first step of the next block
    __builtin_amdgcn_s_waitcnt(0);   // drain the set-up loads (as in the forward)
    for (int tw = 0; tw < steps; tw += kWindow) {
      // lane l: byte soffsets of step tw + l (fetch of R / P and C / Q, and
      // the stores of the step's own diagonal)
      const int dl = d_first - tw - lane;
      const int so_fd = diag_soff(dl - PF, N, M) * ES;
      const int so_fn = SRC == SRC_COST ? (dl - PF > 0 ? dl - PF : 0) * ES : 0;
      const int so_st = (dl > 0 ? dl : 0) * ES;
      // SRC_SQ: the diagonal-major soffset of the step's own diagonal (dS store)
      const int so_sd = SRC == SRC_SQ ? diag_soff(dl, N, M) * ES : 0;
      const int tn = min(kWindow, steps - tw);
      // MW, edge wavefront of a group above the bottom one: lane l holds the
      // record of the row below (the next group's top row) on diagonal
      // dl + 1, i.e. of its cell in column dl - rbot
      RT wn_e = -RINF;
      T wn_g = (T)0, wn_h = (T)0, wn_a = (T)0, wn_cy = (T)0, wn_cvy = (T)0;
      if (MW && EDGE && gsh > 0) {
        const int jc = dl - rbot;
        const bool v = (unsigned)jc < (unsigned)M;
        const unsigned long long* w =
            a.hand + ((size_t)(b * (G - 1) + grp) * M + (v ? jc : 0)) * HWS;
        unsigned long long x[HW];
#pragma unroll
        for (int q = 0; q < HW; ++q) x[q] = kHandSentinel;
        bool gave_up = false;
        const unsigned long long t0w = __builtin_amdgcn_s_memrealtime();
        for (int spin = 0;; ++spin) {
          bool pend = false;
          if (v) {
#pragma unroll
            for (int q = 0; q < HW; ++q) {
              x[q] = __hip_atomic_load(w + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              pend = pend || x[q] == kHandSentinel;
            }
          }
          if (__ballot(pend) == 0) break;
          if (wait_ran_out(a, spin, t0w)) {
            gave_up = true;
            break;
          }
          __builtin_amdgcn_s_sleep(4);
        }
        // as in the forward: report a wait that ran out and go on (the
        // sentinel words decode to NaNs, which flow into the gradients)
        if (gave_up && lane == 0)
          __hip_atomic_fetch_or(a.status, TW_STATUS_WAIT_GAVE_UP, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
        if (v) {
          if constexpr (sizeof(T) == 8) {
            wn_e = word_to_d(x[0]);
            wn_g = word_to_d(x[1]);
            wn_h = word_to_d(x[2]);
            wn_a = word_to_d(x[3]);
            wn_cy = word_to_d(x[4]);
            wn_cvy = word_to_d(x[5]);
          } else if constexpr (RD) {
            wn_e = word_to_d(x[0]);
            wn_g = word_lo(x[1]);
            wn_h = word_hi(x[1]);
            wn_a = word_lo(x[2]);
            wn_cy = word_hi(x[2]);
            wn_cvy = word_lo(x[3]);
          } else {
            wn_e = word_lo(x[0]);
            wn_g = word_hi(x[0]);
            wn_h = word_lo(x[1]);
            wn_a = word_hi(x[1]);
            wn_cy = word_lo(x[2]);
            wn_cvy = word_hi(x[2]);
          }
        }
      }
    for (int t0 = 0; t0 < tn; t0 += kSlots) {
      const int half = (t0 / kSlots) & 1;   // mailbox half of this block
      Rec rec[kSlots];
      if (!EDGE) {
        const Rec* prev = inbox + (half ^ 1) * kSlots;
        rec[0] = carry;
#pragma unroll
        for (int u = 1; u < kSlots; ++u) {
          rec[u].a = prev[u - 1].a;
          if (FLOW) rec[u].b = prev[u - 1].b;
        }
        carry.a = prev[kSlots - 1].a;
        if (FLOW) carry.b = prev[kSlots - 1].b;
      }
      Rec* const out = my_out + half * kSlots;
      // LC: entries of the block's diagonals (and the next one) at
      // non-negative offsets from the diagonal below the block's last
      const int dlo = d_first - tw - t0 - kSlots;
      const ColRec<T>* const cblk = crow + dlo;
      ColRec<T>* const ablk = arow + dlo;
      if (VEC) {
#pragma unroll
        for (int u = 0; u < kSlots; ++u)
#pragma unroll
          for (int k = 0; k < ROWS; ++k) {
            rc[u][k] = cn[u][k];
            rq[u][k] = qn[u][k];
          }
        fetch4(d_first - tw - t0 - kSlots, cn, qn);
      }
      // band: every row of this wavefront is outside |2i - d| <= band on all
      // of the block's diagonals (the forward left those cells at INF)
      bool skip = false;
      if (BAND) {
        const int bhi = d_first - tw - t0, blo = bhi - (kSlots - 1);
        const int wlo =
            wave * 64 * ROWS - ((int)blockDim.x * ROWS - N) - (MW ? kMwRows * gsh : 0);
        skip = (T)(2 * wlo - bhi) > a.band || (T)(blo - 2 * (wlo + 64 * ROWS - 1)) > a.band;
      }
#pragma unroll
      for (int u = 0; u < kSlots; ++u) {
        const int d = d_first - tw - t0 - u;
        ColRec<T> csum;
        if (LC) {
          creg[(u + 1) & 1] = cblk[kSlots - 1 - u];
          // after the row below stored this column's sums (previous step);
          // the step's arithmetic stays behind the read, covering its latency
          __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
          csum = ablk[kSlots - u];
          __builtin_amdgcn_sched_barrier(0);
        }
        RT cr[ROWS];
        T cp[ROWS], cc[ROWS], cq[ROWS];
  #pragma unroll
        for (int k = 0; k < ROWS; ++k) {
          cr[k] = rr[u % PF][k];
          cp[k] = rp[u % PF][k];
          cc[k] = rc[u % PF][k];
          cq[k] = rq[u % PF][k];
        }
        // the row below the last row on diagonal d+1, and the column entering
        // the last row on diagonal d
        Rec ex;
        if (EDGE && MW)   // (the bottom group's window values are the virtual row's)
          ex = {{lane_val(wn_e, t0 + u), lane_val(wn_g, t0 + u), lane_val(wn_h, t0 + u),
                 lane_val(wn_a, t0 + u)},
                {ey_ring[u], COLS ? half_var(a, evy_ring[u]) : (T)0.5,
                 lane_val(wn_cy, t0 + u), lane_val(wn_cvy, t0 + u)}};
        else if (EDGE)
          ex = {{-RINF, (T)0, (T)0, (T)0},
                {ey_ring[u], COLS ? half_var(a, evy_ring[u]) : (T)0.5, (T)0, (T)0}};
        else
          ex = rec[u];

        ne2 = ne1;
        ng2 = ng1;
        nh2 = nh1;
        na2 = na1;
        constexpr bool ZF = EDGE && !MW;   // the edge's row below is zero
        ne1 = shift_next(e1[0], ex.a.x);
        ng1 = ZF ? shift_next0(g1[0]) : shift_next(g1[0], (T)ex.a.y);
        if (PEN) {
          nh1 = ZF ? shift_next0(h1[0]) : shift_next(h1[0], (T)ex.a.z);
          na1 = ZF ? shift_next0(a1[0]) : shift_next(a1[0], (T)ex.a.w);
        }
        if (LC) {
          yc[0] = creg[u & 1].y;
          hyc[0] = creg[u & 1].hy;
        } else if (COLS) {
          const T fy = SRC != SRC_FEAT1 ? (T)0
                       : shift_next(yc[0], EDGE ? uniform((T)ex.b.x) : (T)ex.b.x);
          const T fhy = shift_next(hyc[0], EDGE ? uniform((T)ex.b.y) : (T)ex.b.y);
          const T fcy = SRC != SRC_FEAT1 ? (T)0
                        : ZF ? shift_next0(cy[0]) : shift_next(cy[0], (T)ex.b.z);
          const T fcvy = ZF ? shift_next0(cvy[0]) : shift_next(cvy[0], (T)ex.b.w);
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
        RT xe[ROWS];
        T xg[ROWS], xh[ROWS], xa[ROWS];
  #pragma unroll
        for (int k = 0; k < ROWS; ++k) {
          const bool valid = (unsigned)(d + jb[k]) < (unsigned)M;
          // the cell's adjoints (g, h), dS and the variance / feature terms;
          // all zero for a skipped (out-of-band) block, as for any cell the
          // forward left at INF
          T g = (T)0, h = (T)0, dsq = (T)0, df = (T)0, dvar = (T)0;
          if (BAND && skip) {
            xe[k] = -RINF;
            xa[k] = (T)0;
          } else {
          const RT rk = valid ? cr[k] : RINF;
          const T pk = cp[k];
          T ch, q = (T)0, c = (T)0, rv = (T)1, sq_raw = (T)0, var_raw = (T)1;
          if (SRC == SRC_COST) {
            ch = cc[k] * a.k;
            if (PEN) q = cq[k];
          } else {
            if (SRC == SRC_FEAT1) {
              const T df0 = xr[k] - yc[k];
              sq_raw = df0 * df0;
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
          const RT edn = (k + 1 < ROWS) ? e1[k + 1] : ne1;
          const T gdn = (k + 1 < ROWS) ? g1[k + 1] : ng1;
          const RT edg = (k + 1 < ROWS) ? e2[k + 1] : ne2;
          const T gdg = (k + 1 < ROWS) ? g2[k + 1] : ng2;
          const T wdn = ex2((T)(edn - rk)), wrt = ex2((T)(e1[k] - rk)), wdg = ex2((T)(edg - rk));
          g = fma(wdg, gdg, fma(wrt, g1[k], wdn * gdn));
          if (PEN) {
            const T hdn = (k + 1 < ROWS) ? h1[k + 1] : nh1;
            const T adn = (k + 1 < ROWS) ? a1[k + 1] : na1;
            const T hdg = (k + 1 < ROWS) ? h2[k + 1] : nh2;
            const T adg = (k + 1 < ROWS) ? a2[k + 1] : na2;
            const T wh_dn = wdn * hdn, wh_rt = wrt * h1[k], wh_dg = wdg * hdg;
            const T cpen = fma(wh_dg, pk - adg, fma(wh_rt, pk - a1[k], wh_dn * (pk - adn)));
            g = fma(-cpen, a.inv_gamma, g);
            h = wh_dn + wh_rt + wh_dg;
          }
          // outside the grid, and (band) at unreachable cells, nothing flows
          bool live = valid;
          if (BAND) live = live && rk < RINF;
          g = live ? g : (T)0;
          h = live ? h : (T)0;
          xe[k] = live ? rk - (RT)ch : -RINF;
          xa[k] = valid ? pk - q : (T)0;
          if (SRC != SRC_COST) {
            dsq = sq_raw > (T)0 ? g * rv : (T)0;
            if (SRC == SRC_FEAT1) df = valid ? (T)2 * dsq * (xr[k] - yc[k]) : (T)0;
            dvar = var_raw > a.eps ? (T)0.5 * fma(a.beta, h, -(g * c)) * rv : (T)0;
            dvar = valid ? dvar : (T)0;
          }
          }
          xg[k] = g;
          xh[k] = h;

          const int vn = valid ? vnat[k] : kOob;
          if (SRC == SRC_COST) {
            // (i, j) with an even element index stores itself and (i, j + 1),
            // the lane's previous cell (g1, h1), as one aligned store; an odd
            // one is stored by (i, j - 1)'s pair; left over: even cells in
            // column M - 1 and odd ones in column 0, stored alone
            const int j = d + jb[k];
            const bool ec = ((cpar[k] ^ d) & 1) == 0;
            st_pair<T>(bdC, (valid && ec && j + 1 < M) ? vn : kOob, g, g1[k], so_n);
            bdC.st(g, (valid && (ec ? j == M - 1 : j == 0)) ? vn : kOob, so_n);
            if (PEN) {
              const bool eq = ((qpar[k] ^ d) & 1) == 0;
              st_pair<T>(bdQ, (valid && eq && j + 1 < M) ? vn : kOob, h, h1[k], so_n);
              bdQ.st(h, (valid && (eq ? j == M - 1 : j == 0)) ? vn : kOob, so_n);
            }
          } else {
            if (SRC == SRC_SQ)
              bdC.st(dsq, valid ? vst[k] : kOob, __builtin_amdgcn_readlane(so_sd, t0 + u));
            if (SRC == SRC_FEAT1) dxr[k] += df;
            dvr[k] += dvar;
            if (LC) {
              // this wavefront's sums of column d - row0 (invalid cells add 0)
              ablk[kSlots - u] = {csum.y - df, csum.hy + dvar};
            } else {
              cy[k] -= df;
              cvy[k] += dvar;
              // column d leaves the sweep at row 0: store its sums
              const int vc = ((unsigned)d < (unsigned)M) ? vrow0[k] : kOob;
              if (SRC == SRC_FEAT1) bdY.st(cy[k], vc, so_n);
              bdVY.st(cvy[k], vc, so_n);
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
        // ring reloads only now (see the forward)
        __builtin_amdgcn_sched_barrier(0);
        fetch(d - PF, __builtin_amdgcn_readlane(so_fd, t0 + u),
              __builtin_amdgcn_readlane(so_fn, t0 + u), rr[u % PF], rp[u % PF], rc[u % PF],
              rq[u % PF]);
        if (EDGE && FLOW) {
          ey_ring[u] = col_y(vcol - (u + kSlots) * ES);
          evy_ring[u] = col_vy(vcol - (u + kSlots) * ES);
        }
        if (FLOW) {
          out[u] = {{e1[0], g1[0], h1[0], a1[0]}, {yc[0], hyc[0], cy[0], cvy[0]}};
        } else {
          out[u].a = {e1[0], g1[0], h1[0], a1[0]};
        }
        if (MW && publish) {
          // the group above's row below: this row's record of diagonal d
          const int j = d - row0;
          if (lane == 0 && (unsigned)j < (unsigned)M) {
            unsigned long long* w = a.hand + ((size_t)(b * (G - 1) + grp - 1) * M + j) * HWS;
            unsigned long long x[HW];
            if constexpr (sizeof(T) == 8) {
              x[0] = word_d(e1[0]);
              x[1] = word_d(g1[0]);
              x[2] = word_d(h1[0]);
              x[3] = word_d(a1[0]);
              x[4] = word_d(cy[0]);
              x[5] = word_d(cvy[0]);
            } else if constexpr (RD) {
              x[0] = word_d(e1[0]);
              x[1] = pack_ff(g1[0], h1[0]);
              x[2] = pack_ff(a1[0], cy[0]);
              x[3] = pack_ff(cvy[0], 0.0f);
            } else {
              x[0] = pack_ff(e1[0], g1[0]);
              x[1] = pack_ff(h1[0], a1[0]);
              x[2] = pack_ff(cy[0], cvy[0]);
            }
#pragma unroll
            for (int q = 0; q < HW; ++q)
              __hip_atomic_store(w + q, x[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
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
  // Variance gradients are d/dv of the variance inputs; when those are
  // standard deviations s (v = s^2) the gradient is d/ds = 2 s d/dv.
#pragma unroll
  for (int k = 0; k < ROWS; ++k) {
    const int i = row0 + k;
    if (i >= 0 && i < N) {
      if (SRC == SRC_FEAT1) a.dX[(size_t)b * N + i] = dxr[k];
      if (vgrad) {
        const T sx = a.VX[(size_t)b * N + i];
        a.dVX[(size_t)b * N + i] = a.sigma ? (T)2 * sx * dvr[k] : dvr[k];
      }
    }
  }
  if (LC) {
    // column sums: the wavefronts' partial sums, bottom wavefront first
    __syncthreads();
    for (int j = tid; j < M; j += blockDim.x) {
      T sy = (T)0, svy = (T)0;
      for (int v = nw - 1; v >= 0; --v) {
        sy += acc[v * ncol + cpad + j].y;
        svy += acc[v * ncol + cpad + j].hy;
      }
      if (SRC == SRC_FEAT1) a.dY[(size_t)b * M + j] = sy;
      if (vgrad) {
        const T sy_in = a.VY[(size_t)b * M + j];
        a.dVY[(size_t)b * M + j] = a.sigma ? (T)2 * sy_in * svy : svy;
      }
    }
  } else if (FLOW && a.sigma && vgrad && grp == 0) {
    // the sweep stored d/dv of every column; once all of its stores are
    // complete and visible, scale them to d/ds
    __threadfence();
    __syncthreads();
    for (int j = tid; j < M; j += blockDim.x) {
      const size_t o = (size_t)b * M + j;
      a.dVY[o] = (T)2 * a.VY[o] * a.dVY[o];
    }
  }
}

// ---------------------------------------------------------------- launching

struct Shape {
  int rows;
  int threads;
};

// Threads of a one-workgroup-per-pair sweep for a grid with N rows (N <= M):
// one row per thread, up to the kernels' thread limit (1024 in float, 512 in
// double); rows {0, 0} past it (those pairs run several workgroups).
template <typename T>
static Shape pick_shape(int N, bool backward) {
  const int one_row_max =
      backward ? MaxThreads<T, 1, false, true>::value : MaxThreads<T, 1, false, false>::value;
  if (N > one_row_max) return {0, 0};
  return {1, ((N + 63) / 64) * 64};
}

// LDS of one workgroup: the mailbox rings and the dump area of the
// mailbox stores (records of 4 values forward, 8 backward).
// LDS of a sweep: mailboxes and dump, then with LDS columns (lc) the column
// entries and, in the backward, each wavefront's two column-sum arrays.
template <typename T>
static size_t udtw_lds(bool backward, int nw, bool lc, int N, int M, bool rd = false) {
  // mailbox record bytes (RD: one double and float values)
  const size_t rec = rd ? (backward ? sizeof(RecD8) : sizeof(RecD4))
                        : (backward ? 8 : 4) * sizeof(T);
  size_t n = (size_t)((nw + 1) * kBox + kDump) * rec;
  if (lc) {
    const size_t ncol = (size_t)M + 2 * (size_t)col_pad(N, nw);
    n += ncol * sizeof(ColRec<T>);
    if (backward) n += (size_t)nw * ncol * sizeof(ColRec<T>);
  }
  return n;
}

// Prefetch depth (diagonals) of the register ring for a row count: loads
// are issued this many diagonals before their use, enough to cover an HBM
// miss when a diagonal step takes a few hundred nanoseconds. It divides the
// block of kSlots steps, so ring slots stay compile-time constants.
template <int ROWS>
struct PrefetchDepth {
  static constexpr int value = ROWS <= 4 ? 4 : (ROWS == 8 ? 2 : 1);
};

// MW: the sentinel into the boundary rows (256 g - 1, g >= 1) of R (elements
// of RT) and P (of T).
template <typename T, typename RT>
__global__ void __launch_bounds__(256) mw_fill(RT* R, T* P, int B, int N, int M, int G) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long per = (long long)(G - 1) * M;
  if (idx >= (long long)B * per) return;
  const int b = (int)(idx / per);
  const long long rem = idx - (long long)b * per;
  const int g = 1 + (int)(rem / M), j = (int)(rem % M);
  const int row = g * kMwRows - 1;
  const size_t c = (size_t)b * N * M + diag_soff(row + j, N, M) + row;
  auto sentinel = [](auto zero) {
    using V = decltype(zero);
    if constexpr (sizeof(V) == 4)
      return __uint_as_float((unsigned)mw_sentinel_bits(4));
    else
      return __longlong_as_double((long long)mw_sentinel_bits(8));
  };
  R[c] = sentinel(RT{});
  if (P) P[c] = sentinel(T{});
}

// MW backward: every hand-off word to the sentinel.
// (a template, so that every object including this header may instantiate it)
template <int = 0>
__global__ void __launch_bounds__(256) hand_fill(unsigned long long* w, long long n) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx < n) w[idx] = kHandSentinel;
}

// Several workgroups per pair for the forward when the batch leaves CUs
// idle (at most this many workgroups). Measured at B = 64 / 16, N = M =
// 1024: the D = 1 forward 0.74 -> 0.62 / 0.46 ms, the cost-path forward
// 3.36 -> 2.15 ms; the diagonal-major S forward (D > 1) 0.93 -> 1.07 ms,
// so it keeps one workgroup per pair. TORCHWARP_UDTW_MW=0 turns MW off, 1
// uses it for every source.
constexpr long long kMwMaxGroups = 512;
static inline int mw_mode() {
  static const int mode = [] {
    const char* e = getenv("TORCHWARP_UDTW_MW");
    return e ? atoi(e) : 2;
  }();
  const int forced = test_mw_mode();   // a test's choice, -1: none
  return forced >= 0 ? forced : mode;
}
static inline bool mw_enabled(int src) {
  return mw_mode() == 1 || (mw_mode() == 2 && src != SRC_SQ);
}
// Longer sequences than one workgroup holds at one row per thread (1024 rows
// in float, 512 in double) run with several workgroups per pair in both
// directions (TORCHWARP_UDTW_MW=0 keeps one workgroup per pair and so limits
// the length to those rows).
template <typename T>
static inline bool mw_long(int N) {
  return mw_mode() != 0 && N > MaxThreads<T, 1, false, false>::value;
}
// Several workgroups per pair in both directions: for sequences longer than
// one workgroup holds, and, past one group of rows, whenever the batch has
// fewer pairs than the device has CUs (one workgroup per pair would leave
// CUs idle: at B = 64, N = M = 1024, D = 16 the step takes 1.98 ms with four
// workgroups per pair against 2.29 ms with one); mode 1 splits every pair
// past one group of rows.
template <typename T>
static inline bool mw_split(int B, int N) {
  if (mw_long<T>(N)) return true;
  if (N <= kMwRows || mw_mode() == 0) return false;
  return mw_mode() == 1 || B < num_cus();
}
template <typename T>
static inline bool mw_backward(int B, int N) {
  return mw_split<T>(B, N);
}
// Hand-off workspace of the MW backward (bytes): 0 when it runs one
// workgroup per pair.
template <typename T>
static inline size_t mw_hand_bytes(int B, int N, int M) {
  if (!mw_backward<T>(B, N)) return 0;
  const long long G = (N + kMwRows - 1) / kMwRows;
  return (size_t)B * (size_t)(G - 1) * (size_t)M * hand_words(sizeof(T)) * 8;
}

// One-row-per-thread kernels (LDS columns, several workgroups per pair, or
// columns by DPP) with R carried in T or, for float with RD, in double.
template <typename T, int SRC, bool PEN, bool BAND, bool RD>
static int launch_one_row(bool backward, const UdtwArgs<T>& a, int B, const Shape& sh,
                          bool longseq, hipStream_t stream, const char* what) {
  const int nw = sh.threads / 64;
  dim3 grid(B), block(sh.threads);
  // one row per thread with column operands: stage the columns in LDS when
  // they fit in a quarter of it (several workgroups per CU stay resident)
  if constexpr (SRC != SRC_COST) {
    const size_t lc_lds = udtw_lds<T>(backward, nw, true, a.N, a.M, RD);
    if (!longseq && sh.threads <= 256 && lc_lds <= (size_t)max_lds_bytes() / 4) {
      if (backward)
        hipLaunchKernelGGL(
            (udtw_bwd_kernel<T, 1, SRC, PEN, BAND, PrefetchDepth<1>::value, true, RD>), grid,
            block, lc_lds, stream, a);
      else
        hipLaunchKernelGGL(
            (udtw_fwd_kernel<T, 1, SRC, PEN, BAND, PrefetchDepth<1>::value, true, false, RD>),
            grid, block, lc_lds, stream, a);
      return check_launch(what);
    }
  }
  const int G = (a.N + kMwRows - 1) / kMwRows;
  const bool mw = G > 1 && (longseq || mw_split<T>(B, a.N) ||
                            (!backward && !BAND && (long long)B * G <= kMwMaxGroups &&
                             mw_enabled(SRC)));
  if (mw) {
    using RT = std::conditional_t<RD, double, T>;
    UdtwArgs<T> m = a;
    m.groups = G;
    m.status = status_word();
    if (!m.status) return fail(TW_ELAUNCH, "%s: no device status word", what);
    m.spins = wait_spins(kMwSpins);
    m.wait_ticks = (unsigned long long)(kMwWaitSeconds * 1e3 * realtime_khz());
    m.drop_handoff = wait_drop_handoff();
    const size_t mlds = udtw_lds<T>(backward, kMwRows / 64, false, a.N, a.M, RD);
    const dim3 mgrid((unsigned)((long long)B * G)), mblock(kMwRows);
    if (backward) {
      if (!m.hand) return fail(TW_ESIZE, "%s: internal: no hand-off workspace", what);
      const long long words = (long long)B * (G - 1) * a.M * hand_words(sizeof(T));
      hipLaunchKernelGGL((hand_fill<>), dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                         stream, m.hand, words);
      hipLaunchKernelGGL(
          (udtw_bwd_kernel<T, 1, SRC, PEN, BAND, PrefetchDepth<1>::value, false, RD, true>),
          mgrid, mblock, mlds, stream, m);
    } else {
      const long long fills = (long long)B * (G - 1) * a.M;
      hipLaunchKernelGGL((mw_fill<T, RT>), dim3((unsigned)((fills + 255) / 256)), dim3(256), 0,
                         stream, reinterpret_cast<RT*>(m.R), PEN ? m.P : (T*)nullptr, B, a.N,
                         a.M, G);
      hipLaunchKernelGGL(
          (udtw_fwd_kernel<T, 1, SRC, PEN, BAND, PrefetchDepth<1>::value, false, true, RD>),
          mgrid, mblock, mlds, stream, m);
    }
    return check_launch(what);
  }
  const size_t lds = udtw_lds<T>(backward, nw, false, a.N, a.M, RD);
  if (lds > (size_t)max_lds_bytes()) {
    return fail(TW_ESIZE, "%s: %zu bytes of LDS needed, %d available", what, lds,
                max_lds_bytes());
  }
  // (RD backward at up to 1024 threads: a ring two diagonals deep keeps its
  // doubles within the 128 registers a lane has there)
  if (backward)
    hipLaunchKernelGGL(
        (udtw_bwd_kernel<T, 1, SRC, PEN, BAND, RD ? 2 : PrefetchDepth<1>::value, false, RD>),
        grid, block, lds, stream, a);
  else
    hipLaunchKernelGGL(
        (udtw_fwd_kernel<T, 1, SRC, PEN, BAND, PrefetchDepth<1>::value, false, false, RD>), grid,
        block, lds, stream, a);
  return check_launch(what);
}

template <typename T, int SRC, bool PEN, bool BAND>
static int launch_udtw(bool backward, const UdtwArgs<T>& a, int B, hipStream_t stream,
                       const char* what) {
  if (B == 0) return TW_OK;
  // planes are addressed with 32-bit byte offsets within a pair
  const long long rbytes = a.rd ? 8 : (long long)sizeof(T);
  if ((long long)a.N * a.M * rbytes >= (1LL << 31)) {
    return fail(TW_ESIZE, "%s: one pair's N*M matrix (%d x %d) must stay below 2 GiB", what,
                a.N, a.M);
  }
  const bool longseq = mw_long<T>(a.N);
  const Shape sh = longseq ? Shape{1, kMwRows} : pick_shape<T>(a.N, backward);
  if (sh.rows == 0) {
    return fail(TW_ESIZE, "%s: the shorter sequence has %d steps; one workgroup per pair "
                "(TORCHWARP_UDTW_MW=0) holds up to %d", what, a.N,
                MaxThreads<T, 1, false, false>::value);
  }
  if constexpr (sizeof(T) == 4) {
    if (a.rd) return launch_one_row<T, SRC, PEN, BAND, true>(backward, a, B, sh, longseq, stream, what);
  }
  return launch_one_row<T, SRC, PEN, BAND, false>(backward, a, B, sh, longseq, stream, what);
}

// One direction of the sweep for a cost source, with or without the penalty
// recursion; the band is taken from a.band. Explicitly instantiated in
// udtw_sweep_<type>_<direction>.hip, so the kernel instantiations of the
// four combinations compile in parallel.
template <typename T, int SRC, bool BWD>
int launch_sweep(bool pen, const UdtwArgs<T>& a, int B, hipStream_t s, const char* what) {
  const bool band = a.band > (T)0;
  if (pen)
    return band ? launch_udtw<T, SRC, true, true>(BWD, a, B, s, what)
                : launch_udtw<T, SRC, true, false>(BWD, a, B, s, what);
  return band ? launch_udtw<T, SRC, false, true>(BWD, a, B, s, what)
              : launch_udtw<T, SRC, false, false>(BWD, a, B, s, what);
}

#define TW_SWEEP_EXTERN(T_, BWD_)                                                            \
  extern template int launch_sweep<T_, SRC_COST, BWD_>(bool, const UdtwArgs<T_>&, int,       \
                                                       hipStream_t, const char*);            \
  extern template int launch_sweep<T_, SRC_SQ, BWD_>(bool, const UdtwArgs<T_>&, int,         \
                                                     hipStream_t, const char*);              \
  extern template int launch_sweep<T_, SRC_FEAT1, BWD_>(bool, const UdtwArgs<T_>&, int,      \
                                                        hipStream_t, const char*);
#ifndef TW_SWEEP_INSTANTIATE
TW_SWEEP_EXTERN(float, false)
TW_SWEEP_EXTERN(float, true)
TW_SWEEP_EXTERN(double, false)
TW_SWEEP_EXTERN(double, true)
#endif
#undef TW_SWEEP_EXTERN

}  // namespace tw
