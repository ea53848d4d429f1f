// Banded uDTW / soft-DTW on precomputed matrices: work and storage in
// proportion to the band.
//
// With a Sakoe-Chiba band |i - j| <= w (reference: the mask of
// udtw_cuda.cu:126-130, udtw/_autograd.py:41-43), only (N + M - 1)(w + 1)
// cells of an N x M grid can carry a finite R. This sweep visits only those:
//
//  * Coordinates. Cell (i, j) has band offset l = i - j + w in [0, 2w] and
//    anti-diagonal d = i + j; on diagonal d only offsets of parity
//    (d + w) mod 2 occur. Slot m covers the offsets 2m and 2m + 1 and at
//    step d computes the one of the right parity, so w + 1 slots cover the
//    band with one cell each per step.
//  * Predecessors. (i-1, j) is offset l - 1 and (i, j-1) offset l + 1 on
//    diagonal d - 1, held by slot m or its neighbour m -/+ 1 depending on the
//    parity; (i-1, j-1) is offset l on diagonal d - 2, the slot's own value
//    from two steps before. The backward mirrors this for the successors.
//  * Mapping. One wavefront per pair, S consecutive slots per lane (w + 1 <=
//    64 S): the neighbour slots are in the same lane or, at the lane's ends,
//    one DPP wave shift away. Nothing goes through the LDS and there is no
//    barrier.
//  * Storage. The forward keeps R (scaled by log2(e) / gamma; in double
//    when float calls carry R in double) and Rbar = R - C, and P and
//    Pbar = P - Q, band-compressed: per diagonal d, row 2d holds R (P) and
//    row 2d + 1 Rbar (Pbar) of its NS slots (NS = w + 1 rounded up to a
//    multiple of S, so that a lane's S slots move as one vector access), in
//    the caller's R / P buffers of N M elements; the launcher takes this
//    path only when the 2 (N + M - 1) NS elements fit. The backward needs
//    nothing else of the forward: it reads the planes with one coalesced
//    access per lane and row, and never the inputs C and Q, whose cells lie
//    along anti-diagonals, one cache line per lane. The inputs are read, and
//    the gradients written, only inside the band; further workgroups of the
//    backward's launch zero the gradients outside it, alongside the sweep.
//  * Addressing. A slot's cells of one parity lie on a line through the
//    N x M plane: the offset of its cell on diagonal d is linear in d, and
//    the diagonals on which it is inside the grid form one range, both set
//    up once per slot, so a step costs no index arithmetic beyond a multiply
//    add and two compares per slot.
//  * Loads run PD steps ahead in a register ring (the step loop is unrolled
//    by PD), so their latency stays off the chain of dependent steps.
//
// Arithmetic per cell is the general sweep's: R = C + softmin of the three
// predecessors, P = Q + their softmax-weighted P; the backward's adjoints
// G (of R, seeded with grad_r) and A (of P, seeded with grad_p),
//   G_k = sum_s w_s (G_s - A_s (P_k - Pbar_s) / gamma),  A_k = sum_s w_s A_s,
// w_s = exp((Rbar_s - R_k) / gamma), Rbar_s = R_s - C_s, Pbar_s = P_s - Q_s.
#include <type_traits>

#include "tw_capi.hpp"
#include "tw_common.hpp"
#include "udtw_band.hpp"

namespace tw {
namespace {

template <typename RT>
__device__ __forceinline__ RT band_big() {
  return (RT)0x1p100;
}

template <typename T, typename RT>
struct BandArgs {
  const T *C, *Q;      // [B,N,M]
  RT* R;               // band planes [B][D][NS]
  T* P;
  T *out_r, *out_p;    // forward [B]
  const T *gr, *gp;    // backward [B], element stride gstride
  int gstride;
  T *dC, *dQ;          // backward [B,N,M] (inside the band), or the band layout
  T *zC, *zQ;          // backward: the [B,N,M] planes zeroed outside the band
  int N, M, w, NS, D;
  int B, nzero;        // pairs; backward: workgroups past B zero outside the band
  T k, inv_k, inv_gamma;
};

// Where slot m's cells of parity p lie: band offset l = 2m + p, cell
// (i, j) = ((d + l - w) / 2, (d - l + w) / 2) on the diagonals d of that
// parity, in the grid for d in [lo, hi] (empty when lo > hi). The byte
// offset of the cell in a row-major N x M plane is linear in d:
// (d (M + 1) + (l - w)(M - 1)) / 2 elements (unsigned arithmetic: exact for
// the cells in the grid, whose offsets are below 2^31 bytes).
struct SlotCells {
  int lo, hi;
  unsigned a;   // (l - w)(M - 1), two's complement
  __device__ __forceinline__ void init(int m, int p, int w, int N, int M) {
    const int l = 2 * m + p;
    int lo_ = l - w > w - l ? l - w : w - l;                 // i >= 0, j >= 0
    const int hi1 = 2 * N - 2 + w - l, hi2 = 2 * M - 2 + l - w;   // i <= N-1, j <= M-1
    int hi_ = hi1 < hi2 ? hi1 : hi2;
    if (l > 2 * w) {
      lo_ = 1;
      hi_ = 0;
    }
    lo = lo_;
    hi = hi_;
    a = (unsigned)((l - w) * (M - 1));
  }
  __device__ __forceinline__ bool ok(int d) const { return d >= lo && d <= hi; }
  // The cell's byte offset, or kOob off the grid.
  __device__ __forceinline__ int off(int d, int M, int es) const {
    return ok(d) ? (int)((((unsigned)d * (unsigned)(M + 1) + a) >> 1) * (unsigned)es) : kOob;
  }
  // The same with one of 2^31 and above (out of any buffer's range) off the
  // grid, by integer arithmetic: no select, so that the compiler has no
  // condition to turn the accesses into branches on.
  __device__ __forceinline__ int off_bits(int d, int M, int es) const {
    const unsigned raw = (((unsigned)d * (unsigned)(M + 1) + a) >> 1) * (unsigned)es;
    const unsigned out = (unsigned)(((d - lo) | (hi - d)) >> 31);   // all ones off the grid
    return (int)(raw | (out & 0x80000000u));
  }
};

// The backward stores the gradients in pairs along rows: the cell (i, j)
// of a slot takes (i, j) and (i, j + 1), its right successor, whose G the
// step holds already, as one aligned 8-byte (float) or 16-byte (double)
// store, when the absolute element index of (i, j) is even; a cell with an
// odd index is taken by its left neighbour's pair. The pairs of one store
// instruction cover half the cache lines that one cell per lane would.
// Pair writers are the cells of band offsets l in [0, 2w + 1] (l = 2w + 1 is
// outside the band: it writes the zero there and the band's cell to its
// right) with i in [0, N - 1], j in [0, M - 2], i.e. the steps d in [lo, hi].
// Left over are the cells with an odd index in column 0 and those with an
// even index in column M - 1, stored one by one (at steps dj0 and djm).
struct PairCells : SlotCells {
  int dj0, djm;
  __device__ __forceinline__ void init(int m, int p, int w, int N, int M) {
    const int l = 2 * m + p;
    lo = l - w > w - l ? l - w : w - l;
    const int hi1 = 2 * N - 2 + w - l, hi2 = 2 * M - 4 + l - w;
    hi = hi1 < hi2 ? hi1 : hi2;
    if (l > 2 * w + 1) {
      lo = 1;
      hi = 0;
    }
    a = (unsigned)((l - w) * (M - 1));
    dj0 = l >= w ? l - w : -(1 << 30);   // the step of its cell in column 0
    djm = 2 * M - 2 + l - w;             // ... in column M - 1
  }
  // byte offset of the pair, or one past 2^31 where the cell writes no pair
  // (par: parity of the plane's element index at offset 0)
  __device__ __forceinline__ int pair_off(int d, int M, int esh, unsigned par) const {
    const unsigned raw = ((unsigned)d * (unsigned)(M + 1) + a) >> 1;   // element index
    const unsigned out = (unsigned)(((d - lo) | (hi - d)) >> 31) | ((raw ^ par) & 1u);
    return (int)((raw << esh) | (out << 31));
  }
};

// x where keep is all ones, fill where it is zero (bitwise).
__device__ __forceinline__ float bsel(float x, float fill, unsigned keep) {
  return __uint_as_float((__float_as_uint(x) & keep) | (__float_as_uint(fill) & ~keep));
}
__device__ __forceinline__ double bsel(double x, double fill, unsigned keep) {
  const unsigned long long k = (unsigned long long)(long long)(int)keep;
  return __longlong_as_double((long long)(((unsigned long long)__double_as_longlong(x) & k) |
                                          ((unsigned long long)__double_as_longlong(fill) & ~k)));
}

template <typename T>
__device__ __forceinline__ T tmin3(T a, T b, T c) {
  return fmin(a, fmin(b, c));
}

// S consecutive band slots of one lane, contiguous in a band plane: moved as
// one access of S elements where that is 8 or 16 bytes wide.
template <typename V, int S>
__device__ __forceinline__ void ld_slots(const Buf& b, int o, V (&x)[S]) {
  if constexpr (S * sizeof(V) == 16) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const u4 w = __builtin_amdgcn_raw_buffer_load_b128(b.r, o, 0, 0);
    if constexpr (sizeof(V) == 4) {
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] = __uint_as_float(w[k]);
    } else {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        x[k] = __longlong_as_double((long long)(((unsigned long long)w[2 * k + 1] << 32) | w[2 * k]));
    }
  } else if constexpr (S * sizeof(V) == 8 && sizeof(V) == 4) {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    const u2 w = __builtin_amdgcn_raw_buffer_load_b64(b.r, o, 0, 0);
    x[0] = __uint_as_float(w.x);
    x[1] = __uint_as_float(w.y);
  } else {
#pragma unroll
    for (int k = 0; k < S; ++k) x[k] = b.ld<V>(o == kOob ? kOob : o + k * (int)sizeof(V), 0);
  }
}
template <typename V, int S>
__device__ __forceinline__ void st_slots(const Buf& b, int o, const V (&x)[S]) {
  if constexpr (S * sizeof(V) == 16) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    u4 w;
    if constexpr (sizeof(V) == 4) {
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = __float_as_uint(x[k]);
    } else {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const unsigned long long u = (unsigned long long)__double_as_longlong(x[k]);
        w[2 * k] = (unsigned)u;
        w[2 * k + 1] = (unsigned)(u >> 32);
      }
    }
    __builtin_amdgcn_raw_buffer_store_b128(w, b.r, o, 0, 0);
  } else if constexpr (S * sizeof(V) == 8 && sizeof(V) == 4) {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    const u2 w = {__float_as_uint(x[0]), __float_as_uint(x[1])};
    __builtin_amdgcn_raw_buffer_store_b64(w, b.r, o, 0, 0);
  } else {
#pragma unroll
    for (int k = 0; k < S; ++k) b.st(x[k], o == kOob ? kOob : o + k * (int)sizeof(V), 0);
  }
}

// Materializes x in registers at this point of the program.
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(double& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(unsigned& x) { asm volatile("" : "+v"(x)); }

// The end cell (N-1, M-1): band offset N - M + w on the last diagonal.
__device__ __forceinline__ int end_slot(int N, int M, int w) { return (N - M + w) >> 1; }

// ------------------------------------------------------------ forward

// BIO: C and Q in the band layout [B][D][NS] (slot m of diagonal d at
// d NS + m) instead of [B, N, M].
template <typename T, typename RT, int S, bool PEN, int WP, bool BIO>
__global__ void __launch_bounds__(64) udtw_band_fwd(BandArgs<T, RT> a) {
  constexpr int PD = 8;   // prefetch distance (steps) = unroll of the step loop
  const int b = blockIdx.x, lane = threadIdx.x;
  const int N = a.N, M = a.M, w = a.w, NS = a.NS, D = a.D;
  const RT BIG = band_big<RT>();
  const size_t nm = (size_t)N * M, bsz = (size_t)2 * D * NS;
  const size_t isz = BIO ? (size_t)D * NS : nm;
  Buf bc, bq, br, bp;
  bc.init(a.C + b * isz, (long long)isz);
  if (PEN) bq.init(a.Q + b * isz, (long long)isz);
  br.init(a.R + b * bsz, (long long)bsz);
  if (PEN) bp.init(a.P + b * bsz, (long long)bsz);
  constexpr int es = (int)sizeof(T), rs = (int)sizeof(RT);
  const int m0 = lane * S;
  const bool lane_in = m0 < NS;   // the lane's slots exist in the plane

  SlotCells sc[2][S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    sc[0][s].init(m0 + s, 0, w, N, M);
    sc[1][s].init(m0 + s, 1, w, N, M);
  }
  // R and P of the slots at steps d - 1 and d - 2; the cell (0, 0) (slot
  // w >> 1 at step 0) has the diagonal predecessor R = 0
  RT r1[S], r2[S];
  T q1[S], q2[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    r1[s] = BIG;
    r2[s] = (m0 + s == (w >> 1)) ? (RT)0 : BIG;
    q1[s] = q2[s] = (T)0;
  }
  // ring of the inputs PD steps ahead: [step mod PD][slot]
  T cr[PD][S], qr[PD][S];
  auto fetch = [&](int d, int u) {
    if constexpr (BIO) {
      // the lane's S slots as one access; rows d >= D lie past the planes
      const int o = lane_in ? (d * NS + m0) * es : kOob;
      ld_slots<T, S>(bc, o, cr[u]);
      if (PEN) ld_slots<T, S>(bq, o, qr[u]);
    } else {
      const int p = (u & 1) ^ WP;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int o = sc[p][s].off(d, M, es);
        cr[u][s] = bc.ld<T>(o, 0);
        if (PEN) qr[u][s] = bq.ld<T>(o, 0);
      }
    }
  };
  // in ring order: the loop's first use of each entry then waits only for
  // that entry's loads, on the first pass as on the later ones
#pragma unroll
  for (int u = 0; u < PD; ++u) {
    fetch(u, u);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Whole blocks of PD steps: the steps past D - 1 find no cell in the grid,
  // and their stores fall past the end of the band planes, where the buffer
  // range drops them. (Leaving the block early instead would make the
  // compiler wait for every load in flight at the top of each block.)
  for (int d0 = 0; d0 < D; d0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      const int d = d0 + u;
      const int p = (u & 1) ^ WP;   // offsets 2m + p are on this diagonal
      const RT lo = shift_prev(r1[S - 1], BIG), hi = shift_next(r1[0], BIG);
      T qlo = 0, qhi = 0;
      if (PEN) {
        qlo = shift_prev(q1[S - 1], (T)0);
        qhi = shift_next(q1[0], (T)0);
      }
      RT nr[S], nrb[S];
      T nq[S], nqb[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const bool ok = sc[p][s].ok(d);
        const RT rm = s > 0 ? r1[s - 1] : lo, rp = s < S - 1 ? r1[s + 1] : hi;
        // up (i-1, j) is offset l - 1, left (i, j-1) offset l + 1, both at d - 1
        const RT up = p ? r1[s] : rm, lf = p ? rp : r1[s], dg = r2[s];
        const RT mn = tmin3(up, lf, dg);
        const T eu = ex2((T)(mn - up)), el = ex2((T)(mn - lf)), ed = ex2((T)(mn - dg));
        const T sm = eu + el + ed;
        const RT rb = mn - (RT)lg2(sm);
        const RT rh = (RT)(cr[u][s] * a.k) + rb;
        T pb = (T)0, ph = (T)0;
        if (PEN) {
          const T qm = s > 0 ? q1[s - 1] : qlo, qp = s < S - 1 ? q1[s + 1] : qhi;
          const T pu = p ? q1[s] : qm, pl = p ? qp : q1[s], pd = q2[s];
          pb = (eu * pu + el * pl + ed * pd) * rcp(sm);
          ph = qr[u][s] + pb;
        }
        nr[s] = ok ? rh : BIG;
        nrb[s] = ok ? rb : -BIG;
        nq[s] = ok ? ph : (T)0;
        nqb[s] = ok ? pb : (T)0;
      }
      // rows 2d (R, P) and 2d + 1 (Rbar, Pbar): past the planes' end for d >= D
      const int bo = 2 * d * NS + m0;
      st_slots<RT, S>(br, lane_in ? bo * rs : kOob, nr);
      st_slots<RT, S>(br, lane_in ? (bo + NS) * rs : kOob, nrb);
      if (PEN) {
        st_slots<T, S>(bp, lane_in ? bo * es : kOob, nq);
        st_slots<T, S>(bp, lane_in ? (bo + NS) * es : kOob, nqb);
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        r2[s] = r1[s];
        r1[s] = nr[s];
        q2[s] = q1[s];
        q1[s] = nq[s];
      }
      fetch(d + PD, u);
    }
  }
  // the end cell, read back from the band planes: the lane that stored it
  // reads it (a wave's accesses to one address take effect in order; the
  // fence waits for the stores)
  const int me = end_slot(N, M, w);
  if (lane == me / S) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    const int eo = 2 * (D - 1) * NS + me;
    a.out_r[b] = (T)(br.ld<RT>(eo * rs, 0) * (RT)a.inv_k);
    a.out_p[b] = PEN ? bp.ld<T>(eo * es, 0) : (T)0;
  }
}

// ----------------------------------------------------------- backward

// Vector memory instructions of one slot group: S elements of V in one
// access where that is 8 or 16 bytes wide, else S accesses.
template <typename V, int S>
constexpr int slot_accesses() {
  return (S * sizeof(V) == 16 || (S * sizeof(V) == 8 && sizeof(V) == 4)) ? 1 : S;
}
template <typename T, typename RT, int S, bool PEN>
constexpr int band_bwd_depth() {
  // R, Rbar, P, Pbar of the band planes loaded, pairs of dC and dQ stored
  const int ops = 2 * slot_accesses<RT, S>() + (PEN ? 2 * slot_accesses<T, S>() : 0) +
                  (PEN ? 2 : 1) * S;
  const int pd = 2 * (28 / ops);
  return pd < 2 ? 2 : (pd > 8 ? 8 : pd);
}

// Zero the gradients outside the band: rows r = z, z + Z, ... of the B N
// rows of dC / dQ, one workgroup of 64 lanes along each row. These cells are
// disjoint from the sweep's, so the two run side by side in one launch: the
// sweep's B workgroups leave most of the chip idle.
template <typename T>
__device__ void band_zero_rows(T* dC, T* dQ, int B, int N, int M, int w, int z, int Z) {
  const long long rows = (long long)B * N;
  for (long long r = z; r < rows; r += Z) {
    const int i = (int)(r % N);
    T* c = dC + r * M;
    T* q = dQ ? dQ + r * M : nullptr;
    const int jlo = i - w, jhi = i + w;   // the band's columns of row i
    for (int j = threadIdx.x; j < M; j += 64) {
      if (j < jlo || j > jhi) {
        c[j] = (T)0;
        if (q) q[j] = (T)0;
      }
    }
  }
}

// BIO: dC and dQ in the band layout [B][D][NS], every slot of every
// diagonal written (0 off the grid), and no zeroing outside the band.
template <typename T, typename RT, int S, bool PEN, int WP, bool BIO>
__global__ void __launch_bounds__(64) udtw_band_bwd(BandArgs<T, RT> a) {
  if ((int)blockIdx.x >= a.B) {
    band_zero_rows<T>(a.zC, a.zQ, a.B, a.N, a.M, a.w, (int)blockIdx.x - a.B, a.nzero);
    return;
  }
  // prefetch distance (steps, even): as deep as the memory counter (63
  // outstanding accesses) allows for this step's loads and stores
  constexpr int PD = band_bwd_depth<T, RT, S, PEN>();
  const int b = blockIdx.x, lane = threadIdx.x;
  const int N = a.N, M = a.M, w = a.w, NS = a.NS, D = a.D;
  const RT NEG = -band_big<RT>();
  const size_t nm = (size_t)N * M, bsz = (size_t)2 * D * NS;
  const size_t osz = BIO ? (size_t)D * NS : nm;
  Buf br, bp, bdc, bdq;
  br.init(a.R + b * bsz, (long long)bsz);
  if (PEN) bp.init(a.P + b * bsz, (long long)bsz);
  bdc.init(a.dC + b * osz, (long long)osz);
  // without dQ, an empty range: its stores are dropped
  const bool has_dq = PEN && a.dQ != nullptr;
  if (PEN) bdq.init(has_dq ? a.dQ + b * osz : a.dC, has_dq ? (long long)osz : 0LL);
  constexpr int es = (int)sizeof(T), rs = (int)sizeof(RT);
  const T gR = a.gr[(size_t)b * a.gstride];
  const T gP = PEN ? a.gp[(size_t)b * a.gstride] : (T)0;
  const int m0 = lane * S;
  const bool lane_in = m0 < NS;
  // lanes past the planes' slots load 0: they take R = BIG and Rbar = NEG
  // instead, which gives them and their neighbours zero weights
  unsigned keep = lane_in ? ~0u : 0u;
  pin(keep);
  const int me = end_slot(N, M, w);

  SlotCells sc[2][S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    sc[0][s].init(m0 + s, 0, w, N, M);
    sc[1][s].init(m0 + s, 1, w, N, M);
  }
  PairCells pc[2][S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    pc[0][s].init(m0 + s, 0, w, N, M);
    pc[1][s].init(m0 + s, 1, w, N, M);
  }
  constexpr int esh = sizeof(T) == 4 ? 2 : 3;
  // parities of the planes' element indices at this pair's offset 0
  const unsigned par_c = (unsigned)((((size_t)a.dC >> esh) + (size_t)b * nm) & 1);
  const unsigned par_q = has_dq ? (unsigned)((((size_t)a.dQ >> esh) + (size_t)b * nm) & 1) : 0u;
  // successor state of the slots at steps d + 1 and d + 2: Rbar = R - C
  // (NEG outside the grid: weight 0), Pbar = P - Q, and the adjoints G, A.
  // The end cell's diagonal successor is a virtual cell with Rbar = R and
  // Pbar = P of the end cell (weight 1, no penalty term) and adjoints
  // grad_r, grad_p, which seeds G = grad_r and A = grad_p there.
  RT e1[S], e2[S];
  T g1[S], g2[S], a1[S], a2[S], b1[S], b2[S];
  const int eo = 2 * (D - 1) * NS + me;
  const RT r_end = br.ld<RT>(eo * rs, 0);
  const T p_end = PEN ? bp.ld<T>(eo * es, 0) : (T)0;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const bool end = m0 + s == me;
    e1[s] = NEG;
    e2[s] = end ? r_end : NEG;
    g1[s] = a1[s] = b1[s] = (T)0;
    g2[s] = end ? gR : (T)0;
    a2[s] = end ? gP : (T)0;
    b2[s] = end ? p_end : (T)0;
  }
  // ring PD steps ahead: R, Rbar, P, Pbar of each slot's cell, as the
  // forward left them in the band planes
  RT rr[PD][S], rbr[PD][S];
  T pr[PD][S], pbr[PD][S];
  auto fetch = [&](int d, int u) {
    // below diagonal 0 the band-plane offsets are negative, out of the
    // buffer's range as unsigned offsets
    const int bo = 2 * d * NS + m0;
    ld_slots<RT, S>(br, lane_in ? bo * rs : kOob, rr[u]);
    ld_slots<RT, S>(br, lane_in ? (bo + NS) * rs : kOob, rbr[u]);
    if (PEN) {
      ld_slots<T, S>(bp, lane_in ? bo * es : kOob, pr[u]);
      ld_slots<T, S>(bp, lane_in ? (bo + NS) * es : kOob, pbr[u]);
    }
  };
  // the steps run downwards, d = d1 - u, in whole blocks of PD from D - 1:
  // the steps below 0 find no cell in the grid and store nothing
#pragma unroll
  for (int u = 0; u < PD; ++u) {
    fetch(D - 1 - u, u);   // in ring order, as in the forward
    __builtin_amdgcn_sched_barrier(0);
  }
  // One block of PD steps from d1 down; CUTS: with the single stores at the
  // grid's first and last columns, which only the first and last steps need.
  auto block = [&](int d1, auto cuts) {
    constexpr bool CUTS = decltype(cuts)::value;
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      const int d = d1 - u;
      const int p = (u & 1) ^ WP;
      // successors at d + 1: down (i+1, j) is offset l + 1, right (i, j+1)
      // offset l - 1; diagonal (i+1, j+1) offset l at d + 2
      const RT elo = shift_prev(e1[S - 1], NEG), ehi = shift_next(e1[0], NEG);
      const T glo = shift_prev(g1[S - 1], (T)0), ghi = shift_next(g1[0], (T)0);
      T alo = 0, ahi = 0, blo = 0, bhi = 0;
      if (PEN) {
        alo = shift_prev(a1[S - 1], (T)0);
        ahi = shift_next(a1[0], (T)0);
        blo = shift_prev(b1[S - 1], (T)0);
        bhi = shift_next(b1[0], (T)0);
      }
      RT ne[S];
      T ng[S], na[S], nb[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        // successor slots at d + 1: down = p ? m + 1 : m, right = p ? m : m - 1
        const RT em = s > 0 ? e1[s - 1] : elo, ep = s < S - 1 ? e1[s + 1] : ehi;
        const T gm = s > 0 ? g1[s - 1] : glo, gpp = s < S - 1 ? g1[s + 1] : ghi;
        const RT edn = p ? ep : e1[s], ert = p ? e1[s] : em, edg = e2[s];
        const T gdn = p ? gpp : g1[s], grt = p ? g1[s] : gm, gdg = g2[s];
        // a cell off the grid has R = BIG from the forward: zero weights, so
        // G = A = 0 there
        const RT rk = bsel(rr[u][s], -NEG, keep);
        const T wdn = ex2((T)(edn - rk)), wrt = ex2((T)(ert - rk)), wdg = ex2((T)(edg - rk));
        T G = wdn * gdn + wrt * grt + wdg * gdg;
        T A = (T)0;
        if (PEN) {
          const T am = s > 0 ? a1[s - 1] : alo, ap = s < S - 1 ? a1[s + 1] : ahi;
          const T bm = s > 0 ? b1[s - 1] : blo, bpp = s < S - 1 ? b1[s + 1] : bhi;
          const T adn = p ? ap : a1[s], art = p ? a1[s] : am, adg = a2[s];
          const T bdn = p ? bpp : b1[s], brt = p ? b1[s] : bm, bdg = b2[s];
          const T pk = pr[u][s];
          A = wdn * adn + wrt * art + wdg * adg;
          G -= (wdn * adn * (pk - bdn) + wrt * art * (pk - brt) + wdg * adg * (pk - bdg)) *
               a.inv_gamma;
        }
        if constexpr (!BIO) {
        // (i, j) and its right successor (i, j + 1), G = grt, A = art
        st_pair<T>(bdc, pc[p][s].pair_off(d, M, esh, par_c), G, grt);
        if (PEN) {
          const T art = p ? a1[s] : (s > 0 ? a1[s - 1] : alo);
          st_pair<T>(bdq, pc[p][s].pair_off(d, M, esh, par_q), A, art);
        }
        if constexpr (CUTS) {   // the cells left over at columns 0 and M - 1
          const unsigned raw = sc[p][s].ok(d) ? (unsigned)sc[p][s].off(d, M, es) >> esh : 0u;
          const bool ok = sc[p][s].ok(d);
          const bool one_c = ok && ((d == pc[p][s].dj0 && ((raw ^ par_c) & 1u)) ||
                                    (d == pc[p][s].djm && !((raw ^ par_c) & 1u)));
          const bool one_q = PEN && ok && ((d == pc[p][s].dj0 && ((raw ^ par_q) & 1u)) ||
                                           (d == pc[p][s].djm && !((raw ^ par_q) & 1u)));
          if (__builtin_amdgcn_ballot_w64(one_c || one_q)) {
            bdc.st(G, one_c ? (int)(raw << esh) : kOob, 0);
            if (PEN) bdq.st(A, one_q ? (int)(raw << esh) : kOob, 0);
          }
        }
        }
        ne[s] = bsel(rbr[u][s], NEG, keep);
        ng[s] = G;
        na[s] = A;
        nb[s] = PEN ? pbr[u][s] : (T)0;
      }
      if constexpr (BIO) {
        // the lane's S slots as one access; rows d < 0 have negative
        // offsets, out of the buffer's range as unsigned
        const int o = lane_in ? (d * NS + m0) * es : kOob;
        st_slots<T, S>(bdc, o, ng);
        if (PEN) st_slots<T, S>(bdq, o, na);
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        e2[s] = e1[s];
        e1[s] = ne[s];
        g2[s] = g1[s];
        g1[s] = ng[s];
        a2[s] = a1[s];
        a1[s] = na[s];
        b2[s] = b1[s];
        b1[s] = nb[s];
      }
      // The new state is computed here, before the ring entry it came from
      // is reloaded: computed later (at its uses in the next steps), it would
      // keep the old entry alive past the reload, and the loop's back edge
      // would need copies of the ring, each waiting for its load.
#pragma unroll
      for (int s = 0; s < S; ++s) {
        pin(e1[s]);
        pin(g1[s]);
        if (PEN) {
          pin(a1[s]);
          pin(b1[s]);
        }
      }
      fetch(d - PD, u);
      __builtin_amdgcn_sched_barrier(0);   // ring order, as in the prologue
    }
  };
  // A slot meets column 0 at d = l - w <= w and column M - 1 at
  // d = 2M - 2 + l - w >= 2N - 2 - w (N <= M): the blocks between take no
  // single stores.
  const int a_lo = 2 * N - w - 3, c_hi = w + 1;
  int d1 = D - 1;
  for (; d1 >= 0 && d1 >= a_lo; d1 -= PD) block(d1, std::true_type());
  for (; d1 - PD + 1 > c_hi; d1 -= PD) block(d1, std::false_type());
  for (; d1 >= 0; d1 -= PD) block(d1, std::true_type());
}

int band_slots(int w) {
  const int ns = w + 1;
  return ns <= 64 ? 1 : (ns <= 128 ? 2 : (ns <= 256 ? 4 : 0));
}

template <typename T, typename RT, int S, bool PEN, bool BIO>
int band_launch(bool bwd, const BandArgs<T, RT>& a, int B, hipStream_t s) {
  // parity of step 0 (forward) / of step D - 1 (backward)
  const int wp = bwd ? ((a.D - 1 + a.w) & 1) : (a.w & 1);
  if (bwd) {
    // The sweep's waves issue one dependent step after another: a wave of
    // the zeroing role beside one on its SIMD would take issue cycles from
    // it. While the sweep's workgroups leave CUs free, an LDS reservation
    // (unused) of over half a CU's LDS keeps every workgroup on a CU of its
    // own; with more pairs than CUs it would serialise the sweeps instead.
    const dim3 grid((unsigned)(B + a.nzero));
    const size_t lds = a.nzero > 0 && B <= num_cus() ? (size_t)max_lds_bytes() / 2 + 256 : 0;
    if (wp)
      hipLaunchKernelGGL((udtw_band_bwd<T, RT, S, PEN, 1, BIO>), grid, dim3(64), lds, s, a);
    else
      hipLaunchKernelGGL((udtw_band_bwd<T, RT, S, PEN, 0, BIO>), grid, dim3(64), lds, s, a);
  } else {
    if (wp)
      hipLaunchKernelGGL((udtw_band_fwd<T, RT, S, PEN, 1, BIO>), dim3(B), dim3(64), 0, s, a);
    else
      hipLaunchKernelGGL((udtw_band_fwd<T, RT, S, PEN, 0, BIO>), dim3(B), dim3(64), 0, s, a);
  }
  return TW_OK;
}

template <typename T, typename RT>
int band_run(bool bwd, bool bio, const UdtwArgs<T>& u, int B, hipStream_t s, const char* what,
             T* zero_c, T* zero_q) {
  BandArgs<T, RT> a;
  a.C = u.C;
  a.Q = u.Q;
  a.R = reinterpret_cast<RT*>(u.R);
  a.P = u.P;
  a.out_r = u.out_r;
  a.out_p = u.out_p;
  a.gr = u.gr;
  a.gp = u.gp;
  a.gstride = u.gstride;
  a.dC = u.dC;
  a.dQ = u.dQ;
  // the zeros outside the band: into dC / dQ themselves, or with the band
  // layout into the given [B, N, M] planes (none given: no zeroing)
  a.zC = bio ? zero_c : u.dC;
  a.zQ = bio ? zero_q : u.dQ;
  a.N = u.N;
  a.M = u.M;
  a.w = (int)u.band;
  // slots per diagonal in the band planes: w + 1, rounded up to whole lanes
  // of S slots so that a lane's slots move as one access
  const int S = band_slots(a.w);
  a.NS = (a.w + 1 + S - 1) / S * S;
  a.D = u.N + u.M - 1;
  a.B = B;
  // zeroing workgroups: at least 4 rows each, at most 1024
  const long long rows = (long long)B * u.N;
  a.nzero = bwd && a.zC ? (int)((rows + 3) / 4 < 1024 ? (rows + 3) / 4 : 1024) : 0;
  a.k = u.k;
  a.inv_k = u.inv_k;
  a.inv_gamma = u.inv_gamma;
  // the penalty: on when Q is given; from features (band_io, beta != 0) the
  // backward has no Q to give
  const bool pen = u.Q != nullptr || (bio && u.beta != (T)0);
#define TW_BAND(S_)                                                             \
  (bio ? (pen ? band_launch<T, RT, S_, true, true>(bwd, a, B, s)                \
              : band_launch<T, RT, S_, false, true>(bwd, a, B, s))              \
       : (pen ? band_launch<T, RT, S_, true, false>(bwd, a, B, s)               \
              : band_launch<T, RT, S_, false, false>(bwd, a, B, s)))
  if (S == 1)
    TW_BAND(1);
  else if (S == 2)
    TW_BAND(2);
  else
    TW_BAND(4);
#undef TW_BAND
  return check_launch(what);
}

}  // namespace

int band_mode() {
  static const int mode = [] {
    const char* e = getenv("TORCHWARP_UDTW_BAND");
    return e ? atoi(e) : -1;
  }();
  return mode;
}

bool band_path(int N, int M, double band) {
  if (!(band > 0) || band_mode() == 0) return false;
  const double wd = band < 1e9 ? band : 1e9;
  const long long w = (long long)wd;   // |i - j| <= band  <=>  |i - j| <= floor(band)
  const int S = band_slots((int)(w < 1 << 20 ? w : 1 << 20));
  if (S == 0) return false;
  // a band narrower than the grid, whose compressed planes (two rows of
  // w + 1 slots per diagonal, rounded up to a multiple of S) fit in N M
  // elements
  if (w >= (N < M ? N : M) - 1) return false;
  // the end cell inside the band (N <= M: M - N <= w)
  if ((long long)M - N > w) return false;
  const long long ns = (w + 1 + S - 1) / S * S;
  return 2 * (long long)(N + M - 1) * ns <= (long long)N * M;
}

template <typename T>
int band_sweep(bool bwd, const UdtwArgs<T>& a, int B, hipStream_t s, const char* what,
               bool band_io, T* zero_c, T* zero_q) {
  if (B == 0) return TW_OK;
  // planes are addressed with 32-bit byte offsets within a pair
  const long long rbytes = a.rd ? 8 : (long long)sizeof(T);
  if ((long long)a.N * a.M * rbytes >= (1LL << 31)) {
    return fail(TW_ESIZE, "%s: one pair's N*M matrix (%d x %d) must stay below 2 GiB", what,
                a.N, a.M);
  }
  if (sizeof(T) == 4 && a.rd)
    return band_run<T, double>(bwd, band_io, a, B, s, what, zero_c, zero_q);
  return band_run<T, T>(bwd, band_io, a, B, s, what, zero_c, zero_q);
}

template int band_sweep<float>(bool, const UdtwArgs<float>&, int, hipStream_t, const char*, bool,
                               float*, float*);
template int band_sweep<double>(bool, const UdtwArgs<double>&, int, hipStream_t, const char*,
                                bool, double*, double*);

// ----------------------------------------------------- from features (F > 1)
//
// The band's cost C = max(S, 0) / var and penalty Q = beta ln var, S the
// squared distance of rows i and j, var = max(h(vx_i) + h(vy_j), eps), are
// built only inside the band, in the band layout the sweep reads: element
// d NS + m of a pair's plane holds the cell of slot m on diagonal d (0 off
// the grid). The backward sweep leaves dC / dQ in the same layout, and the
// feature gradients are reduced from them row by row and column by column.

namespace {

template <typename T>
struct BandFeat {
  const T *X, *Y, *VX, *VY;   // [B,N,F], [B,M,F], [B,N], [B,M]
  T *Cb, *Qb;                 // band layout [B][D][NS] (Qb null without a penalty)
  const T *dCb, *dQb;         // the backward sweep's gradients, same layout
  T *dX, *dY, *dVX, *dVY;     // dVX / dVY may be null
  int N, M, F, w, NS, D;
  T hv1, hv0, eps, beta, beta_ln2;
  int sigma;
};

template <typename T>
__device__ __forceinline__ T bf_hvar(const BandFeat<T>& a, T v) {
  return v * fma(a.hv1, v, a.hv0);
}

constexpr int kBfDiags = 32;   // diagonals per workgroup of the builder

// XCD-aware placement. Workgroup ids go round-robin over the device's kXcds
// XCDs (MI355X: 8), each with its own L2; pair b's W workgroups take the ids
// congruent to b modulo kXcds, so a pair's features and band planes are
// read through one L2. Launch ceil(B / kXcds) kXcds W workgroups; returns
// false for the ids past the last pair. (On another XCD count the mapping
// stays exact and only the locality changes.)
constexpr int kXcds = 8;
__device__ __forceinline__ bool xcd_place(int W, int B, int& b, int& local) {
  const int id = (int)blockIdx.x, x = id % kXcds, r = id / kXcds;
  b = x + kXcds * (r / W);
  local = r % W;
  return b < B;
}
static unsigned xcd_grid(int W, int B) {
  return (unsigned)((B + kXcds - 1) / kXcds) * kXcds * (unsigned)W;
}

// A row of F <= FM features into registers: 16-byte loads where the rows
// are 16-byte aligned (V16), else one element at a time.
template <typename T, int FM, bool V16>
__device__ __forceinline__ void bf_row(const T* p, int F, T (&r)[FM]) {
  if constexpr (V16) {
    constexpr int EV = 16 / (int)sizeof(T);
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int q = 0; q < FM / EV; ++q) {
      if (q * EV < F) {
        const u4 w = *reinterpret_cast<const u4*>(p + q * EV);
        if constexpr (sizeof(T) == 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) r[q * 4 + e] = __uint_as_float(w[e]);
        } else {
          r[q * 2] = __longlong_as_double((long long)(((unsigned long long)w[1] << 32) | w[0]));
          r[q * 2 + 1] =
              __longlong_as_double((long long)(((unsigned long long)w[3] << 32) | w[2]));
        }
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < FM; ++k)
      if (k < F) r[k] = p[k];
  }
}

// One lane per slot m, walking kBfDiags diagonals. From one diagonal to the
// next a slot's cell moves down a row (offset parity 0) or right a column
// (parity 1), so each step loads one new row of X or of Y, and the lanes of
// a wavefront load consecutive rows and store consecutive elements.
// F <= FM; the squared distance sums the features in order with fma.
template <typename T, bool PEN, int FM, bool V16>
__global__ void __launch_bounds__(64) band_feat_build(BandFeat<T> a, int B, int ngx) {
  int b, local;
  if (!xcd_place(ngx * ((a.D + kBfDiags - 1) / kBfDiags), B, b, local)) return;
  const int gx = local % ngx, gy = local / ngx;
  const int m = gx * 64 + threadIdx.x;
  if (m >= a.NS) return;
  const int N = a.N, M = a.M, F = a.F, w = a.w, NS = a.NS;
  const T* X = a.X + (size_t)b * N * F;
  const T* Y = a.Y + (size_t)b * M * F;
  const T* VX = a.VX + (size_t)b * N;
  const T* VY = a.VY + (size_t)b * M;
  const size_t pb = (size_t)b * a.D * NS;
  const int d0 = gy * kBfDiags;
  const int d1 = d0 + kBfDiags < a.D ? d0 + kBfDiags : a.D;
  // the slot's cell at d0 (2i, 2j), and the rows it holds (clamped to the grid)
  int i2 = d0 + 2 * m + ((d0 + w) & 1) - w;
  int j2 = 2 * d0 - i2;
  T x[FM], y[FM];
#pragma unroll
  for (int k = 0; k < FM; ++k) x[k] = y[k] = (T)0;
  auto clampi = [](int v, int n) { return v < 0 ? 0 : (v > n - 1 ? n - 1 : v); };
  bf_row<T, FM, V16>(X + (size_t)clampi(i2 >> 1, N) * F, F, x);
  bf_row<T, FM, V16>(Y + (size_t)clampi(j2 >> 1, M) * F, F, y);
  for (int d = d0; d < d1; ++d) {
    const int l = 2 * m + ((d + w) & 1);
    if (d > d0) {
      // parity 0 at d - 1: the cell moved down a row, else right a column
      if (((d - 1 + w) & 1) == 0) {
        i2 += 2;
        bf_row<T, FM, V16>(X + (size_t)clampi(i2 >> 1, N) * F, F, x);
      } else {
        j2 += 2;
        bf_row<T, FM, V16>(Y + (size_t)clampi(j2 >> 1, M) * F, F, y);
      }
    }
    T c = (T)0, q = (T)0;
    if (l <= 2 * w && i2 >= 0 && j2 >= 0 && i2 < 2 * N && j2 < 2 * M) {
      const int i = i2 >> 1, j = j2 >> 1;
      T sq = (T)0;
#pragma unroll
      for (int k = 0; k < FM; ++k) {
        if (k < F) {
          const T df = x[k] - y[k];
          sq = fma(df, df, sq);
        }
      }
      const T var = fmax(bf_hvar(a, VX[i]) + bf_hvar(a, VY[j]), a.eps);
      c = (sq > (T)0 ? sq : (T)0) * rcp(var);
      if (PEN) q = a.beta_ln2 * lg2(var);
    }
    const size_t o = pb + (size_t)d * NS + m;
    a.Cb[o] = c;
    if (PEN) a.Qb[o] = q;
  }
}

// Any F (features summed in order with fma, as above): both rows loaded per
// cell.
template <typename T, bool PEN>
__global__ void __launch_bounds__(64) band_feat_build_any(BandFeat<T> a, int B, int ngx) {
  int b, local;
  if (!xcd_place(ngx * ((a.D + kBfDiags - 1) / kBfDiags), B, b, local)) return;
  const int gx = local % ngx, gy = local / ngx;
  const int m = gx * 64 + threadIdx.x;
  if (m >= a.NS) return;
  const int N = a.N, M = a.M, F = a.F, w = a.w, NS = a.NS;
  const T* X = a.X + (size_t)b * N * F;
  const T* Y = a.Y + (size_t)b * M * F;
  const size_t pb = (size_t)b * a.D * NS;
  const int d0 = gy * kBfDiags;
  const int d1 = d0 + kBfDiags < a.D ? d0 + kBfDiags : a.D;
  for (int d = d0; d < d1; ++d) {
    const int l = 2 * m + ((d + w) & 1);
    const int i2 = d + l - w, j2 = d - l + w;   // 2i and 2j
    T c = (T)0, q = (T)0;
    if (l <= 2 * w && i2 >= 0 && j2 >= 0 && i2 < 2 * N && j2 < 2 * M) {
      const int i = i2 >> 1, j = j2 >> 1;
      const T* xr = X + (size_t)i * F;
      const T* yr = Y + (size_t)j * F;
      T sq = (T)0;
      for (int k = 0; k < F; ++k) {
        const T df = xr[k] - yr[k];
        sq = fma(df, df, sq);
      }
      const T var =
          fmax(bf_hvar(a, a.VX[(size_t)b * N + i]) + bf_hvar(a, a.VY[(size_t)b * M + j]), a.eps);
      c = (sq > (T)0 ? sq : (T)0) * rcp(var);
      if (PEN) q = a.beta_ln2 * lg2(var);
    }
    const size_t o = pb + (size_t)d * NS + m;
    a.Cb[o] = c;
    if (PEN) a.Qb[o] = q;
  }
}

// The reducer walks, per lane, the cells of its row (or column) "own" in
// order: step t in [0, 2w] is the cell with the other index own - w + t, on
// diagonal 2 own - w + t, in slot (2w - t) / 2 (rows) or t / 2 (columns).
// The 64 lanes of a workgroup take 64 consecutive rows (columns) and kT
// steps at a time, those whose cells lie in one aligned block of kT / 2
// slots (64 bytes). Their cells lie in a tile of 127 + kT diagonals by those
// slots of the band planes, and their other indices in 63 + kT consecutive
// rows of the other side's features: the workgroup loads both into LDS with
// contiguous reads, one 64-byte sector per diagonal and plane (a lane's own
// cells are spread one per diagonal, one cache line each), and the steps
// read only LDS. A whole tile's loads are held in registers, which float
// affords at 32 steps per tile and double at 16.
template <typename T>
struct BgTile {
  static constexpr int kT = sizeof(T) == 4 ? 32 : 16;
  static constexpr int kTD = 127 + kT;   // diagonals of a tile
  static constexpr int kSL = kT / 2;     // slots of a tile: 64 bytes
  static constexpr int kTS = kSL + 1;    // LDS row of a diagonal (odd: rows 2
                                         // apart start on different banks)
  static constexpr int kTR = 63 + kT;    // other-side rows of a tile
};
constexpr int kBfChunk = 16;             // features per pass

// Workgroups [0, nrb) take rows i, the others columns j: the lane of row i
// sums its band cells (i, j) for j ascending, the lane of column j its cells
// (i, j) for i ascending (a fixed order: deterministic). Per cell, as the
// general sweep's backward: dS = dC / var where S > 0, and
// dvar = (beta dQ - dC C) / var, half of it to each side's half variance.
template <typename T, bool PEN>
__global__ void __launch_bounds__(64) band_feat_grad(BandFeat<T> a, int B, int nrb, int ncb) {
  constexpr int NPL = PEN ? 3 : 2;
  constexpr int kBgT = BgTile<T>::kT, kBgTD = BgTile<T>::kTD, kSL = BgTile<T>::kSL,
                kBgTS = BgTile<T>::kTS, kBgTR = BgTile<T>::kTR;
  // feature rows padded by 16 bytes: the 16-byte reads of consecutive rows
  // by consecutive lanes fall on distinct banks
  constexpr int YP = kBfChunk + 16 / (int)sizeof(T);
  __shared__ T tile[NPL][kBgTD * kBgTS];
  __shared__ __align__(16) T yt[kBgTR * YP];
  __shared__ T hvt[kBgTR];
  int b, g;
  if (!xcd_place(nrb + ncb, B, b, g)) return;
  const bool rows = g < nrb;
  const int lane = threadIdx.x;
  const int o0 = (g - (rows ? 0 : nrb)) * 64;
  const int own = o0 + lane;
  const int N = a.N, M = a.M, F = a.F, w = a.w, NS = a.NS, D = a.D;
  const int n_own = rows ? N : M, n_oth = rows ? M : N;
  const bool lane_in = own < n_own;
  const int ownc = lane_in ? own : n_own - 1;
  const T* xown = (rows ? a.X + (size_t)b * N * F : a.Y + (size_t)b * M * F) + (size_t)ownc * F;
  const T* oth = rows ? a.Y + (size_t)b * M * F : a.X + (size_t)b * N * F;
  const T* vown = rows ? a.VX + (size_t)b * N : a.VY + (size_t)b * M;
  const T* voth = rows ? a.VY + (size_t)b * M : a.VX + (size_t)b * N;
  const size_t pb = (size_t)b * D * NS;
  Buf bpl[NPL], bo;
  bpl[0].init(a.Cb + pb, (long long)D * NS);
  bpl[1].init(a.dCb + pb, (long long)D * NS);
  if (PEN) bpl[NPL - 1].init(a.dQb + pb, (long long)D * NS);
  bo.init(oth, (long long)n_oth * F);
  Buf bv;
  bv.init(voth, (long long)n_oth);
  constexpr int es = (int)sizeof(T);
  const T hv = bf_hvar(a, vown[ownc]);
  T dv = (T)0;
  for (int f0 = 0; f0 < F; f0 += kBfChunk) {
    const int fc = F - f0 < kBfChunk ? F - f0 : kBfChunk;
    T acc[kBfChunk], xo[kBfChunk];
#pragma unroll
    for (int k = 0; k < kBfChunk; ++k) {
      acc[k] = (T)0;
      xo[k] = k < fc ? xown[f0 + k] : (T)0;
    }
    // Tile kt holds the steps whose cells lie in slots [kSL kt, kSL kt + kSL)
    // (one 64-byte sector of each diagonal): steps from tA = 2w - kT kt -
    // kT + 1 (rows) or kT kt (columns), on diagonals from 2 o0 - w + tA,
    // with other-side rows from o0 - w + tA. Rows take the tiles in
    // descending kt, columns ascending, so a lane adds its cells in
    // ascending step order. All of a tile's global loads are issued at once,
    // a tile ahead, into registers (the LDS allows one wavefront per SIMD,
    // so registers are free), and are in flight while the tile before is
    // reduced; cells off the planes and rows off the grid load 0 by the
    // buffer's range check.
    constexpr int TE = kBgTD * kSL, TB = (TE + 63) / 64;
    constexpr int YE = kBgTR * kBfChunk, YB = (YE + 63) / 64;
    constexpr int HB = (kBgTR + 63) / 64;
    const int KT = 2 * w / kBgT + 1;
    auto tile_kt = [&](int i) { return rows ? KT - 1 - i : i; };
    auto tile_t0 = [&](int kt) { return rows ? 2 * w - kBgT * kt - kBgT + 1 : kBgT * kt; };
    T v[NPL][TB], vy[YB], vh[HB];
    auto fetch = [&](int kt) {
      const int tA = tile_t0(kt);
      const int dbase = 2 * o0 - w + tA, ms = kSL * kt, ub = o0 - w + tA;
#pragma unroll
      for (int k = 0; k < TB; ++k) {
        const int e = 64 * k + lane;
        const int dd = e / kSL, ss = e % kSL;
        const int d = dbase + dd, m = ms + ss;
        const int o = (e < TE && d >= 0 && d < D && m < NS) ? (d * NS + m) * es : kOob;
#pragma unroll
        for (int q = 0; q < NPL; ++q) v[q][k] = bpl[q].template ld<T>(o, 0);
      }
#pragma unroll
      for (int k = 0; k < YB; ++k) {
        const int e = 64 * k + lane;
        const int rr = e / kBfChunk, kk = e - rr * kBfChunk;
        const int u = ub + rr;
        const int o = (e < YE && u >= 0 && u < n_oth && kk < fc) ? (u * F + f0 + kk) * es : kOob;
        vy[k] = bo.template ld<T>(o, 0);
      }
#pragma unroll
      for (int k = 0; k < HB; ++k) {
        const int u = ub + 64 * k + lane;
        vh[k] = bv.template ld<T>(u >= 0 && u < n_oth ? u * es : kOob, 0);
      }
    };
    fetch(tile_kt(0));
    for (int i = 0; i < KT; ++i) {
      const int kt = tile_kt(i), tA = tile_t0(kt), ms = kSL * kt;
      __syncthreads();
#pragma unroll
      for (int k = 0; k < TB; ++k) {
        const int e = 64 * k + lane;
        if (e < TE) {
          const int dd = e / kSL, ss = e % kSL;
#pragma unroll
          for (int q = 0; q < NPL; ++q) tile[q][dd * kBgTS + ss] = v[q][k];
        }
      }
#pragma unroll
      for (int k = 0; k < YB; ++k) {
        const int e = 64 * k + lane;
        const int rr = e / kBfChunk, kk = e - rr * kBfChunk;
        if (e < YE) yt[rr * YP + kk] = vy[k];
      }
#pragma unroll
      for (int k = 0; k < HB; ++k) {
        const int rr = 64 * k + lane;
        // a row off the grid loaded 0, whose half variance is 0
        if (rr < kBgTR) hvt[rr] = bf_hvar(a, vh[k]);
      }
      __syncthreads();
      if (i + 1 < KT) fetch(tile_kt(i + 1));
      const int t0 = tA > 0 ? tA : 0;
      const int t1 = tA + kBgT < 2 * w + 1 ? tA + kBgT : 2 * w + 1;
      for (int t = t0; t < t1; ++t) {
        const int u = own - w + t;   // the other index
        if (!lane_in || u < 0 || u >= n_oth) continue;
        const int m = rows ? (2 * w - t) >> 1 : t >> 1;
        const int e = (2 * lane + t - tA) * kBgTS + (m - ms);
        const int rr = lane + t - tA;
        const T c = tile[0][e], g = tile[1][e];
        const T var_raw = hv + hvt[rr];
        const T rv = rcp(fmax(var_raw, a.eps));
        const T dsq = c > (T)0 ? g * rv : (T)0;
        if (f0 == 0) {
          const T h = PEN ? tile[NPL - 1][e] : (T)0;
          dv += var_raw > a.eps ? (T)0.5 * fma(a.beta, h, -(g * c)) * rv : (T)0;
        }
        T yo[kBfChunk];
        bf_row<T, kBfChunk, true>(yt + rr * YP, kBfChunk, yo);
#pragma unroll
        for (int k = 0; k < kBfChunk; ++k) acc[k] = fma(dsq, xo[k] - yo[k], acc[k]);
      }
    }
    if (lane_in) {
      T* out = (rows ? a.dX + (size_t)b * N * F : a.dY + (size_t)b * M * F) + (size_t)own * F + f0;
#pragma unroll
      for (int k = 0; k < kBfChunk; ++k)
        if (k < fc) out[k] = (T)2 * acc[k];
    }
  }
  T* dvp = rows ? a.dVX : a.dVY;
  if (dvp && lane_in) {
    // the gradient of a standard deviation s is 2 s d/dv
    const T v = vown[own];
    dvp[(size_t)b * n_own + own] = a.sigma ? (T)2 * v * dv : dv;
  }
}

template <typename T>
BandFeat<T> bf_args(const UdtwArgs<T>& u, const T* X, const T* Y, int F) {
  BandFeat<T> f = {};
  f.X = X;
  f.Y = Y;
  f.VX = u.VX;
  f.VY = u.VY;
  f.N = u.N;
  f.M = u.M;
  f.F = F;
  f.w = (int)u.band;
  const int S = band_slots(f.w);
  f.NS = (f.w + 1 + S - 1) / S * S;
  f.D = u.N + u.M - 1;
  f.hv1 = u.hv1;
  f.hv0 = u.hv0;
  f.eps = u.eps;
  f.beta = u.beta;
  f.beta_ln2 = u.beta_ln2;
  f.sigma = u.sigma;
  return f;
}

template <typename T>
void bf_build(const BandFeat<T>& f, bool pen, int B, hipStream_t s) {
  // rows as 16-byte loads: F a multiple of 16 bytes and 16-byte aligned bases
  const bool v16 = (f.F * sizeof(T)) % 16 == 0 && ((uintptr_t)f.X & 15) == 0 &&
                   ((uintptr_t)f.Y & 15) == 0;
  const int fm = f.F <= 16 ? 16 : (f.F <= 32 ? 32 : (f.F <= 64 && sizeof(T) == 4 ? 64 : 0));
  {
    const int ngx = (f.NS + 63) / 64;
    const dim3 grid(xcd_grid(ngx * ((f.D + kBfDiags - 1) / kBfDiags), B));
#define TW_BFB(PEN_, FM_)                                                                        \
  do {                                                                                           \
    if (v16)                                                                                     \
      hipLaunchKernelGGL((band_feat_build<T, PEN_, FM_, true>), grid, dim3(64), 0, s, f, B, ngx); \
    else                                                                                         \
      hipLaunchKernelGGL((band_feat_build<T, PEN_, FM_, false>), grid, dim3(64), 0, s, f, B,      \
                         ngx);                                                                   \
  } while (0)
#define TW_BFB_FM(PEN_)                                                                         \
  do {                                                                                          \
    if (fm == 16)                                                                               \
      TW_BFB(PEN_, 16);                                                                         \
    else if (fm == 32)                                                                          \
      TW_BFB(PEN_, 32);                                                                         \
    else if constexpr (sizeof(T) == 4) {                                                        \
      if (fm == 64) TW_BFB(PEN_, 64);                                                           \
    }                                                                                           \
    if (fm == 0)                                                                                \
      hipLaunchKernelGGL((band_feat_build_any<T, PEN_>), grid, dim3(64), 0, s, f, B, ngx);      \
  } while (0)
    if (pen)
      TW_BFB_FM(true);
    else
      TW_BFB_FM(false);
#undef TW_BFB_FM
#undef TW_BFB
  }
}

}  // namespace

size_t band_feat_plane_elems(int N, int M, double band) {
  const int w = (int)band;
  const int S = band_slots(w);
  if (S == 0) return 0;
  return (size_t)(N + M - 1) * (size_t)((w + 1 + S - 1) / S * S);
}

bool band_feat_path(int N, int M, int F, double band) {
  if (F < 1 || !band_path(N, M, band)) return false;
  // a pair's feature rows are addressed with 32-bit byte offsets
  if ((long long)(N > M ? N : M) * F * 8 >= (1LL << 31)) return false;
  // the backward keeps three planes (C rebuilt when the forward's are not
  // given, dC, dQ) in the N M elements per pair of its workspace
  return 3 * band_feat_plane_elems(N, M, band) <= (size_t)N * M;
}

template <typename T>
int band_feat_fwd(const UdtwArgs<T>& u, const T* X, const T* Y, int F, int B, T* ws,
                  hipStream_t s, const char* what) {
  if (B == 0) return TW_OK;
  if (((uintptr_t)ws & 15) != 0)
    return fail(TW_EINVAL, "%s: the workspace must be 16-byte aligned", what);
  const bool pen = u.beta != (T)0;
  BandFeat<T> f = bf_args(u, X, Y, F);
  const size_t pl = (size_t)B * f.D * f.NS;
  f.Cb = ws;
  f.Qb = pen ? ws + pl : nullptr;
  bf_build<T>(f, pen, B, s);
  if (int e = check_launch(what)) return e;
  UdtwArgs<T> a = u;
  a.C = f.Cb;
  a.Q = f.Qb;
  return band_sweep<T>(false, a, B, s, what, true);
}

template <typename T>
int band_feat_bwd(const UdtwArgs<T>& u, const T* X, const T* Y, int F, int B, const T* ws_fwd,
                  T* ws, T* dX, T* dY, hipStream_t s, const char* what) {
  if (B == 0) return TW_OK;
  if (((uintptr_t)ws & 15) != 0)
    return fail(TW_EINVAL, "%s: the workspace must be 16-byte aligned", what);
  const bool pen = u.beta != (T)0;
  BandFeat<T> f = bf_args(u, X, Y, F);
  const size_t pl = (size_t)B * f.D * f.NS;
  // the cost plane: the forward's, or rebuilt at the workspace's start
  T* dst = ws;
  if (ws_fwd) {
    f.Cb = const_cast<T*>(ws_fwd);
  } else {
    f.Cb = ws;
    f.Qb = nullptr;
    bf_build<T>(f, false, B, s);
    if (int e = check_launch(what)) return e;
    dst = ws + pl;
  }
  f.dCb = dst;
  f.dQb = pen ? dst + pl : nullptr;
  UdtwArgs<T> a = u;
  a.dC = dst;
  a.dQ = pen ? dst + pl : nullptr;
  if (int e = band_sweep<T>(true, a, B, s, what, true)) return e;
  f.dX = dX;
  f.dY = dY;
  f.dVX = u.dVX;
  f.dVY = u.dVY;
  const int nrb = (f.N + 63) / 64, ncb = (f.M + 63) / 64;
  const dim3 grid(xcd_grid(nrb + ncb, B));
  if (pen)
    hipLaunchKernelGGL((band_feat_grad<T, true>), grid, dim3(64), 0, s, f, B, nrb, ncb);
  else
    hipLaunchKernelGGL((band_feat_grad<T, false>), grid, dim3(64), 0, s, f, B, nrb, ncb);
  return check_launch(what);
}

template int band_feat_fwd<float>(const UdtwArgs<float>&, const float*, const float*, int, int,
                                  float*, hipStream_t, const char*);
template int band_feat_fwd<double>(const UdtwArgs<double>&, const double*, const double*, int,
                                   int, double*, hipStream_t, const char*);
template int band_feat_bwd<float>(const UdtwArgs<float>&, const float*, const float*, int, int,
                                  const float*, float*, float*, float*, hipStream_t, const char*);
template int band_feat_bwd<double>(const UdtwArgs<double>&, const double*, const double*, int,
                                   int, const double*, double*, double*, double*, hipStream_t,
                                   const char*);

// ------------------------------------------------ cost path, band layout
//
// The cost path's forward reads C and Q at the band's cells of the [B, N, M]
// planes, one cache line per lane and slot at every step of its chain. When
// the caller's R buffer has room behind the band planes, a gather pass first
// copies the band's cells of C and Q into the band layout there (an LDS
// transpose of 32-row tiles, XCD-aware placement), and the sweep then reads
// them coalesced (as from features).

namespace {

constexpr int kGatherRows = 32;   // rows of the [N, M] planes per gather workgroup

// One workgroup per 32 rows of a pair: each plane's band segments of those
// rows (columns i - w .. i + w) are read row by row into LDS, contiguous in
// memory, and written out diagonal by diagonal, where the tile's cells of a
// diagonal are consecutive slots. Slots no row of the grid fills are left
// as they are: the sweep masks the cells off the grid.
template <typename T, bool PEN>
__global__ void __launch_bounds__(256) band_gather(const T* __restrict__ C,
                                                   const T* __restrict__ Q, T* Cb, T* Qb, int B,
                                                   int N, int M, int w, int NS, int D, int ntile) {
  extern __shared__ __align__(16) unsigned char gather_lds[];
  T* tile = reinterpret_cast<T*>(gather_lds);
  int b, tl;
  if (!xcd_place(ntile, B, b, tl)) return;
  const int i0 = tl * kGatherRows;
  const int RW = 2 * w + 1;   // row-local columns: c = j - (i - w)
  const int rows = N - i0 < kGatherRows ? N - i0 : kGatherRows;
  const size_t nm = (size_t)N * M;
  constexpr int NP = PEN ? 2 : 1;
  const T* src[2] = {C + b * nm, PEN ? Q + b * nm : nullptr};
  T* dst[2] = {Cb + (size_t)b * D * NS, PEN ? Qb + (size_t)b * D * NS : nullptr};
  // (a thread's column c of all 32 rows, of both planes, loaded before any is
  // stored, so the loads are in flight together; 8 diagonals x 32 rows per
  // pass of the threads on the way out)
  for (int c = threadIdx.x; c < RW; c += blockDim.x) {
    T v[NP][kGatherRows];
#pragma unroll
    for (int r = 0; r < kGatherRows; ++r) {
      const int i = i0 + r, j = i - w + c;
      const bool in = r < rows && j >= 0 && j < M;
#pragma unroll
      for (int q = 0; q < NP; ++q) v[q][r] = in ? src[q][(size_t)i * M + j] : (T)0;
    }
#pragma unroll
    for (int q = 0; q < NP; ++q)
#pragma unroll
      for (int r = 0; r < kGatherRows; ++r)
        if (r < rows) tile[(q * kGatherRows + r) * RW + c] = v[q][r];
  }
  __syncthreads();
  // diagonals 2 i0 - w .. 2 (i0 + rows - 1) + w, rows r of each
  const int dlo = 2 * i0 - w, nd = 2 * (rows - 1) + RW;
  const int r = threadIdx.x & (kGatherRows - 1);
  for (int dd = threadIdx.x / kGatherRows; dd < nd; dd += blockDim.x / kGatherRows) {
    const int d = dlo + dd, i = i0 + r, j = d - i;
    const int l = i - j + w;
    if (r >= rows || d < 0 || d >= D || j < 0 || j >= M || l < 0 || l > 2 * w) continue;
#pragma unroll
    for (int q = 0; q < NP; ++q)
      dst[q][(size_t)d * NS + (l >> 1)] = tile[(q * kGatherRows + r) * RW + (j - i + w)];
  }
}

}  // namespace

template <typename T>
int band_cost_fwd(const UdtwArgs<T>& u, int B, hipStream_t s, const char* what) {
  if (B == 0) return TW_OK;
  const int w = (int)u.band;
  const int S = band_slots(w);
  const int NS = (w + 1 + S - 1) / S * S, D = u.N + u.M - 1;
  const bool pen = u.Q != nullptr;
  // R's elements per pair hold the band planes (2 D NS of RT) first; the
  // gathered C, Q go behind all pairs' planes
  const size_t rs = u.rd ? 8 : sizeof(T);
  const size_t planes = (size_t)B * 2 * D * NS * rs;
  const size_t room = (size_t)B * u.N * u.M * rs;
  const size_t need = (size_t)B * D * NS * sizeof(T) * (pen ? 2 : 1);
  char* tail = reinterpret_cast<char*>(u.R) + planes;
  // the gather's tile: 32 rows of 2 w + 1 columns of each plane
  const size_t lds = (size_t)(pen ? 2 : 1) * kGatherRows * (2 * w + 1) * sizeof(T);
  if (planes + need > room || ((uintptr_t)tail & 15) != 0 || lds > (size_t)max_lds_bytes() ||
      (long long)u.N * u.M * (long long)rs >= (1LL << 31))
    return band_sweep<T>(false, u, B, s, what);   // (which also reports the size limit)
  T* Cb = reinterpret_cast<T*>(tail);
  T* Qb = pen ? Cb + (size_t)B * D * NS : nullptr;
  const int ntile = (u.N + kGatherRows - 1) / kGatherRows;
  const dim3 grid(xcd_grid(ntile, B));
  if (pen)
    hipLaunchKernelGGL((band_gather<T, true>), grid, dim3(256), lds, s, u.C, u.Q, Cb, Qb, B, u.N,
                       u.M, w, NS, D, ntile);
  else
    hipLaunchKernelGGL((band_gather<T, false>), grid, dim3(256), lds, s, u.C, u.Q, Cb, Qb, B,
                       u.N, u.M, w, NS, D, ntile);
  if (int e = check_launch(what)) return e;
  UdtwArgs<T> a = u;
  a.C = Cb;
  a.Q = Qb;
  return band_sweep<T>(false, a, B, s, what, true);
}

template int band_cost_fwd<float>(const UdtwArgs<float>&, int, hipStream_t, const char*);
template int band_cost_fwd<double>(const UdtwArgs<double>&, int, hipStream_t, const char*);

namespace {

// The reverse of band_gather: the band-layout dC (and dQ) of 32 rows read
// diagonal by diagonal into LDS (a diagonal's cells of the tile are
// consecutive slots; eight diagonals' loads of a lane in flight together),
// then written into the [N, M] planes row by row, each row's band segment
// contiguous. Cells outside the band are not written (zeroed elsewhere).
template <typename T, bool PEN>
__global__ void __launch_bounds__(256) band_scatter(const T* __restrict__ dCb,
                                                    const T* __restrict__ dQb, T* dC, T* dQ,
                                                    int B, int N, int M, int w, int NS, int D,
                                                    int ntile) {
  extern __shared__ __align__(16) unsigned char scatter_lds[];
  T* tile = reinterpret_cast<T*>(scatter_lds);
  int b, tl;
  if (!xcd_place(ntile, B, b, tl)) return;
  const int i0 = tl * kGatherRows;
  const int RW = 2 * w + 1;
  const int rows = N - i0 < kGatherRows ? N - i0 : kGatherRows;
  const size_t nm = (size_t)N * M;
  const int dlo = 2 * i0 - w, nd = 2 * (rows - 1) + RW;
  const int r = threadIdx.x & (kGatherRows - 1);
  constexpr int DPASS = 256 / kGatherRows, UN = 8;
  constexpr int NP = PEN ? 2 : 1;
  const T* src[2] = {dCb + (size_t)b * D * NS, PEN ? dQb + (size_t)b * D * NS : nullptr};
  T* dst[2] = {dC + b * nm, PEN ? dQ + b * nm : nullptr};
  // both planes' diagonal runs in flight together (UN per plane and lane)
  for (int dd0 = threadIdx.x / kGatherRows; dd0 < nd; dd0 += DPASS * UN) {
    T v[NP][UN];
    int e[UN];
#pragma unroll
    for (int k = 0; k < UN; ++k) {
      const int dd = dd0 + DPASS * k;
      const int d = dlo + dd, i = i0 + r, j = d - i;
      const int l = i - j + w;
      const bool in = dd < nd && r < rows && d >= 0 && d < D && j >= 0 && j < M && l >= 0 &&
                      l <= 2 * w;
#pragma unroll
      for (int q = 0; q < NP; ++q) v[q][k] = in ? src[q][(size_t)d * NS + (l >> 1)] : (T)0;
      e[k] = in ? r * RW + (j - i + w) : -1;
    }
#pragma unroll
    for (int k = 0; k < UN; ++k)
      if (e[k] >= 0) {
#pragma unroll
        for (int q = 0; q < NP; ++q) tile[q * kGatherRows * RW + e[k]] = v[q][k];
      }
  }
  __syncthreads();
  for (int rr = 0; rr < rows; ++rr) {
    const int i = i0 + rr;
    for (int c = threadIdx.x; c < RW; c += blockDim.x) {
      const int j = i - w + c;
      if (j >= 0 && j < M) {
#pragma unroll
        for (int q = 0; q < NP; ++q)
          dst[q][(size_t)i * M + j] = tile[(q * kGatherRows + rr) * RW + c];
      }
    }
  }
}

}  // namespace

size_t band_cost_workspace_elems(int B, int N, int M, double band) {
  if (B <= 0 || N <= 0 || M <= 0 || N > M || !band_path(N, M, band)) return 0;
  // dC and dQ in the band layout, and 16 bytes of slack for the alignment
  return (size_t)2 * B * band_feat_plane_elems(N, M, band) + 2;
}

template <typename T>
int band_cost_bwd(const UdtwArgs<T>& u, int B, hipStream_t s, const char* what, T* ws,
                  size_t ws_bytes) {
  if (B == 0) return TW_OK;
  const size_t pl = (size_t)B * band_feat_plane_elems(u.N, u.M, u.band);
  const bool pen = u.Q != nullptr;
  // the band layout's planes, 16-byte aligned within the workspace
  T* base = ws ? reinterpret_cast<T*>(((uintptr_t)ws + 15) & ~(uintptr_t)15) : nullptr;
  const size_t skip = ws ? (size_t)(reinterpret_cast<char*>(base) - reinterpret_cast<char*>(ws)) : 0;
  const int w = (int)u.band;
  // the scatter's tile: 32 rows of 2 w + 1 columns of each plane
  const size_t lds = (size_t)(pen ? 2 : 1) * kGatherRows * (2 * w + 1) * sizeof(T);
  if (!ws || ws_bytes < skip + (pen ? 2 : 1) * pl * sizeof(T) || lds > (size_t)max_lds_bytes())
    return band_sweep<T>(true, u, B, s, what);   // gradients straight into [B, N, M]
  UdtwArgs<T> a = u;
  a.dC = base;
  a.dQ = pen ? base + pl : nullptr;
  if (int e = band_sweep<T>(true, a, B, s, what, true, u.dC, pen ? u.dQ : nullptr)) return e;
  const int S = band_slots(w);
  const int NS = (w + 1 + S - 1) / S * S, D = u.N + u.M - 1;
  const int ntile = (u.N + kGatherRows - 1) / kGatherRows;
  const dim3 grid(xcd_grid(ntile, B));
  if (pen)
    hipLaunchKernelGGL((band_scatter<T, true>), grid, dim3(256), lds, s, a.dC, a.dQ, u.dC, u.dQ,
                       B, u.N, u.M, w, NS, D, ntile);
  else
    hipLaunchKernelGGL((band_scatter<T, false>), grid, dim3(256), lds, s, a.dC, a.dQ, u.dC,
                       u.dQ, B, u.N, u.M, w, NS, D, ntile);
  return check_launch(what);
}

template int band_cost_bwd<float>(const UdtwArgs<float>&, int, hipStream_t, const char*, float*,
                                  size_t);
template int band_cost_bwd<double>(const UdtwArgs<double>&, int, hipStream_t, const char*,
                                   double*, size_t);

}  // namespace tw
