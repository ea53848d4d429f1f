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
  T *dC, *dQ;          // backward [B,N,M] (inside the band)
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

template <typename T, typename RT, int S, bool PEN, int WP>
__global__ void __launch_bounds__(64) udtw_band_fwd(BandArgs<T, RT> a) {
  constexpr int PD = 8;   // prefetch distance (steps) = unroll of the step loop
  const int b = blockIdx.x, lane = threadIdx.x;
  const int N = a.N, M = a.M, w = a.w, NS = a.NS, D = a.D;
  const RT BIG = band_big<RT>();
  const size_t nm = (size_t)N * M, bsz = (size_t)2 * D * NS;
  Buf bc, bq, br, bp;
  bc.init(a.C + b * nm, (long long)nm);
  if (PEN) bq.init(a.Q + b * nm, (long long)nm);
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
    const int p = (u & 1) ^ WP;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int o = sc[p][s].off(d, M, es);
      cr[u][s] = bc.ld<T>(o, 0);
      if (PEN) qr[u][s] = bq.ld<T>(o, 0);
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

template <typename T, typename RT, int S, bool PEN, int WP>
__global__ void __launch_bounds__(64) udtw_band_bwd(BandArgs<T, RT> a) {
  if ((int)blockIdx.x >= a.B) {
    band_zero_rows<T>(a.dC, a.dQ, a.B, a.N, a.M, a.w, (int)blockIdx.x - a.B, a.nzero);
    return;
  }
  // prefetch distance (steps, even): as deep as the memory counter (63
  // outstanding accesses) allows for this step's loads and stores
  constexpr int PD = band_bwd_depth<T, RT, S, PEN>();
  const int b = blockIdx.x, lane = threadIdx.x;
  const int N = a.N, M = a.M, w = a.w, NS = a.NS, D = a.D;
  const RT NEG = -band_big<RT>();
  const size_t nm = (size_t)N * M, bsz = (size_t)2 * D * NS;
  Buf br, bp, bdc, bdq;
  br.init(a.R + b * bsz, (long long)bsz);
  if (PEN) bp.init(a.P + b * bsz, (long long)bsz);
  bdc.init(a.dC + b * nm, (long long)nm);
  // without dQ, an empty range: its stores are dropped
  const bool has_dq = PEN && a.dQ != nullptr;
  if (PEN) bdq.init(has_dq ? a.dQ + b * nm : a.dC, has_dq ? (long long)nm : 0LL);
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
        ne[s] = bsel(rbr[u][s], NEG, keep);
        ng[s] = G;
        na[s] = A;
        nb[s] = PEN ? pbr[u][s] : (T)0;
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

template <typename T, typename RT, int S, bool PEN>
int band_launch(bool bwd, const BandArgs<T, RT>& a, int B, hipStream_t s) {
  // parity of step 0 (forward) / of step D - 1 (backward)
  const int wp = bwd ? ((a.D - 1 + a.w) & 1) : (a.w & 1);
  if (bwd) {
    // The sweep's waves issue one dependent step after another: a wave of
    // the zeroing role beside one on its SIMD would take issue cycles from
    // it. An LDS reservation (unused) of over half a CU's LDS keeps every
    // workgroup on a CU of its own.
    const dim3 grid((unsigned)(B + a.nzero));
    const size_t lds = (size_t)max_lds_bytes() / 2 + 256;
    if (wp)
      hipLaunchKernelGGL((udtw_band_bwd<T, RT, S, PEN, 1>), grid, dim3(64), lds, s, a);
    else
      hipLaunchKernelGGL((udtw_band_bwd<T, RT, S, PEN, 0>), grid, dim3(64), lds, s, a);
  } else {
    if (wp)
      hipLaunchKernelGGL((udtw_band_fwd<T, RT, S, PEN, 1>), dim3(B), dim3(64), 0, s, a);
    else
      hipLaunchKernelGGL((udtw_band_fwd<T, RT, S, PEN, 0>), dim3(B), dim3(64), 0, s, a);
  }
  return TW_OK;
}

template <typename T, typename RT>
int band_run(bool bwd, const UdtwArgs<T>& u, int B, hipStream_t s, const char* what) {
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
  a.nzero = bwd ? (int)((rows + 3) / 4 < 1024 ? (rows + 3) / 4 : 1024) : 0;
  a.k = u.k;
  a.inv_k = u.inv_k;
  a.inv_gamma = u.inv_gamma;
  const bool pen = u.Q != nullptr;
#define TW_BAND(S_)                                                       \
  (pen ? band_launch<T, RT, S_, true>(bwd, a, B, s)                       \
       : band_launch<T, RT, S_, false>(bwd, a, B, s))
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
int band_sweep(bool bwd, const UdtwArgs<T>& a, int B, hipStream_t s, const char* what) {
  if (B == 0) return TW_OK;
  // planes are addressed with 32-bit byte offsets within a pair
  const long long rbytes = a.rd ? 8 : (long long)sizeof(T);
  if ((long long)a.N * a.M * rbytes >= (1LL << 31)) {
    return fail(TW_ESIZE, "%s: one pair's N*M matrix (%d x %d) must stay below 2 GiB", what,
                a.N, a.M);
  }
  if (sizeof(T) == 4 && a.rd) return band_run<T, double>(bwd, a, B, s, what);
  return band_run<T, T>(bwd, a, B, s, what);
}

template int band_sweep<float>(bool, const UdtwArgs<float>&, int, hipStream_t, const char*);
template int band_sweep<double>(bool, const UdtwArgs<double>&, int, hipStream_t, const char*);

}  // namespace tw
