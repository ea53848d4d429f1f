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
// Forward: on the matrix cores in both precisions (v_mfma_f32_16x16x4f32,
// v_mfma_f64_16x16x4f64; a 16 x 16*TN output strip per wavefront), with
// 4-element chunk loads when D % 4 == 0 and element loads otherwise; a plain
// FMA kernel only for blocks whose byte offsets pass 31 bits. Backward: when a
// pair's dS fits in LDS and C <= 64, one fused kernel per pair streams A and B
// once (threads along D, dB partial sums in registers); otherwise two tiled
// passes that each read dS once (dA by row blocks, dB by column blocks), on
// the matrix cores in both precisions (D > 64 in 64-feature slices in fp32,
// D > 32 in 32-feature slices in fp64); FMA kernels only past 31-bit
// offsets.
//
// The uDTW feature path (sqdist_raw / sqdist_raw_bwd) keeps S and dS by
// anti-diagonals (plane_index), the layout in which the sweeps' per-diagonal
// accesses are coalesced; the tiled backward then reads each 64 x 64 tile
// along its anti-diagonals, whose cells are contiguous.

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

// Element (r, c) of a pair's R x C plane (R <= C): row-major, or with DG by
// anti-diagonals (the cells of diagonal r + c contiguous, by row), the layout
// the uDTW sweeps read and write coalesced.
template <bool DG>
__device__ __forceinline__ long long plane_index(int r, int c, int R, int C) {
  if (!DG) return (long long)r * C + c;
  const int d = r + c, lo = d - C + 1 > 0 ? d - C + 1 : 0;
  return diag_offset(d, R, C) + (r - lo);
}

// ------------------------------------------------------------ FMA kernels

template <typename T, int MET, bool DG>
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
  out[(size_t)p * R * C + plane_index<DG>(r, c, R, C)] = finish_cost<T, MET>(aa + bq - (T)2 * ab);
}

// dA[r, d] = 2 (sum_c dS[r,c] a[r,d] - sum_c dS[r,c] b[c,d])
template <typename T, int MET, bool DG>
__global__ void __launch_bounds__(256) pair_bwd_a_fma(const T* __restrict__ A,
                                                      const T* __restrict__ Bm,
                                                      const T* __restrict__ cost,
                                                      const T* __restrict__ dcost,
                                                      T* __restrict__ dA, int R, int C, int D) {
  const int p = blockIdx.y;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long long)R * D) return;
  const int r = (int)(idx / D), d = (int)(idx % D);
  const size_t pp = (size_t)p * R * C;
  T rs = 0, acc = 0;
  for (int c = 0; c < C; ++c) {
    const size_t o = pp + plane_index<DG>(r, c, R, C);
    const T ds = cost_adjoint<T, MET>(dcost[o], MET == MET_RAW ? (T)0 : cost[o]);
    rs += ds;
    acc += ds * Bm[((size_t)p * C + c) * D + d];
  }
  dA[((size_t)p * R + r) * D + d] = (T)2 * (rs * A[((size_t)p * R + r) * D + d] - acc);
}

// dB[c, d] = 2 (sum_r dS[r,c] b[c,d] - sum_r dS[r,c] a[r,d])
template <typename T, int MET, bool DG>
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
    const size_t o = (size_t)p * R * C + plane_index<DG>(r, c, R, C);
    const T ds = cost_adjoint<T, MET>(dcost[o], MET == MET_RAW ? (T)0 : cost[o]);
    cs += ds;
    acc += ds * A[((size_t)p * R + r) * D + d];
  }
  dB[((size_t)p * C + c) * D + d] = (T)2 * (cs * Bm[((size_t)p * C + c) * D + d] - acc);
}


// Tiled fp64 backward, one pass over dS per output: a workgroup owns
// 64 rows (dA, COLS false) or 64 columns (dB, COLS true) of a pair and
// streams the other axis in 64-wide tiles. Each dS tile is read with
// coalesced 256-byte rows and staged in LDS as [owned][streamed] next to the
// matching 64 x D block of the other operand; four threads share an owned
// index and each accumulates DPT of its outputs, summing in a fixed order. A
// launch covers the features k0 .. k0 + 4 DPT - 1 (DPT <= 8); larger D takes
// one launch pair per 32-feature slice.
template <typename T, int MET, bool COLS, int DPT, bool DG>
__global__ void __launch_bounds__(256) pair_bwd_tiled(const T* __restrict__ A,
                                                      const T* __restrict__ Bm,
                                                      const T* __restrict__ cost,
                                                      const T* __restrict__ dcost,
                                                      T* __restrict__ dOut, int R, int C, int D,
                                                      int k0) {
  constexpr int TL = 64;
  // row pitch: TL + 1 keeps row-wise and column-wise accesses conflict-free;
  // the diagonal loads (DG) need TL + 2 (a diagonal's cells then fall in
  // distinct banks)
  __shared__ T ds[TL][TL + (DG ? 2 : 1)];
  __shared__ T op[TL][4 * DPT + 1];
  const int p = blockIdx.y, tid = threadIdx.x;
  const int own0 = blockIdx.x * TL;
  const int nown = COLS ? C : R, nstr = COLS ? R : C;
  const size_t prc = (size_t)p * R * C;
  const T* other = COLS ? A + (size_t)p * R * D : Bm + (size_t)p * C * D;
  const T* self = COLS ? Bm + (size_t)p * C * D : A + (size_t)p * R * D;
  const int oi = tid >> 2, dg = tid & 3;
  T acc[DPT];
#pragma unroll
  for (int k = 0; k < DPT; ++k) acc[k] = 0;
  T sum = 0;
  for (int s0 = 0; s0 < nstr; s0 += TL) {
    __syncthreads();
    const int r0 = COLS ? s0 : own0, c0 = COLS ? own0 : s0;
    if (DG) {
      // by the tile's 127 anti-diagonals, four per pass (one per wavefront):
      // the cells of one are contiguous in the diagonal-major plane, so the
      // wavefront-uniform start of its run is computed once; all 32 loads
      // are issued before the LDS stores
      const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), ln = tid & 63;
      T v[(2 * TL) / 4];
#pragma unroll
      for (int it = 0; it < (2 * TL) / 4; ++it) {
        const int dd = 4 * it + wv;
        const int rr = (dd < TL ? 0 : dd - TL + 1) + ln, cc = dd - rr;
        const int r = r0 + rr, c = c0 + cc, d = r0 + c0 + dd;
        const long long run = diag_offset(d, R, C) - (d - C + 1 > 0 ? d - C + 1 : 0);
        v[it] = 0;
        if (dd < 2 * TL - 1 && rr < TL && cc >= 0 && r < R && c < C) {
          const size_t o = prc + (size_t)(run + r);
          v[it] = cost_adjoint<T, MET>(dcost[o], MET == MET_RAW ? (T)0 : cost[o]);
        }
      }
#pragma unroll
      for (int it = 0; it < (2 * TL) / 4; ++it) {
        const int dd = 4 * it + wv;
        const int rr = (dd < TL ? 0 : dd - TL + 1) + ln, cc = dd - rr;
        if (dd < 2 * TL - 1 && rr < TL && cc >= 0) {
          if (COLS)
            ds[cc][rr] = v[it];
          else
            ds[rr][cc] = v[it];
        }
      }
    } else {
#pragma unroll 4
      for (int e = tid; e < TL * TL; e += 256) {
        const int rr = e >> 6, cc = e & 63;
        const int r = r0 + rr, c = c0 + cc;
        T v = 0;
        if (r < R && c < C) {
          const size_t o = prc + (size_t)r * C + c;
          v = cost_adjoint<T, MET>(dcost[o], MET == MET_RAW ? (T)0 : cost[o]);
        }
        if (COLS)
          ds[cc][rr] = v;
        else
          ds[rr][cc] = v;
      }
    }
    for (int e = tid; e < TL * 4 * DPT; e += 256) {
      const int si = e / (4 * DPT), d = e - si * (4 * DPT);
      op[si][d] = (s0 + si < nstr && k0 + d < D) ? other[(size_t)(s0 + si) * D + k0 + d] : (T)0;
    }
    __syncthreads();
#pragma unroll 8
    for (int si = 0; si < TL; ++si) {
      const T v = ds[oi][si];
      sum += v;
#pragma unroll
      for (int k = 0; k < DPT; ++k) acc[k] += v * op[si][dg * DPT + k];
    }
  }
  const int o = own0 + oi;
  if (o < nown) {
#pragma unroll
    for (int k = 0; k < DPT; ++k) {
      const int d = k0 + dg * DPT + k;
      if (d < D) dOut[((size_t)p * nown + o) * D + d] = (T)2 * (sum * self[(size_t)o * D + d] - acc[k]);
    }
  }
}

// ----------------------------------------------------------- MFMA forward
//
// v_mfma_f32_16x16x4f32 operand layout (wave64): A (16x4) lane l holds
// A[l % 16][l / 16]; B (4x16) lane l holds B[l / 16][l % 16]; the 16x16
// result gives lane l, register i the element (4 (l / 16) + i, l % 16).
// v_mfma_f64_16x16x4f64 takes its operands the same way and gives lane l,
// register i the element (l / 16 + 4 i, l % 16).
// The reduction index may be permuted consistently in both operands: lane l
// loads the float4 A[row][k0 + 4 g .. +3] (g = l / 16) and its B row
// likewise, and MFMA j of a 16-wide k block consumes component j, i.e.
// k = k0 + 4 g + j. Each row then contributes one contiguous 64-byte segment
// per k block.

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));

// The four consecutive elements a lane contributes per k block, and the
// accumulator of one 16 x 16 MFMA tile (four elements per lane), per type.
template <typename T> struct Mfma;
template <> struct Mfma<float> {
  typedef f32x4 V;
  // v_mfma_f32_16x16x4f32
  static __device__ __forceinline__ V op(float a, float b, V c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  // row of result register i in lane group g (the column is lane % 16)
  static __device__ __forceinline__ int row(int g, int i) { return 4 * g + i; }
};
template <> struct Mfma<double> {
  typedef f64x4 V;
  // v_mfma_f64_16x16x4f64: the same operand layout, one double per lane for
  // A and B; the four result registers of lane group g hold rows g, g + 4,
  // g + 8, g + 12 (measured on gfx950)
  static __device__ __forceinline__ V op(double a, double b, V c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int row(int g, int i) { return g + 4 * i; }
};

__device__ __forceinline__ f32x4 ld4(const Buf& b, int v, int s) {
  const unsigned int __attribute__((ext_vector_type(4))) w =
      __builtin_amdgcn_raw_buffer_load_b128(b.r, v, s, 0);
  return f32x4{__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z),
               __uint_as_float(w.w)};
}
// Four doubles (32 bytes) as two 16-byte loads.
__device__ __forceinline__ f64x4 ld4d(const Buf& b, int v, int s) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(b.r, v, s, 0);
  const u32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(b.r, v == kOob ? kOob : v + 16, s, 0);
  auto dbl = [](unsigned int x, unsigned int y) {
    return __longlong_as_double((long long)(((unsigned long long)y << 32) | x));
  };
  return f64x4{dbl(lo.x, lo.y), dbl(lo.z, lo.w), dbl(hi.x, hi.y), dbl(hi.z, hi.w)};
}

// Elements k..k+3 of the row at byte offset v as four single loads (rows of
// any D are only element-aligned); elements at or past D, and every element
// of a row at kOob, read 0.
__device__ __forceinline__ f32x4 ld4_elems(const Buf& b, int v, int k, int D, float) {
  f32x4 x;
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = b.ldf(v == kOob || k + j >= D ? kOob : v + (k + j) * 4, 0);
  return x;
}
__device__ __forceinline__ f64x4 ld4_elems(const Buf& b, int v, int k, int D, double) {
  f64x4 x;
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = b.ldd(v == kOob || k + j >= D ? kOob : v + (k + j) * 8, 0);
  return x;
}
__device__ __forceinline__ f32x4 ld4_chunk(const Buf& b, int v, int s, float) { return ld4(b, v, s); }
__device__ __forceinline__ f64x4 ld4_chunk(const Buf& b, int v, int s, double) {
  return ld4d(b, v, s);
}

// D4: D % 4 == 0, each row's chunk is one aligned 4-element load; otherwise
// four single-element loads with the tail masked. Byte offsets within a
// pair's blocks fit 31 bits (the launcher checks).
template <typename T, int MET, int TN, bool DG, bool D4>
__global__ void __launch_bounds__(256) pair_fwd_mfma(const T* __restrict__ A,
                                                     const T* __restrict__ Bm,
                                                     T* __restrict__ out, int R, int C,
                                                     int D) {
  typedef typename Mfma<T>::V V;
  constexpr int ES = (int)sizeof(T);
  const int p = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int strip = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int RT = (R + 15) >> 4, CT = (C + 16 * TN - 1) / (16 * TN);
  if (strip >= RT * CT) return;   // no barrier below: a finished wave may leave
  const int r0 = (strip % RT) * 16, c0 = (strip / RT) * 16 * TN;
  const int g = lane >> 4, li = lane & 15;

  Buf ba, bb;
  ba.init(A + (size_t)p * R * D, (long long)R * D);
  bb.init(Bm + (size_t)p * C * D, (long long)C * D);
  const int ra = r0 + li;
  // D4: offset of the lane's chunk; else of its row
  const int va = ra < R ? (ra * D + (D4 ? 4 * g : 0)) * ES : kOob;
  int vb[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int cb = c0 + 16 * t + li;
    vb[t] = cb < C ? (cb * D + (D4 ? 4 * g : 0)) * ES : kOob;
  }
  V acc[TN];
  T na = 0, nb[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    acc[t] = V{0, 0, 0, 0};
    nb[t] = 0;
  }
  for (int k0 = 0; k0 < D; k0 += 16) {
    const bool kin = k0 + 4 * g < D;   // D % 4 == 0: a chunk is all in or all out
    const V a4 = D4 ? ld4_chunk(ba, kin ? va : kOob, k0 * ES, T(0))
                    : ld4_elems(ba, va, k0 + 4 * g, D, T(0));
    na += a4.x * a4.x + a4.y * a4.y + a4.z * a4.z + a4.w * a4.w;
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const V b4 = D4 ? ld4_chunk(bb, kin ? vb[t] : kOob, k0 * ES, T(0))
                      : ld4_elems(bb, vb[t], k0 + 4 * g, D, T(0));
      nb[t] += b4.x * b4.x + b4.y * b4.y + b4.z * b4.z + b4.w * b4.w;
      acc[t] = Mfma<T>::op(a4.x, b4.x, acc[t]);
      acc[t] = Mfma<T>::op(a4.y, b4.y, acc[t]);
      acc[t] = Mfma<T>::op(a4.z, b4.z, acc[t]);
      acc[t] = Mfma<T>::op(a4.w, b4.w, acc[t]);
    }
  }
  // squared norms: sum the four k groups of each row (lanes li, li+16, li+32, li+48)
  na += __shfl_xor(na, 16);
  na += __shfl_xor(na, 32);
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    nb[t] += __shfl_xor(nb[t], 16);
    nb[t] += __shfl_xor(nb[t], 32);
  }
  T* o = out + (size_t)p * R * C;
  if (!DG) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rt = Mfma<T>::row(g, i), r = r0 + rt;
      const T nr = __shfl(na, rt);   // lane rt holds row rt's norm
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const int c = c0 + 16 * t + li;
        if (r < R && c < C) o[(size_t)r * C + c] = finish_cost<T, MET>(nr + nb[t] - T(2) * acc[t][i]);
      }
    }
    return;
  }
  // Diagonal-major plane: the wavefront's 16 x 16 TN strip goes through LDS
  // and leaves by anti-diagonals, four per store (one per 16 lanes), each a
  // contiguous run of up to 16 cells. Only this wavefront touches its tile,
  // and its LDS operations complete in order.
  constexpr int W = 16 * TN, PITCH = W + 2;   // pitch W + 2: a diagonal's cells in distinct banks
  __shared__ T tile[4][16][PITCH];
  T(*tl)[PITCH] = tile[threadIdx.x >> 6];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rt = Mfma<T>::row(g, i);
    const T nr = __shfl(na, rt);
#pragma unroll
    for (int t = 0; t < TN; ++t)
      tl[rt][16 * t + li] = finish_cost<T, MET>(nr + nb[t] - T(2) * acc[t][i]);
  }
  if ((long long)R * C < (1LL << 31)) {
    // Lane l holds the run starts (plane_index minus the row) of tile
    // diagonals l and l + 64, below 2^31 by the plane size; each store picks
    // its group's start from four v_readlane results instead of evaluating
    // diag_offset per cell.
    int run0 = 0, run1 = 0;
    {
      const int d0 = r0 + c0 + lane, d1 = d0 + 64;
      if (d0 <= R + C - 2) run0 = (int)(diag_offset(d0, R, C) - (d0 - C + 1 > 0 ? d0 - C + 1 : 0));
      if (d1 <= R + C - 2) run1 = (int)(diag_offset(d1, R, C) - (d1 - C + 1 > 0 ? d1 - C + 1 : 0));
    }
#pragma unroll
    for (int dd0 = 0; dd0 < 16 + W - 1; dd0 += 4) {
      const int dd = dd0 + g, rr = li, cc = dd - rr;
      const int r = r0 + rr, c = c0 + cc;
      int sk[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        sk[k] = dd0 + k < 64 ? __builtin_amdgcn_readlane(run0, (dd0 + k) & 63)
                             : __builtin_amdgcn_readlane(run1, (dd0 + k) & 63);
      const int st = g == 0 ? sk[0] : (g == 1 ? sk[1] : (g == 2 ? sk[2] : sk[3]));
      if (dd < 16 + W - 1 && cc >= 0 && cc < W && r < R && c < C) o[(size_t)st + r] = tl[rr][cc];
    }
    return;
  }
  for (int dd0 = 0; dd0 < 16 + W - 1; dd0 += 4) {
    const int dd = dd0 + g, rr = li, cc = dd - rr;
    const int r = r0 + rr, c = c0 + cc;
    if (dd < 16 + W - 1 && cc >= 0 && cc < W && r < R && c < C)
      o[plane_index<true>(r, c, R, C)] = tl[rr][cc];
  }
}

// ---------------------------------------------------------- MFMA backward
//
// The tiled backward's two passes (dA by 64-row blocks, dB by 64-column
// blocks, each reading dS once) with the contraction on the matrix cores
// (v_mfma_f32_16x16x4f32 / v_mfma_f64_16x16x4f64). A launch covers the
// features k0 .. k0 + 16NB - 1 (NB <= 4 in fp32, 2 in fp64, which keeps the
// static LDS below 64 KB); larger D takes one launch pair per 64- (32-)
// feature slice. A workgroup owns 64 indices of one side; per 64-wide tile of
// the streamed side it stages dS as ds[owned][streamed] and the other operand
// transposed, opT[d][streamed], both with rows of 68 elements (aligned for
// the 4-element reads; the diagonal stores of the DG loader step 67 elements
// per lane, so they do not conflict). Wavefront w owns rows 16w..16w+15 and
// accumulates its 16 x 16NB block of dS . other, lane l reading the
// 4-element vectors ds[16w + l % 16][kb + 4 (l / 16)] and
// opT[16n + l % 16][kb + 4 (l / 16)] (the k-permuted operand layout of the
// forward). The row sums of dS come from the same vectors. The next tile's
// dS is loaded into registers before the MFMAs of this one. Workgroups are
// numbered so that the tiles of one pair run on one XCD (the hardware
// assigns workgroup i to XCD i % 8): the runs of a diagonal-major tile share
// their end cache lines with the neighbouring tiles.
template <typename T, int MET, bool COLS, int NB, bool DG>
__global__ void __launch_bounds__(256) pair_bwd_mfma(const T* __restrict__ A,
                                                     const T* __restrict__ Bm,
                                                     const T* __restrict__ cost,
                                                     const T* __restrict__ dcost,
                                                     T* __restrict__ dOut, int P, int R,
                                                     int C, int D, int k0) {
  typedef typename Mfma<T>::V V;
  constexpr int TL = 64, PT = TL + 4, ES = (int)sizeof(T);
  __shared__ __align__(32) T ds[TL][PT];
  __shared__ __align__(32) T opT[16 * NB][PT];
  const int nown = COLS ? C : R, nstr = COLS ? R : C;
  const int gx = (nown + TL - 1) / TL;
  const unsigned total = (unsigned)gx * P, L = blockIdx.x;
  const unsigned id = (total & 7) ? L : (L & 7) * (total >> 3) + (L >> 3);
  const int p = id / gx, own0 = (id % gx) * TL;
  const int tid = threadIdx.x, ln = tid & 63, lr = ln & 15, lg = ln >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const size_t prc = (size_t)p * R * C;
  const T* other = COLS ? A + (size_t)p * R * D : Bm + (size_t)p * C * D;
  const T* self = COLS ? Bm + (size_t)p * C * D : A + (size_t)p * R * D;

  // The next tile goes into registers while this one is contracted: dS (DG
  // by the tile's 127 anti-diagonals, four per pass, one per wavefront, each
  // a contiguous run; else by rows) and the other operand's 64 x 16NB block.
  // Lane l first computes the run starts of tile diagonals l and l + 64,
  // which each pass then takes with v_readlane. Loads are raw buffer loads;
  // lanes outside the plane pass kOob and read 0.
  constexpr int NV = DG ? (2 * TL) / 4 : TL * TL / 256, NW = 4 * NB;
  Buf bd, bo;
  bd.init(dcost + prc, (long long)R * C);
  bo.init(other, (long long)nstr * D);
  T v[NV], w[NW];
  auto load = [&](int s0) {
    const int r0 = COLS ? s0 : own0, c0 = COLS ? own0 : s0;
    int run[2] = {0, 0};
    if (DG) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int d = r0 + c0 + 64 * h + ln;
        if (d <= R + C - 2)
          run[h] = (int)(diag_offset(d, R, C) - (d - C + 1 > 0 ? d - C + 1 : 0));
      }
    }
#pragma unroll
    for (int it = 0; it < NV; ++it) {
      int r, c, so = 0;
      bool ok;
      if (DG) {
        const int dd = 4 * it + wv;   // it < 16: dd < 64
        const int rr = (dd < TL ? 0 : dd - TL + 1) + ln, cc = dd - rr;
        r = r0 + rr;
        c = c0 + cc;
        ok = dd < 2 * TL - 1 && rr < TL && cc >= 0;
        so = __builtin_amdgcn_readlane(run[it < 16 ? 0 : 1], dd & 63) * ES;
      } else {
        const int e = it * 256 + tid;
        r = r0 + (e >> 6);
        c = c0 + (e & 63);
        ok = true;
      }
      const int vo = !(ok && r < R && c < C) ? kOob : (DG ? r : r * C + c) * ES;
      if (MET == MET_RAW) {
        v[it] = bd.template ld<T>(vo, so);
      } else {
        const size_t oo = prc + (size_t)r * C + c;
        v[it] = vo == kOob ? T(0) : cost_adjoint<T, MET>(dcost[oo], cost[oo]);
      }
    }
#pragma unroll
    for (int it = 0; it < NW; ++it) {
      const int e = it * 256 + tid, si = e & 63, dcol = e >> 6;
      w[it] = bo.template ld<T>(
          s0 + si < nstr && k0 + dcol < D ? ((s0 + si) * D + k0 + dcol) * ES : kOob, 0);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int it = 0; it < NV; ++it) {
      int rr, cc;
      bool ok;
      if (DG) {
        const int dd = 4 * it + wv;
        rr = (dd < TL ? 0 : dd - TL + 1) + ln;
        cc = dd - rr;
        ok = dd < 2 * TL - 1 && rr < TL && cc >= 0;
      } else {
        const int e = it * 256 + tid;
        rr = e >> 6;
        cc = e & 63;
        ok = true;
      }
      if (ok) {
        if (COLS)
          ds[cc][rr] = v[it];
        else
          ds[rr][cc] = v[it];
      }
    }
#pragma unroll
    for (int it = 0; it < NW; ++it) {
      const int e = it * 256 + tid;
      opT[e >> 6][e & 63] = w[it];
    }
  };

  V acc[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) acc[n] = V{0, 0, 0, 0};
  T rs = 0;
  load(0);
  for (int s0 = 0; s0 < nstr; s0 += TL) {
    __syncthreads();   // the previous tile's LDS reads are done
    stash();
    __syncthreads();
    if (s0 + TL < nstr) load(s0 + TL);
#pragma unroll
    for (int kb = 0; kb < TL; kb += 16) {
      const V a4 = *reinterpret_cast<const V*>(&ds[16 * wv + lr][kb + 4 * lg]);
      rs += (a4.x + a4.y) + (a4.z + a4.w);
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const V b4 = *reinterpret_cast<const V*>(&opT[16 * n + lr][kb + 4 * lg]);
        acc[n] = Mfma<T>::op(a4.x, b4.x, acc[n]);
        acc[n] = Mfma<T>::op(a4.y, b4.y, acc[n]);
        acc[n] = Mfma<T>::op(a4.z, b4.z, acc[n]);
        acc[n] = Mfma<T>::op(a4.w, b4.w, acc[n]);
      }
    }
  }
  // row sums: the four k groups of row l % 16 sit in lanes l % 16 + 16 g
  rs += __shfl_xor(rs, 16);
  rs += __shfl_xor(rs, 32);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rt = Mfma<T>::row(lg, i), o = own0 + 16 * wv + rt;   // result row of register i
    const T so = __shfl(rs, rt);
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const int d = k0 + 16 * n + lr;
      if (o < nown && d < D)
        dOut[((size_t)p * nown + o) * D + d] = T(2) * (so * self[(size_t)o * D + d] - acc[n][i]);
    }
  }
}

// ------------------------------------------------ fused per-pair backward
//
// One workgroup per pair with dS = adjoint(dcost) [R, C] in LDS together
// with its row and column sums. Threads run along D; each keeps the C values
// B[:, d] and the C partial sums of dB[:, d] in registers and walks the rows
// once: dA[r, d] = 2 (rs[r] a - sum_c dS[r,c] B[c,d]), dB partial
// += dS[r, c] a, a = A[r, d]. A and B are read once and dA, dB written once.

template <typename T, int MET, int CMAX, bool DG>
__global__ void __launch_bounds__(256) pair_bwd_small(const T* __restrict__ A,
                                                      const T* __restrict__ Bm,
                                                      const T* __restrict__ cost,
                                                      const T* __restrict__ dcost,
                                                      T* __restrict__ dA, T* __restrict__ dB,
                                                      int R, int C, int D) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* dS = reinterpret_cast<T*>(smem_raw);   // [R][CMAX], zero-padded
  T* rs = dS + (size_t)R * CMAX;            // [R]
  T* cs = rs + R;                           // [CMAX]
  const int p = blockIdx.x, tid = threadIdx.x;
  const size_t prc = (size_t)p * R * C;
  for (int e = tid; e < R * CMAX; e += blockDim.x) {
    const int r = e / CMAX, c = e % CMAX;
    T v = (T)0;
    if (c < C) {
      const size_t o = prc + plane_index<DG>(r, c, R, C);
      v = cost_adjoint<T, MET>(dcost[o], MET == MET_RAW ? (T)0 : cost[o]);
    }
    dS[e] = v;
  }
  __syncthreads();
  for (int r = tid; r < R; r += blockDim.x) {
    T acc = 0;
    for (int c = 0; c < C; ++c) acc += dS[r * CMAX + c];
    rs[r] = acc;
  }
  for (int c = tid; c < CMAX; c += blockDim.x) {
    T acc = 0;
    for (int r = 0; r < R; ++r) acc += dS[r * CMAX + c];
    cs[c] = acc;
  }
  __syncthreads();
  const T* Ap = A + (size_t)p * R * D;
  const T* Bp = Bm + (size_t)p * C * D;
  for (int d = tid; d < D; d += blockDim.x) {
    T bc[CMAX], gb[CMAX];
#pragma unroll
    for (int c = 0; c < CMAX; ++c) {
      bc[c] = c < C ? Bp[(size_t)c * D + d] : (T)0;
      gb[c] = (T)0;
    }
#pragma unroll 4
    for (int r = 0; r < R; ++r) {
      const T a = Ap[(size_t)r * D + d];
      const T* row = dS + r * CMAX;
      T s = (T)0;
#pragma unroll
      for (int c = 0; c < CMAX; ++c) {
        s += row[c] * bc[c];
        gb[c] += row[c] * a;
      }
      dA[((size_t)p * R + r) * D + d] = (T)2 * (rs[r] * a - s);
    }
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (c < C) dB[((size_t)p * C + c) * D + d] = (T)2 * (cs[c] * bc[c] - gb[c]);
  }
}

// ------------------------------------------------------------- launchers

static inline unsigned blocks_for(long long n) { return (unsigned)((n + 255) / 256); }
// Pairs per launch: the launches below put the pair index in grid.y.
constexpr int kMaxPairsPerLaunch = 65535;

// DG: the cost plane is stored by anti-diagonals (plane_index; raw metric,
// R <= C), as the uDTW sweeps read it.
template <typename T, bool DG>
static int pair_cost_fwd_impl(const T* A, const T* Bm, int P, int R, int C, int D, int metric,
                              T* out, hipStream_t s, const char* what) {
  if (P < 0 || R <= 0 || C <= 0 || D <= 0) return fail(TW_EINVAL, "%s: bad sizes", what);
  if (DG && (metric != MET_RAW || R > C))
    return fail(TW_EINVAL, "%s: internal: diagonal planes are raw with R <= C", what);
  if (P == 0) return TW_OK;
  if (!A || !Bm || !out) return fail(TW_EINVAL, "%s: null pointer", what);
  if (metric != MET_RAW && metric != MET_SQ && metric != MET_EUC)
    return fail(TW_EINVAL, "%s: unknown metric %d", what, metric);
  if ((long long)R * D >= (1LL << 29) || (long long)C * D >= (1LL << 29))
    return fail(TW_ESIZE, "%s: one pair's block must stay below 2 GiB", what);
  if (P > kMaxPairsPerLaunch) {
    // the pair index is grid.y (at most 65535): launch in chunks of pairs
    for (int p0 = 0; p0 < P; p0 += kMaxPairsPerLaunch) {
      const int np = P - p0 < kMaxPairsPerLaunch ? P - p0 : kMaxPairsPerLaunch;
      if (int e = pair_cost_fwd_impl<T, DG>(A + (size_t)p0 * R * D, Bm + (size_t)p0 * C * D, np,
                                            R, C, D, metric, out + (size_t)p0 * R * C, s, what))
        return e;
    }
    return TW_OK;
  }
  // the MFMA kernel addresses a pair's blocks with 31-bit byte offsets
  const long long lim = (1LL << 31) / (long long)sizeof(T);
  if ((long long)R * D < lim && (long long)C * D < lim) {
    // TN column tiles of 16 per wavefront share the A operand
    const int TN = C > 32 ? 4 : (C > 16 ? 2 : 1);
    const long long strips = (long long)((R + 15) / 16) * ((C + 16 * TN - 1) / (16 * TN));
    dim3 grid((unsigned)((strips + 3) / 4), P), block(256);
#define TW_PAIR_MFMA(MET_, TN_)                                                                \
  do {                                                                                         \
    if (D % 4 == 0)                                                                            \
      hipLaunchKernelGGL((pair_fwd_mfma<T, MET_, TN_, DG, true>), grid, block, 0, s, A, Bm,    \
                         out, R, C, D);                                                        \
    else                                                                                       \
      hipLaunchKernelGGL((pair_fwd_mfma<T, MET_, TN_, DG, false>), grid, block, 0, s, A, Bm,   \
                         out, R, C, D);                                                        \
  } while (0)
#define TW_PAIR_MFMA_TN(MET_)          \
  if (TN == 4) TW_PAIR_MFMA(MET_, 4);  \
  else if (TN == 2) TW_PAIR_MFMA(MET_, 2); \
  else TW_PAIR_MFMA(MET_, 1);
    if (metric == MET_RAW) { TW_PAIR_MFMA_TN(MET_RAW) }
    else if constexpr (!DG) {
      if (metric == MET_SQ) { TW_PAIR_MFMA_TN(MET_SQ) }
      else { TW_PAIR_MFMA_TN(MET_EUC) }
    }
#undef TW_PAIR_MFMA_TN
#undef TW_PAIR_MFMA
    return check_launch(what);
  }
  dim3 grid(blocks_for((long long)R * C), P), block(256);
  if (metric == MET_RAW) {
    hipLaunchKernelGGL((pair_fwd_fma<T, MET_RAW, DG>), grid, block, 0, s, A, Bm, out, R, C, D);
  } else if constexpr (!DG) {
    if (metric == MET_SQ)
      hipLaunchKernelGGL((pair_fwd_fma<T, MET_SQ, false>), grid, block, 0, s, A, Bm, out, R, C, D);
    else
      hipLaunchKernelGGL((pair_fwd_fma<T, MET_EUC, false>), grid, block, 0, s, A, Bm, out, R, C, D);
  }
  return check_launch(what);
}

template <typename T, bool DG>
static int pair_cost_bwd_impl(const T* A, const T* Bm, const T* cost, const T* dcost, int P,
                              int R, int C, int D, int metric, T* dA, T* dB, hipStream_t s,
                              const char* what) {
  if (P < 0 || R <= 0 || C <= 0 || D <= 0) return fail(TW_EINVAL, "%s: bad sizes", what);
  if (DG && (metric != MET_RAW || R > C))
    return fail(TW_EINVAL, "%s: internal: diagonal planes are raw with R <= C", what);
  if (P == 0) return TW_OK;
  if (!A || !Bm || !dcost || !dA || !dB) return fail(TW_EINVAL, "%s: null pointer", what);
  if (metric != MET_RAW && !cost) return fail(TW_EINVAL, "%s: metric needs the cost", what);
  if (metric != MET_RAW && metric != MET_SQ && metric != MET_EUC)
    return fail(TW_EINVAL, "%s: unknown metric %d", what, metric);
  if (P > kMaxPairsPerLaunch) {
    // the pair index is grid.y (at most 65535): launch in chunks of pairs
    for (int p0 = 0; p0 < P; p0 += kMaxPairsPerLaunch) {
      const int np = P - p0 < kMaxPairsPerLaunch ? P - p0 : kMaxPairsPerLaunch;
      const size_t oa = (size_t)p0 * R * D, ob = (size_t)p0 * C * D, oc = (size_t)p0 * R * C;
      if (int e = pair_cost_bwd_impl<T, DG>(A + oa, Bm + ob, cost ? cost + oc : nullptr,
                                            dcost + oc, np, R, C, D, metric, dA + oa, dB + ob, s,
                                            what))
        return e;
    }
    return TW_OK;
  }
  const int cmax = C <= 8 ? 8 : (C <= 16 ? 16 : (C <= 32 ? 32 : (C <= 64 ? 64 : 0)));
  const size_t lds = ((size_t)R * cmax + R + cmax) * sizeof(T);
  if (cmax && lds <= 48 * 1024) {
#define TW_PAIR_SMALL(MET_, CM_)                                                            \
  hipLaunchKernelGGL((pair_bwd_small<T, MET_, CM_, DG>), dim3(P), dim3(256), lds, s, A, Bm, cost, \
                     dcost, dA, dB, R, C, D)
#define TW_PAIR_SMALL_C(MET_)                  \
  if (cmax == 8) TW_PAIR_SMALL(MET_, 8);        \
  else if (cmax == 16) TW_PAIR_SMALL(MET_, 16); \
  else if (cmax == 32) TW_PAIR_SMALL(MET_, 32); \
  else TW_PAIR_SMALL(MET_, 64);
    if (metric == MET_RAW) { TW_PAIR_SMALL_C(MET_RAW) }
    else if constexpr (!DG) {
      if (metric == MET_SQ) { TW_PAIR_SMALL_C(MET_SQ) }
      else { TW_PAIR_SMALL_C(MET_EUC) }
    }
#undef TW_PAIR_SMALL_C
#undef TW_PAIR_SMALL
    return check_launch(what);
  }
  {
    // byte offsets within a pair's plane and operands fit 31 bits
    constexpr long long lim = (1LL << 31) / (long long)sizeof(T);
    constexpr int slice = sizeof(T) == 4 ? 64 : 32;
    const long long big = (long long)(R > C ? R : C) * D;
    if ((long long)R * C < lim && big < lim) {
      const unsigned ga = (unsigned)((R + 63) / 64) * P, gb = (unsigned)((C + 63) / 64) * P;
#define TW_PAIR_MFMA(MET_, NB_)                                                                  \
  hipLaunchKernelGGL((pair_bwd_mfma<T, MET_, false, NB_, DG>), dim3(ga), dim3(256), 0, s, A, Bm, \
                     cost, dcost, dA, P, R, C, D, k0);                                           \
  hipLaunchKernelGGL((pair_bwd_mfma<T, MET_, true, NB_, DG>), dim3(gb), dim3(256), 0, s, A, Bm,  \
                     cost, dcost, dB, P, R, C, D, k0);
#define TW_PAIR_MFMA_D(MET_)                                      \
  if constexpr (sizeof(T) == 4) {                                 \
    switch (nb) {                                                 \
      case 1: TW_PAIR_MFMA(MET_, 1) break;                        \
      case 2: TW_PAIR_MFMA(MET_, 2) break;                        \
      case 3: TW_PAIR_MFMA(MET_, 3) break;                        \
      default: TW_PAIR_MFMA(MET_, 4) break;                       \
    }                                                             \
  } else {                                                        \
    if (nb == 1) { TW_PAIR_MFMA(MET_, 1) } else { TW_PAIR_MFMA(MET_, 2) } \
  }
      // the passes are separable over features: larger D runs as slices,
      // each reading dS again
      for (int k0 = 0; k0 < D; k0 += slice) {
        const int nb = ((D - k0 < slice ? D - k0 : slice) + 15) / 16;
        if (metric == MET_RAW) { TW_PAIR_MFMA_D(MET_RAW) }
        else if constexpr (!DG) {
          if (metric == MET_SQ) { TW_PAIR_MFMA_D(MET_SQ) }
          else { TW_PAIR_MFMA_D(MET_EUC) }
        }
      }
#undef TW_PAIR_MFMA_D
#undef TW_PAIR_MFMA
      return check_launch(what);
    }
  }
  // float64 past 31-bit offsets: FMA tiles (a pass with 64 features would
  // need 66 KB of static LDS), D > 32 as 32-feature slices
  if (sizeof(T) == 8) {
    const dim3 ga((R + 63) / 64, P), gb((C + 63) / 64, P), block(256);
#define TW_PAIR_TILED(MET_, DPT_)                                                               \
  hipLaunchKernelGGL((pair_bwd_tiled<T, MET_, false, DPT_, DG>), ga, block, 0, s, A, Bm, cost,  \
                     dcost, dA, R, C, D, k0);                                                   \
  hipLaunchKernelGGL((pair_bwd_tiled<T, MET_, true, DPT_, DG>), gb, block, 0, s, A, Bm, cost,   \
                     dcost, dB, R, C, D, k0);
#define TW_PAIR_TILED_D(MET_)                      \
  switch (dpt) {                                   \
    case 1: TW_PAIR_TILED(MET_, 1) break;          \
    case 2: TW_PAIR_TILED(MET_, 2) break;          \
    case 4: TW_PAIR_TILED(MET_, 4) break;          \
    default: TW_PAIR_TILED(MET_, 8) break;         \
  }
    if constexpr (sizeof(T) == 8) {
      for (int k0 = 0; k0 < D; k0 += 32) {
        const int w = D - k0 < 32 ? D - k0 : 32;
        const int dpt = w <= 4 ? 1 : (w <= 8 ? 2 : (w <= 16 ? 4 : 8));
        if (metric == MET_RAW) { TW_PAIR_TILED_D(MET_RAW) }
        else if constexpr (!DG) {
          if (metric == MET_SQ) { TW_PAIR_TILED_D(MET_SQ) }
          else { TW_PAIR_TILED_D(MET_EUC) }
        }
      }
    }
#undef TW_PAIR_TILED_D
#undef TW_PAIR_TILED
    return check_launch(what);
  }
  dim3 ga(blocks_for((long long)R * D), P), gb(blocks_for((long long)C * D), P), block(256);
#define TW_PAIR_BWD(MET_)                                                                     \
  hipLaunchKernelGGL((pair_bwd_a_fma<T, MET_, DG>), ga, block, 0, s, A, Bm, cost, dcost, dA, \
                     R, C, D);                                                                \
  hipLaunchKernelGGL((pair_bwd_b_fma<T, MET_, DG>), gb, block, 0, s, A, Bm, cost, dcost, dB, \
                     R, C, D);
  if (metric == MET_RAW) {
    TW_PAIR_BWD(MET_RAW)
  } else if constexpr (!DG) {
    if (metric == MET_SQ) { TW_PAIR_BWD(MET_SQ) }
    else { TW_PAIR_BWD(MET_EUC) }
  }
#undef TW_PAIR_BWD
  return check_launch(what);
}

// Row-major cost planes (the public pairwise-cost entry points, JEANIE).
template <typename T>
int pair_cost_fwd(const T* A, const T* Bm, int P, int R, int C, int D, int metric, T* out,
                  hipStream_t s, const char* what) {
  return pair_cost_fwd_impl<T, false>(A, Bm, P, R, C, D, metric, out, s, what);
}

template <typename T>
int pair_cost_bwd(const T* A, const T* Bm, const T* cost, const T* dcost, int P, int R, int C,
                  int D, int metric, T* dA, T* dB, hipStream_t s, const char* what) {
  return pair_cost_bwd_impl<T, false>(A, Bm, cost, dcost, P, R, C, D, metric, dA, dB, s, what);
}

template <typename T>
int sqdist_raw(const T* X, const T* Y, int P, int R, int C, int D, T* out, hipStream_t s,
               const char* what) {
  return pair_cost_fwd_impl<T, true>(X, Y, P, R, C, D, MET_RAW, out, s, what);
}

template <typename T>
int sqdist_raw_bwd(const T* X, const T* Y, const T* dS, int P, int R, int C, int D, T* dX, T* dY,
                   hipStream_t s, const char* what) {
  return pair_cost_bwd_impl<T, true>(X, Y, nullptr, dS, P, R, C, D, MET_RAW, dX, dY, s, what);
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
