// Second-order uDTW / soft-DTW: the tangent of the first-order gradient.
//
// For L = gR * r + gP * p (r = R[N-1,M-1], p = P[N-1,M-1]) the first-order
// backward returns (dL/dC, dL/dQ) = (Gt, At). The reference differentiates
// that backward with torch.func over its autograd-native dynamic program
// (udtw/_ops.py:322-339 DPBackward.backward / jvp on udtw/_autograd.py:32-74);
// here its derivative along a direction (tC, tQ, tgR, tgP) is computed by two
// explicit tangent sweeps:
//
//   forward, cell (i,j), predecessors k with softmin weights w_k:
//     R  = C + softmin(R_k)            tR = tC + sum_k w_k tR_k
//     P  = Q + sum_k w_k P_k           tP = tQ + sum_k w_k tP_k + tw_k P_k,
//     tw_k = -(w_k / g)(tR_k - tRbar),  tRbar = tR - tC
//   backward, cell k, successors s, w = exp((Rbar_s - R_k)/g),
//   tw = -(w/g)(tR_k - tRbar_s), dP = P_k - Pbar_s, tdP = tP_k - tPbar_s:
//     At  += w At_s                    tAt += w tAt_s + tw At_s
//     Gt  += w Gt_s - w At_s dP / g
//     tGt += w tGt_s + tw Gt_s - (w tAt_s + tw At_s) dP / g - w At_s tdP / g
//   seeded at the end cell with (gR, gP, tgR, tgP).
//
// Outputs: (tGt, tAt) -- the tangent of (dL/dC, dL/dQ) -- and tR, tP at the
// end cell. (dL/dC, dL/dQ) is the gradient of L, so its Jacobian is L's
// symmetric Hessian: with tgR = tgP = 0 the same numbers are the
// vector-Jacobian product of a double backward, and (tR, tP) at the end cell
// its gradients with respect to gR and gP.
//
// Layout: one workgroup per pair walks the anti-diagonals, rows spread over
// its threads (row i on thread i mod blockDim). Three diagonals of the values
// a cell reads from its neighbours rotate through a ring in LDS (or, when
// the ring is larger than the LDS, in a per-pair slice of the workspace; one
// workgroup's global stores are visible to its own loads after a barrier).
// The forward's R, tR, P, tP planes go to the workspace in a skewed layout
// (cell (i,j) at ((i + j) mod M) * N + i: one diagonal is one contiguous
// row), so the backward reads them coalesced.
#include "tw_capi.hpp"
#include "tw_common.hpp"

namespace tw {
namespace {

template <typename T>
struct TanArgs {
  const T *cost, *pen, *tcost, *tpen;  // [B,N,M]; pen / tcost / tpen may be null
  const T *gr, *gp, *tgr, *tgp;        // [B]; gp, tgr, tgp may be null
  T *out_c, *out_q;                    // [B,N,M]; out_q null without a penalty
  T *out_r, *out_p;                    // [B]; may be null
  T* planes;                           // [B][NQF][M][N]
  T* gring;                            // [B][ring] when the ring is not in LDS
  long long ring;                      // ring elements per pair
  int N, M;
  T gamma, band;                       // band <= 0: no band
};

constexpr double kLog2e = 1.4426950408889634;
constexpr double kLn2 = 0.6931471805599453;
// Threads per workgroup at most (rows beyond take further turns of the row
// loop): at 512 the float64 sweeps keep every value in registers.
constexpr int kTanThreads = 512;

template <typename T>
__host__ __device__ __forceinline__ T ld0(const T* p, size_t k) {
  return p ? p[k] : T(0);
}

// Arithmetic of the sweeps. float: the hardware transcendental unit; double:
// the math library (also callable on the host, where the sweeps of one pair
// can be run sequentially to check their indexing).
__device__ __forceinline__ float t_ex2(float x) { return ex2(x); }
__device__ __forceinline__ float t_lg2(float x) { return lg2(x); }
__host__ __device__ __forceinline__ double t_ex2(double x) { return exp2(x); }
__host__ __device__ __forceinline__ double t_lg2(double x) { return log2(x); }
template <typename T> __host__ __device__ __forceinline__ T t_inf();
template <> __host__ __device__ __forceinline__ float t_inf<float>() { return __builtin_inff(); }
template <> __host__ __device__ __forceinline__ double t_inf<double>() { return __builtin_inf(); }

// The workgroup as the sweeps see it: thread index, thread count, barrier.
struct WorkgroupCtx {
  __device__ int tid() const { return threadIdx.x; }
  __device__ int size() const { return blockDim.x; }
  __device__ void sync() const { __syncthreads(); }
};

// Both sweeps of pair b; `ring` holds the exchanged diagonals.
// Forward ring: quantity q (R, tR, P, tP) of diagonal slot s, row i at
// (q * 3 + s) * N + i. Backward ring: (Rbar, tRbar, Gt, tGt, Pbar, tPbar,
// At, tAt) likewise.
template <typename T, bool PEN, class Ctx>
__host__ __device__ inline void tangent_pair(const TanArgs<T>& a, int b, T* ring, const Ctx& ctx) {
  constexpr int NQF = PEN ? 4 : 2;
  const int N = a.N, M = a.M, BS = ctx.size(), tid = ctx.tid();
  const size_t nm = (size_t)N * M;
  const T* C = a.cost + b * nm;
  const T* Q = PEN ? a.pen + b * nm : nullptr;
  const T* TC = a.tcost ? a.tcost + b * nm : nullptr;
  const T* TQ = (PEN && a.tpen) ? a.tpen + b * nm : nullptr;
  T* pl = a.planes + (size_t)b * NQF * nm;
  const T ig = T(1) / a.gamma;
  const T k2 = T(kLog2e) * ig, ln2g = T(kLn2) * a.gamma;
  const T INF = t_inf<T>();
  const int D = N + M - 1;
  auto rq = [&](int q, int s, int i) -> T& { return ring[(size_t)(q * 3 + s) * N + i]; };
  auto in_band = [&](int i, int j) { return !(a.band > T(0)) || fabs(T(i - j)) <= a.band; };

  // ------------------------------------------------------ forward tangent
  for (int d = 0, dm = 0; d < D; ++d, dm = (dm + 1 == M) ? 0 : dm + 1) {
    const int sd = d % 3, s1 = (d + 2) % 3, s2 = (d + 1) % 3;
    for (int i = tid; i < N; i += BS) {
      const int j = d - i;
      if (j < 0 || j >= M) continue;
      const size_t cij = (size_t)i * M + j;
      const T c = C[cij], tc = ld0(TC, cij);
      T r = INF, tr = T(0), p = T(0), tp = T(0);
      if (in_band(i, j)) {
        if (d == 0) {
          r = c;
          tr = tc;
          if (PEN) {
            p = Q[cij];
            tp = ld0(TQ, cij);
          }
        } else {
          T Ru = INF, Rl = INF, Rg = INF, Du = 0, Dl = 0, Dg = 0;
          T Pu = 0, Pl = 0, Pg = 0, Eu = 0, El = 0, Eg = 0;
          if (i > 0) {
            Ru = rq(0, s1, i - 1);
            Du = rq(1, s1, i - 1);
            if (PEN) {
              Pu = rq(2, s1, i - 1);
              Eu = rq(3, s1, i - 1);
            }
          }
          if (j > 0) {
            Rl = rq(0, s1, i);
            Dl = rq(1, s1, i);
            if (PEN) {
              Pl = rq(2, s1, i);
              El = rq(3, s1, i);
            }
          }
          if (i > 0 && j > 0) {
            Rg = rq(0, s2, i - 1);
            Dg = rq(1, s2, i - 1);
            if (PEN) {
              Pg = rq(2, s2, i - 1);
              Eg = rq(3, s2, i - 1);
            }
          }
          const T m = fmin(Ru, fmin(Rl, Rg));
          if (m < INF) {
            const T eu = t_ex2((m - Ru) * k2), el = t_ex2((m - Rl) * k2), eg = t_ex2((m - Rg) * k2);
            const T S = eu + el + eg, iS = T(1) / S;
            const T wu = eu * iS, wl = el * iS, wg = eg * iS;
            r = c + (m - ln2g * t_lg2(S));
            const T trb = wu * Du + wl * Dl + wg * Dg;
            tr = tc + trb;
            if (PEN) {
              const T pb = wu * Pu + wl * Pl + wg * Pg;
              p = Q[cij] + pb;
              const T cross = wu * (Du - trb) * (Pu - pb) + wl * (Dl - trb) * (Pl - pb) +
                              wg * (Dg - trb) * (Pg - pb);
              tp = ld0(TQ, cij) + (wu * Eu + wl * El + wg * Eg) - ig * cross;
            }
          }
        }
      }
      rq(0, sd, i) = r;
      rq(1, sd, i) = tr;
      const size_t k = (size_t)dm * N + i;
      pl[k] = r;
      pl[nm + k] = tr;
      if (PEN) {
        rq(2, sd, i) = p;
        rq(3, sd, i) = tp;
        pl[2 * nm + k] = p;
        pl[3 * nm + k] = tp;
      }
      if (d == D - 1) {
        if (a.out_r) a.out_r[b] = tr;
        if (PEN && a.out_p) a.out_p[b] = tp;
      }
    }
    ctx.sync();
  }

  // ----------------------------------------------------- backward tangent
  const T gR = a.gr[b], gP = (PEN && a.gp) ? a.gp[b] : T(0);
  const T tgR = a.tgr ? a.tgr[b] : T(0), tgP = (PEN && a.tgp) ? a.tgp[b] : T(0);
  for (int d = D - 1, dm = (D - 1) % M; d >= 0; --d, dm = (dm == 0) ? M - 1 : dm - 1) {
    const int sd = d % 3, n1 = (d + 1) % 3, n2 = (d + 2) % 3;
    for (int i = tid; i < N; i += BS) {
      const int j = d - i;
      if (j < 0 || j >= M) continue;
      const size_t cij = (size_t)i * M + j, k = (size_t)dm * N + i;
      const T r = pl[k], tr = pl[nm + k];
      T p = 0, tp = 0;
      if (PEN) {
        p = pl[2 * nm + k];
        tp = pl[3 * nm + k];
      }
      T G = 0, tG = 0, A = 0, tA = 0;
      if (r < INF) {
        if (d == D - 1) {
          G = gR;
          tG = tgR;
          A = gP;
          tA = tgP;
        } else {
          // successors: (i+1, j) on d+1 row i+1, (i, j+1) on d+1 row i,
          // (i+1, j+1) on d+2 row i+1
#pragma unroll
          for (int s = 0; s < 3; ++s) {
            const int si = (s == 1) ? i : i + 1, sj = (s == 0) ? j : j + 1;
            if (si >= N || sj >= M) continue;
            const int sl = (s == 2) ? n2 : n1;
            const T Rb = rq(0, sl, si);
            const T w = t_ex2((Rb - r) * k2);
            const T tw = -(w * ig) * (tr - rq(1, sl, si));
            const T Gs = rq(2, sl, si), tGs = rq(3, sl, si);
            if (PEN) {
              const T As = rq(6, sl, si), tAs = rq(7, sl, si);
              const T dP = p - rq(4, sl, si), tdP = tp - rq(5, sl, si);
              A += w * As;
              tA += w * tAs + tw * As;
              G += w * Gs - w * As * dP * ig;
              tG += w * tGs + tw * Gs - (w * tAs + tw * As) * dP * ig - w * As * tdP * ig;
            } else {
              G += w * Gs;
              tG += w * tGs + tw * Gs;
            }
          }
        }
      }
      a.out_c[b * nm + cij] = tG;
      if (PEN) a.out_q[b * nm + cij] = tA;
      const T c = C[cij];
      rq(0, sd, i) = (r < INF) ? r - c : -INF;
      rq(1, sd, i) = tr - ld0(TC, cij);
      rq(2, sd, i) = G;
      rq(3, sd, i) = tG;
      if (PEN) {
        rq(4, sd, i) = p - Q[cij];
        rq(5, sd, i) = tp - ld0(TQ, cij);
        rq(6, sd, i) = A;
        rq(7, sd, i) = tA;
      }
    }
    ctx.sync();
  }
}

template <typename T, bool PEN>
__global__ __launch_bounds__(kTanThreads) void udtw_tangent_kernel(TanArgs<T> a) {
  extern __shared__ __align__(16) unsigned char tan_lds[];
  const int b = blockIdx.x;
  T* ring = a.gring ? a.gring + (size_t)b * a.ring : reinterpret_cast<T*>(tan_lds);
  tangent_pair<T, PEN>(a, b, ring, WorkgroupCtx{});
}

// Off until the cause of the fault their first GPU run hit is found (the
// arguments are still checked, so the entry points report misuse first).
constexpr bool kTangentEnabled = false;

int threads_for(int N) {
  const int t = ((N + 63) / 64) * 64;
  return t < kTanThreads ? t : kTanThreads;
}

// Per-pair sizes (elements): the forward planes and the ring.
size_t plane_elems(int N, int M, bool pen) { return (size_t)(pen ? 4 : 2) * N * M; }
size_t ring_elems(int N, bool pen) { return (size_t)3 * (pen ? 8 : 4) * N; }

bool ring_in_lds(int N, bool pen, size_t es) {
  return ring_elems(N, pen) * es <= (size_t)max_lds_bytes();
}

size_t workspace_bytes(int B, int N, int M, bool pen, size_t es) {
  if (B <= 0 || N <= 0 || M <= 0) return 0;
  size_t per = plane_elems(N, M, pen);
  if (!ring_in_lds(N, pen, es)) per += ring_elems(N, pen);
  return (size_t)B * per * es;
}

template <typename T>
int tangent(const T* cost, const T* pen, const T* tcost, const T* tpen, const T* gr,
            const T* gp, const T* tgr, const T* tgp, int B, int N, int M, T gamma, T band,
            T* out_c, T* out_q, T* out_r, T* out_p, T* ws, size_t ws_bytes, hipStream_t stream,
            const char* what) {
  if (B < 0 || N < 1 || M < 1) return fail(TW_EINVAL, "%s: bad sizes B=%d N=%d M=%d", what, B, N, M);
  if (B == 0) return TW_OK;
  if (!(gamma > T(0))) return fail(TW_EINVAL, "%s: gamma must be positive", what);
  if (!cost || !gr || !out_c) return fail(TW_EINVAL, "%s: null cost, grad or output", what);
  const bool has_pen = pen != nullptr;
  if (has_pen && !out_q) return fail(TW_EINVAL, "%s: a penalty needs d_pen_tangent", what);
  const size_t need = workspace_bytes(B, N, M, has_pen, sizeof(T));
  if (!ws || ws_bytes < need) {
    return fail(TW_EINVAL, "%s: workspace of %zu bytes given, %zu needed", what, ws_bytes, need);
  }
  if (!kTangentEnabled) {
    return fail(TW_EINVAL,
                "%s: the second-order sweeps are disabled in this build: their first run on an "
                "MI355X stopped with a memory aperture violation whose cause is not yet found",
                what);
  }
  TanArgs<T> a;
  a.cost = cost;
  a.pen = pen;
  a.tcost = tcost;
  a.tpen = tpen;
  a.gr = gr;
  a.gp = gp;
  a.tgr = tgr;
  a.tgp = tgp;
  a.out_c = out_c;
  a.out_q = out_q;
  a.out_r = out_r;
  a.out_p = out_p;
  a.planes = ws;
  a.ring = (long long)ring_elems(N, has_pen);
  const bool lds = ring_in_lds(N, has_pen, sizeof(T));
  a.gring = lds ? nullptr : ws + (size_t)B * plane_elems(N, M, has_pen);
  a.N = N;
  a.M = M;
  a.gamma = gamma;
  a.band = band;
  const size_t shm = lds ? ring_elems(N, has_pen) * sizeof(T) : 0;
  const dim3 grid((unsigned)B), block((unsigned)threads_for(N));
  if (has_pen) {
    hipLaunchKernelGGL((udtw_tangent_kernel<T, true>), grid, block, shm, stream, a);
  } else {
    hipLaunchKernelGGL((udtw_tangent_kernel<T, false>), grid, block, shm, stream, a);
  }
  return check_launch(what);
}

}  // namespace
}  // namespace tw

using namespace tw;

extern "C" {

size_t tw_udtw_tangent_workspace_bytes(int B, int N, int M, int has_penalty, int elem_size) {
  return workspace_bytes(B, N, M, has_penalty != 0, (size_t)elem_size);
}

int tw_udtw_cost_tangent_f32(const float* cost, const float* pen, const float* t_cost,
                             const float* t_pen, const float* grad_dist, const float* grad_pen,
                             const float* t_grad_dist, const float* t_grad_pen, int B, int N,
                             int M, float gamma, float bandwidth, float* t_d_cost,
                             float* t_d_pen, float* t_dist, float* t_pen_sum, float* workspace,
                             size_t workspace_bytes, hipStream_t stream) {
  return tangent<float>(cost, pen, t_cost, t_pen, grad_dist, grad_pen, t_grad_dist, t_grad_pen,
                        B, N, M, gamma, bandwidth, t_d_cost, t_d_pen, t_dist, t_pen_sum,
                        workspace, workspace_bytes, stream, "tw_udtw_cost_tangent_f32");
}

int tw_udtw_cost_tangent_f64(const double* cost, const double* pen, const double* t_cost,
                             const double* t_pen, const double* grad_dist,
                             const double* grad_pen, const double* t_grad_dist,
                             const double* t_grad_pen, int B, int N, int M, double gamma,
                             double bandwidth, double* t_d_cost, double* t_d_pen, double* t_dist,
                             double* t_pen_sum, double* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
  return tangent<double>(cost, pen, t_cost, t_pen, grad_dist, grad_pen, t_grad_dist, t_grad_pen,
                         B, N, M, gamma, bandwidth, t_d_cost, t_d_pen, t_dist, t_pen_sum,
                         workspace, workspace_bytes, stream, "tw_udtw_cost_tangent_f64");
}

}  // extern "C"
