/*
 * torchwarp_hip.h -- C ABI of the gfx950 (MI355X) backend for torchwarp's
 * alignment hot path: soft-DTW, uncertainty-DTW (uDTW), JEANIE and FVM,
 * forward and backward, plus the pairwise cost builders.
 *
 * Conventions
 *  - Every pointer is a device pointer; the caller allocates every output and
 *    workspace buffer (the library never allocates). All tensors are dense
 *    and row-major in the layout stated for each argument.
 *  - Launches are asynchronous on `stream`; no host synchronisation.
 *  - Returns TW_OK (0) or an error code; the message is in tw_last_error()
 *    (thread-local). B = 0 is a no-op returning TW_OK.
 *  - _f32 and _f64 variants compute in float / double.
 *  - "R" and "P" buffers of the uDTW functions are internal tensors carried
 *    from a forward call to the matching backward call (opaque layout; P is
 *    [B, N*M] elements, R takes tw_udtw_carry_bytes bytes). The JEANIE "R"
 *    is the accumulator in the cost's own layout.
 *
 * Citations (file:line) are into the reference torchwarp sources
 * (src/torchwarp/...): each entry point replaces the named pybind function
 * of the reference CUDA extension and the Python op that wraps it.
 */
#ifndef TORCHWARP_HIP_H
#define TORCHWARP_HIP_H

#include <stddef.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TW_ABI_VERSION 1

#define TW_OK 0
#define TW_EINVAL 1  /* bad argument */
#define TW_ELAUNCH 2 /* kernel launch failed */
#define TW_ESIZE 3   /* problem larger than this build handles / workspace too small */
#define TW_EWAIT 4   /* an earlier launch's bounded cross-workgroup wait gave up */

/* Bits of the per-device asynchronous status word (tw_async_status). */
#define TW_STATUS_WAIT_GAVE_UP 1u

/* Pairwise metrics (tw_pair_cost_*, tw_jeanie_feat_*). */
#define TW_METRIC_RAW 0   /* |a|^2 + |b|^2 - 2 a.b, unclamped */
#define TW_METRIC_SQEUC 1 /* max(., 0)                        */
#define TW_METRIC_EUC 2   /* sqrt(max(., 0)), zero gradient at 0 */

int tw_version(void);
const char* tw_last_error(void);

/* Asynchronous status of the current device. A uDTW sweep split over several
 * workgroups per pair hands boundary rows between them and waits for each
 * with a poll bounded in time (2 s on the device's real-time counter); if a
 * wait runs out (the producing workgroup was held off the GPU for that long)
 * the kernel sets TW_STATUS_WAIT_GAVE_UP in a per-device word, its outputs
 * become NaN, and it exits normally. This call
 * synchronises the device, then returns TW_EWAIT if the bit is set (clearing
 * it when `clear` is non-zero) or TW_OK. It is sticky across calls, like an
 * asynchronous launch error, and must not be called during stream capture.
 * No counterpart in the reference: its kernels never wait on each other. */
int tw_async_status(int clear);
/* Test hook (no counterpart in the reference): a limit of `spins` poll rounds
 * for those waits (spins > 0; 0 restores the time bound alone) and, with
 * drop_handoff != 0, boundary
 * rows that are never handed over, so that a test can make a wait give up
 * while every kernel still exits normally. Process-wide; not for production. */
void tw_test_set_wait(int spins, int drop_handoff);
/* Test hook (no counterpart in the reference): how uDTW splits a pair over
 * workgroups, overriding TORCHWARP_UDTW_MW: 0 one workgroup per pair (then
 * at most 1024 rows in float, 512 in double), 1 several workgroups whenever a
 * pair has more than 256 rows, 2 the default (several workgroups for
 * sequences longer than one workgroup holds, and for small batches in the
 * forward), -1 back to the environment's choice. Process-wide; sizes queried
 * before a change do not apply after it. Not for production. */
void tw_test_set_mw(int mode);

/* ---------------------------------------------------------------- uDTW --
 * Bytes of the R buffer a uDTW forward fills and the matching backward reads,
 * for B pairs of N x M (N <= M) at this gamma: B*N*M*elem_size, except that
 * _f32 calls keep R in double precision (B*N*M*8 bytes) when the accumulated
 * cost can grow large against float32's spacing ((N + M - 1) log2(e) / gamma
 * above 2048, one row per thread serving N, the double plane below 2 GiB). No counterpart in the reference,
 * whose float32 kernels keep R in float32. Host only. */
size_t tw_udtw_carry_bytes(int B, int N, int M, double gamma, int elem_size);

/* DP on precomputed matrices, N <= M (callers transpose).
 * Replaces udtw_cuda.cu:624-657 (forward) / :659-690 (backward) and the ops
 * torchwarp_udtw::dp / dp_backward (udtw/_ops.py:100-138).
 * cost, pen: [B,N,M]; pen may be NULL (zero penalty, P unused).
 * R: tw_udtw_carry_bytes(B, N, M, gamma, elem) bytes, P: [B, N*M], internal;
 * out_dist, out_pen: [B].
 * Backward: the forward's bandwidth; grad_dist, grad_pen [B] (grad_pen may be
 * NULL iff pen is NULL), read with element stride grad_stride (1, or 0 for one
 * value shared by every pair, e.g. the expanded gradient of a mean);
 * d_cost, d_pen [B,N,M] (d_pen may be NULL); workspace of
 * tw_udtw_cost_workspace_bytes(...) bytes (NULL when that is 0): sequences
 * longer than one workgroup holds (N > 1024 in float, 512 in double) run with
 * several workgroups per pair, which hand boundary records to each other
 * through it. There is no length limit beyond the 2 GiB of one pair's N*M
 * planes (32-bit offsets within a pair). */
size_t tw_udtw_cost_workspace_bytes(int B, int N, int M, int elem_size);
/* The workspace with which a banded backward (a Sakoe-Chiba band narrower
 * than the grid) first keeps d_cost / d_pen in the band layout of its sweep
 * and then scatters them into [B,N,M], instead of writing them there one
 * cache line per lane (no counterpart in the reference, which only masks);
 * at least tw_udtw_cost_workspace_bytes. A smaller workspace keeps the
 * direct writes. */
size_t tw_udtw_cost_band_workspace_bytes(int B, int N, int M, double bandwidth, int elem_size);
int tw_udtw_cost_fwd_f32(const float* cost, const float* pen, int B, int N, int M, float gamma,
                         float bandwidth, float* R, float* P, float* out_dist, float* out_pen,
                         hipStream_t stream);
int tw_udtw_cost_fwd_f64(const double* cost, const double* pen, int B, int N, int M,
                         double gamma, double bandwidth, double* R, double* P, double* out_dist,
                         double* out_pen, hipStream_t stream);
int tw_udtw_cost_bwd_f32(const float* cost, const float* pen, const float* R, const float* P,
                         const float* grad_dist, const float* grad_pen, int B, int N, int M,
                         float gamma, float bandwidth, int grad_stride, float* d_cost,
                         float* d_pen, float* workspace, size_t workspace_bytes,
                         hipStream_t stream);
int tw_udtw_cost_bwd_f64(const double* cost, const double* pen, const double* R,
                         const double* P, const double* grad_dist, const double* grad_pen, int B,
                         int N, int M, double gamma, double bandwidth, int grad_stride,
                         double* d_cost, double* d_pen, double* workspace,
                         size_t workspace_bytes, hipStream_t stream);

/* Second order of the DP on precomputed matrices: the derivative of the
 * backward's (d_cost, d_pen) along a direction (t_cost, t_pen, t_grad_dist,
 * t_grad_pen), and the derivatives of (dist, pen) along (t_cost, t_pen).
 * Replaces the reference's double backward and forward-mode rule of
 * torchwarp_udtw::dp_backward (udtw/_ops.py:322-339 DPBackward.backward /
 * jvp), which run torch.func over udtw/_autograd.py:32-74. Because
 * (d_cost, d_pen) is a gradient, its Jacobian is symmetric: with
 * t_grad_* = 0, (t_d_cost, t_d_pen) is also the vector-Jacobian product a
 * double backward needs, and (t_dist, t_pen_sum) its gradients with respect
 * to grad_dist and grad_pen.
 * cost, pen, t_cost, t_pen, t_d_cost, t_d_pen: [B,N,M] (any N, M); pen NULL
 * means no penalty (then t_pen, grad_pen, t_grad_pen, t_d_pen, t_pen_sum are
 * unused); t_cost, t_pen, t_grad_* NULL mean zero; grad_dist, grad_pen,
 * t_grad_*, t_dist, t_pen_sum: [B] (t_dist, t_pen_sum may be NULL). Same
 * bandwidth convention as the forward. workspace:
 * tw_udtw_tangent_workspace_bytes(B, N, M, pen != NULL, elem) bytes (the
 * forward's R, P and their tangents, and for long sequences the diagonals
 * the sweeps exchange).
 * Currently switched off: after checking the arguments the calls return
 * TW_EINVAL without launching (their first run on an MI355X stopped with a
 * memory aperture violation whose cause is not yet found). */
size_t tw_udtw_tangent_workspace_bytes(int B, int N, int M, int has_penalty, int elem_size);
int tw_udtw_cost_tangent_f32(const float* cost, const float* pen, const float* t_cost,
                             const float* t_pen, const float* grad_dist, const float* grad_pen,
                             const float* t_grad_dist, const float* t_grad_pen, int B, int N,
                             int M, float gamma, float bandwidth, float* t_d_cost,
                             float* t_d_pen, float* t_dist, float* t_pen_sum, float* workspace,
                             size_t workspace_bytes, hipStream_t stream);
int tw_udtw_cost_tangent_f64(const double* cost, const double* pen, const double* t_cost,
                             const double* t_pen, const double* grad_dist,
                             const double* grad_pen, const double* t_grad_dist,
                             const double* t_grad_pen, int B, int N, int M, double gamma,
                             double bandwidth, double* t_d_cost, double* t_d_pen, double* t_dist,
                             double* t_pen_sum, double* workspace, size_t workspace_bytes,
                             hipStream_t stream);

/* uDTW straight from the features, N <= M. Replaces udtw_cuda.cu:738-775
 * (fused_forward) / :777-814 (fused_backward) together with the bmm / vecdot /
 * diagonal permutations of the ops torchwarp_udtw::fused / fused_backward
 * (udtw/_ops.py:157-211). X [B,N,D], Y [B,M,D], vx [B,N], vy [B,M]: the
 * variances sigma^2, or with sigma != 0 the standard deviations sigma (the
 * kernels square them; this folds the reference's sigma.pow(2) of
 * udtw/functional.py:157-158 and its backward into the call).
 * beta == 0 (soft-DTW) skips the penalty: P may be NULL, out_pen gets 0.
 * R: tw_udtw_carry_bytes(B, N, M, gamma, elem) bytes, P: [B, N*M], internal.
 * D == 1 runs fully fused; the forward with D > 1 needs workspace of
 * B*N*M elements (the squared distances), the backward
 * tw_udtw_feat_workspace_bytes(...) bytes: those squared distances (D > 1),
 * then, for sequences longer than one workgroup holds (N > 1024 in float, 512
 * in double; several workgroups per pair), their boundary hand-off records.
 * There is no length limit beyond the 2 GiB of one pair's N*M planes.
 * Backward: grad_dist / grad_pen
 * with element stride grad_stride (1, or 0: one shared value); writes
 * dX [B,N,D], dY [B,M,D] and, unless both are NULL, dvx [B,N], dvy [B,M]
 * (gradients with respect to vx, vy as given: d sigma when sigma != 0).
 * fwd_workspace: for D > 1, the forward's workspace as that call left it (it
 * holds the pairwise squared distances), or NULL to recompute them into
 * workspace. The backward writes their adjoint into workspace; fwd_workspace
 * is only read, unless it is workspace itself. */
size_t tw_udtw_feat_workspace_bytes(int B, int N, int M, int D, int elem_size);

/* Workspace of tw_udtw_feat_fwd / tw_udtw_feat_bwd for a given bandwidth (the
 * band of udtw_cuda.cu:126-130). A Sakoe-Chiba band narrower than the grid
 * runs the banded feature path, D = 1 included: cost, penalty, R and P in a
 * band layout built in a workspace of B*N*M elements, which both directions
 * then need; otherwise this equals tw_udtw_feat_workspace_bytes. No
 * counterpart in the reference, whose band only masks cells. */
size_t tw_udtw_feat_band_workspace_bytes(int B, int N, int M, int D, double bandwidth,
                                         int elem_size);
int tw_udtw_feat_fwd_f32(const float* X, const float* Y, const float* vx, const float* vy, int B,
                         int N, int M, int D, float gamma, float beta, float eps,
                         float bandwidth, int sigma, float* R, float* P, float* out_dist,
                         float* out_pen, float* workspace, size_t workspace_bytes,
                         hipStream_t stream);
int tw_udtw_feat_fwd_f64(const double* X, const double* Y, const double* vx, const double* vy,
                         int B, int N, int M, int D, double gamma, double beta, double eps,
                         double bandwidth, int sigma, double* R, double* P, double* out_dist,
                         double* out_pen, double* workspace, size_t workspace_bytes,
                         hipStream_t stream);
int tw_udtw_feat_bwd_f32(const float* X, const float* Y, const float* vx, const float* vy,
                         const float* R, const float* P, const float* grad_dist,
                         const float* grad_pen, int B, int N, int M, int D, float gamma,
                         float beta, float eps, float bandwidth, int sigma, int grad_stride,
                         float* dX, float* dY, float* dvx, float* dvy,
                         const float* fwd_workspace, float* workspace,
                         size_t workspace_bytes, hipStream_t stream);
int tw_udtw_feat_bwd_f64(const double* X, const double* Y, const double* vx, const double* vy,
                         const double* R, const double* P, const double* grad_dist,
                         const double* grad_pen, int B, int N, int M, int D, double gamma,
                         double beta, double eps, double bandwidth, int sigma, int grad_stride,
                         double* dX, double* dY, double* dvx, double* dvy,
                         const double* fwd_workspace, double* workspace,
                         size_t workspace_bytes, hipStream_t stream);

/* -------------------------------------------------------------- JEANIE --
 * 3-D DP on a cost [B, K1*K2, T, U] (swap_tu = 0) or [B, K1*K2, U, T]
 * (swap_tu = 1: the DP runs on the transposed grid, T <= U required).
 * Shifts are clamped to K-1. R: accumulator, same layout as cost; out: [B].
 * Replaces jeanie_cuda.cu:564-587 (forward) / :589-619 (backward) and the
 * ops torchwarp_jeanie::dp / dp_backward (jeanie/_ops.py:110-139).
 * grad_R (dL/dR, same layout) may be NULL. */
int tw_jeanie_cost_fwd_f32(const float* cost, int B, int K1, int K2, int T, int U, int swap_tu,
                           int s1, int s2, float gamma, float* R, float* out, hipStream_t stream);
int tw_jeanie_cost_fwd_f64(const double* cost, int B, int K1, int K2, int T, int U, int swap_tu,
                           int s1, int s2, double gamma, double* R, double* out,
                           hipStream_t stream);
int tw_jeanie_cost_bwd_f32(const float* cost, const float* R, const float* grad_out,
                           const float* grad_R, int B, int K1, int K2, int T, int U, int swap_tu,
                           int s1, int s2, float gamma, float* d_cost, hipStream_t stream);
int tw_jeanie_cost_bwd_f64(const double* cost, const double* R, const double* grad_out,
                           const double* grad_R, int B, int K1, int K2, int T, int U,
                           int swap_tu, int s1, int s2, double gamma, double* d_cost,
                           hipStream_t stream);

/* JEANIE from features: query [B, K1*K2, T, D], support [B, U, D],
 * metric TW_METRIC_SQEUC or TW_METRIC_EUC. Writes the cost [B, K1*K2, T, U]
 * (saved for the backward), the accumulator R (same layout) and out [B].
 * Replaces jeanie_cuda.cu:621-648 / :650-683 with the ops
 * torchwarp_jeanie::features / features_backward (jeanie/_ops.py:155-230).
 * Backward workspace: B*K1*K2*T*U elements. */
int tw_jeanie_feat_fwd_f32(const float* query, const float* support, int B, int K1, int K2, int T,
                           int U, int D, int s1, int s2, float gamma, int metric, float* cost,
                           float* R, float* out, hipStream_t stream);
int tw_jeanie_feat_fwd_f64(const double* query, const double* support, int B, int K1, int K2,
                           int T, int U, int D, int s1, int s2, double gamma, int metric,
                           double* cost, double* R, double* out, hipStream_t stream);
int tw_jeanie_feat_bwd_f32(const float* query, const float* support, const float* cost,
                           const float* R, const float* grad_out, const float* grad_R, int B,
                           int K1, int K2, int T, int U, int D, int s1, int s2, float gamma,
                           int metric, float* d_query, float* d_support, float* workspace,
                           hipStream_t stream);
int tw_jeanie_feat_bwd_f64(const double* query, const double* support, const double* cost,
                           const double* R, const double* grad_out, const double* grad_R, int B,
                           int K1, int K2, int T, int U, int D, int s1, int s2, double gamma,
                           int metric, double* d_query, double* d_support, double* workspace,
                           hipStream_t stream);

/* ----------------------------------------------------------------- FVM --
 * fvm_from_cost (jeanie/fvm.py:15-38: logsumexp over the viewpoints, then
 * soft_dtw_from_cost, sdtw.py:29-47) on cost [B, K, T, U], K = product of
 * the viewpoint dims. temporal: [B, T*U] (saved), R: [B, T*U] internal,
 * out [B], scratch [B]. Backward workspace: tw_fvm_workspace_bytes(...)
 * bytes (B*T*U elements, plus the hand-off records of the soft-DTW backward
 * when min(T, U) is longer than one workgroup holds). */
size_t tw_fvm_workspace_bytes(int B, int K, int T, int U, int elem_size);
int tw_fvm_cost_fwd_f32(const float* cost, int B, int K, int T, int U, float gamma,
                        float* temporal, float* R, float* out, float* scratch,
                        hipStream_t stream);
int tw_fvm_cost_fwd_f64(const double* cost, int B, int K, int T, int U, double gamma,
                        double* temporal, double* R, double* out, double* scratch,
                        hipStream_t stream);
int tw_fvm_cost_bwd_f32(const float* cost, const float* temporal, const float* R,
                        const float* grad_out, int B, int K, int T, int U, float gamma,
                        float* d_cost, float* workspace, size_t workspace_bytes,
                        hipStream_t stream);
int tw_fvm_cost_bwd_f64(const double* cost, const double* temporal, const double* R,
                        const double* grad_out, int B, int K, int T, int U, double gamma,
                        double* d_cost, double* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* FVM backward that allocates nothing: as tw_fvm_cost_bwd_*, without the
 * workspace argument. No counterpart in the reference; it is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid allocation). Its scratch is a file-scope device array
 * of tw_noalloc_scratch_bytes() bytes (16 MiB) that each device holds for the
 * life of the process; calls needing more (tw_fvm_workspace_bytes > that
 * size) return TW_ESIZE without launching. Every call on a device shares the
 * array: calls that overlap on one device (other streams, other host
 * threads) race. Calls no allocating routine. */
size_t tw_noalloc_scratch_bytes(void);
int tw_fvm_cost_bwd_noalloc_f32(const float* cost, const float* temporal, const float* R,
                                const float* grad_out, int B, int K, int T, int U, float gamma,
                                float* d_cost, hipStream_t stream);
int tw_fvm_cost_bwd_noalloc_f64(const double* cost, const double* temporal, const double* R,
                                const double* grad_out, int B, int K, int T, int U, double gamma,
                                double* d_cost, hipStream_t stream);

/* ------------------------------------------------------- pairwise cost --
 * A [P, R, D] against Bm [P, C, D] -> cost [P, R, C] with a TW_METRIC_*.
 * Replaces euclidean_cost / squared_euclidean_cost (jeanie/distances.py:15-38)
 * and the Gram + norm construction of udtw/_ops.py:164-165,
 * jeanie/_ops.py:162-167. Backward: d_cost -> dA [P,R,D], dB [P,C,D]
 * (cost is needed for the SQEUC / EUC masks; NULL allowed for RAW). */
int tw_pair_cost_fwd_f32(const float* A, const float* Bm, int P, int R, int C, int D, int metric,
                         float* cost, hipStream_t stream);
int tw_pair_cost_fwd_f64(const double* A, const double* Bm, int P, int R, int C, int D,
                         int metric, double* cost, hipStream_t stream);
int tw_pair_cost_bwd_f32(const float* A, const float* Bm, const float* cost, const float* d_cost,
                         int P, int R, int C, int D, int metric, float* dA, float* dB,
                         hipStream_t stream);
int tw_pair_cost_bwd_f64(const double* A, const double* Bm, const double* cost,
                         const double* d_cost, int P, int R, int C, int D, int metric,
                         double* dA, double* dB, hipStream_t stream);

/* RBF-style cost: A [P, R, D] against Bm [P, C, D] ->
 * cost[p, r, c] = sum_d 2 - 2 exp(-sigma (A[p,r,d] - Bm[p,c,d])^2), sigma > 0.
 * Replaces rbf_cost (jeanie/distances.py:41-51) and its autograd backward
 * without forming the [.., T, U, D] difference tensor. Backward:
 * d_cost [P, R, C] -> dA [P, R, D], dB [P, C, D]. */
int tw_rbf_cost_fwd_f32(const float* A, const float* Bm, int P, int R, int C, int D, float sigma,
                        float* cost, hipStream_t stream);
int tw_rbf_cost_fwd_f64(const double* A, const double* Bm, int P, int R, int C, int D,
                        double sigma, double* cost, hipStream_t stream);
int tw_rbf_cost_bwd_f32(const float* A, const float* Bm, const float* d_cost, int P, int R, int C,
                        int D, float sigma, float* dA, float* dB, hipStream_t stream);
int tw_rbf_cost_bwd_f64(const double* A, const double* Bm, const double* d_cost, int P, int R,
                        int C, int D, double sigma, double* dA, double* dB, hipStream_t stream);

/* --------------------------------------------------------- hard paths --
 * Optimal (gamma = 0) alignment path with bit-exact indices. Replaces the
 * numpy DP + backtrack of paths.py:85-127 (_optimal_3d / optimal_path).
 * cost: [B, K, T, U] float64 (K = 1 for a plain cost matrix); max_shift: the
 * viewpoint window; start_view: -1 or the only viewpoint allowed at (0,0).
 * Workspace r_ws: B*K*T*U doubles, back_ws: B*K*T*U ints. Output path:
 * [B, T+U-1, 3] ints (t, u, k) from (0,0) on, path_len: [B] entries used. */
int tw_optimal_path_f64(const double* cost, int B, int K, int T, int U, int max_shift,
                        int start_view, double* r_ws, int* back_ws, int* path, int* path_len,
                        hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TORCHWARP_HIP_H */
