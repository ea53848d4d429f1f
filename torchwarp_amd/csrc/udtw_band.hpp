// Banded uDTW / soft-DTW sweep on precomputed matrices (udtw_band.hip).
#pragma once

#include "udtw_sweep.hpp"

namespace tw {

// TORCHWARP_UDTW_BAND: 0 never takes the banded sweep, otherwise (-1, unset)
// it serves every band it can.
int band_mode();
// True when the banded sweep serves an N x M problem (N <= M) with this
// bandwidth: a band narrower than the grid that holds the end cell, at most
// 256 slots across, whose band-compressed planes fit in the N M elements of
// the caller's R / P.
bool band_path(int N, int M, double band);
// The banded forward (bwd false) or backward; R / P hold the band-compressed
// planes. C / Q (forward) and dC / dQ (backward) are [B, N, M], or with
// band_io in the band layout [B][N + M - 1][NS]; the penalty is on when Q is
// given, or with band_io when a.beta != 0.
// With band_io, the backward zeroes zero_c / zero_q ([B, N, M]) outside the
// band alongside the sweep (null: no zeroing).
template <typename T>
int band_sweep(bool bwd, const UdtwArgs<T>& a, int B, hipStream_t s, const char* what,
               bool band_io = false, T* zero_c = nullptr, T* zero_q = nullptr);
// The banded backward on the cost path: with a workspace of
// band_cost_workspace_elems elements, dC / dQ first in the band layout there
// (the sweep's other workgroups zeroing a.dC / a.dQ outside the band), then
// scattered into a.dC / a.dQ; with less, straight into a.dC / a.dQ.
size_t band_cost_workspace_elems(int B, int N, int M, double band);
template <typename T>
int band_cost_bwd(const UdtwArgs<T>& a, int B, hipStream_t s, const char* what, T* ws,
                  size_t ws_bytes);
// The banded forward on the cost path: the band's cells of C and Q first
// gathered into the band layout behind the band planes in R's buffer when
// it has the room (else the sweep reads the [B, N, M] planes).
template <typename T>
int band_cost_fwd(const UdtwArgs<T>& a, int B, hipStream_t s, const char* what);
// Elements of one pair's band-layout plane (N + M - 1 diagonals of NS slots).
size_t band_feat_plane_elems(int N, int M, double band);
// True when the feature path with F > 1 features runs banded: the banded
// sweep serves the problem and three band-layout planes fit in N M elements.
bool band_feat_path(int N, int M, int F, double band);
// The banded feature path: the band's cost and penalty built from X, Y and
// the variances of `a` into the band layout at `ws` (the forward's
// workspace, which the backward reads back), then the banded sweep. The
// backward rebuilds the cost plane when ws_fwd is null, takes dC / dQ from
// the banded sweep into `ws` and reduces them to dX, dY and a.dVX / a.dVY.
template <typename T>
int band_feat_fwd(const UdtwArgs<T>& a, const T* X, const T* Y, int F, int B, T* ws,
                  hipStream_t s, const char* what);
template <typename T>
int band_feat_bwd(const UdtwArgs<T>& a, const T* X, const T* Y, int F, int B, const T* ws_fwd,
                  T* ws, T* dX, T* dY, hipStream_t s, const char* what);

}  // namespace tw
