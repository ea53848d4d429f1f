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
// The banded forward (bwd false) or backward on the cost path; R / P hold the
// band-compressed planes.
template <typename T>
int band_sweep(bool bwd, const UdtwArgs<T>& a, int B, hipStream_t s, const char* what);

}  // namespace tw
