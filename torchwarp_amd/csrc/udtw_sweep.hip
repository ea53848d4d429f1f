// uDTW sweep launchers: one object per (type, direction, cost source), built
// from this file with TW_SWEEP_T, TW_SWEEP_BWD and TW_SWEEP_SRC defined, so
// the kernel instantiations compile in parallel.
#define TW_SWEEP_INSTANTIATE
#include "udtw_sweep.hpp"

#if !defined(TW_SWEEP_T) || !defined(TW_SWEEP_BWD) || !defined(TW_SWEEP_SRC)
#error "compile with -DTW_SWEEP_T=float|double -DTW_SWEEP_BWD=0|1 -DTW_SWEEP_SRC=0|1|2"
#endif

namespace tw {

template int launch_sweep<TW_SWEEP_T, TW_SWEEP_SRC, (bool)TW_SWEEP_BWD>(
    bool, const UdtwArgs<TW_SWEEP_T>&, int, hipStream_t, const char*);

}  // namespace tw
