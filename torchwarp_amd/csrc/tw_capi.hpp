// Host-side helpers shared by the C-ABI entry points: error reporting and
// launch checks. The library never allocates device memory; callers pass
// every output and workspace buffer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#define TW_OK 0
#define TW_EINVAL 1
#define TW_ELAUNCH 2
#define TW_ESIZE 3
#define TW_EWAIT 4
#define TW_STATUS_WAIT_GAVE_UP 1u

namespace tw {

// Formats the thread-local last-error message and returns `code`.
int fail(int code, const char* fmt, ...);
// Checks hipGetLastError after a launch; returns TW_OK or TW_ELAUNCH.
int check_launch(const char* what);
// Device limits of the current device, queried once per device.
int max_lds_bytes();
// Frequency of the device's real-time counter (s_memrealtime), kHz.
double realtime_khz();
// Compute units of the current device.
int num_cus();
// Device address of the current device's asynchronous status word (bit
// TW_STATUS_WAIT_GAVE_UP: a bounded cross-workgroup wait ran out), or null.
unsigned int* status_word();
// Poll limit of a cross-workgroup wait (dflt unless a test set one) and the
// test hook that keeps boundary rows from being handed over.
int wait_spins(int dflt);
int wait_drop_handoff();
// Several-workgroups-per-pair mode a test set (tw_test_set_mw), or -1.
int test_mw_mode();

}  // namespace tw
