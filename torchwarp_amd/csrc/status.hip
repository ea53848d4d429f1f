// Asynchronous status of the sweeps that hand rows between workgroups, and
// the host-set knobs of their bounded waits.
//
// Every device holds one status word in a file-scope device variable. A
// kernel whose bounded wait for another workgroup's boundary row runs out
// sets bit TW_STATUS_WAIT_GAVE_UP with a vector atomic OR and carries on
// (its outputs are then NaN, the sentinel the row was pre-filled with).
// tw_async_status() reads the word of the current device after a device
// synchronisation and reports it, like a sticky asynchronous error.
//
// The kernels take the word's device address as an argument: host code
// never passes the variable's name to a kernel (in host code it is a
// stand-in, not a device address). The address is looked up once per device
// with hipGetSymbolAddress, with that device current.

#include <atomic>
#include <mutex>

#include "tw_capi.hpp"
#include "../../include/torchwarp_hip.h"

static __device__ __align__(256) unsigned int g_status_word;

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_status_once[kMaxDevices];
unsigned int* g_status_ptr[kMaxDevices];

std::atomic<int> g_test_spins{0};
std::atomic<int> g_test_drop{0};
std::atomic<int> g_test_mw{-1};
}  // namespace

namespace tw {

unsigned int* status_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::call_once(g_status_once[dev], [dev] {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_status_word)) != hipSuccess) p = nullptr;
    g_status_ptr[dev] = static_cast<unsigned int*>(p);
  });
  return g_status_ptr[dev];
}

int wait_spins(int dflt) {
  const int s = g_test_spins.load(std::memory_order_relaxed);
  return s > 0 ? s : dflt;
}

int wait_drop_handoff() { return g_test_drop.load(std::memory_order_relaxed); }

int test_mw_mode() { return g_test_mw.load(std::memory_order_relaxed); }

}  // namespace tw

extern "C" {

int tw_async_status(int clear) {
  unsigned int* p = tw::status_word();
  if (!p) return tw::fail(TW_ELAUNCH, "tw_async_status: the status word has no device address");
  if (hipDeviceSynchronize() != hipSuccess)
    return tw::fail(TW_ELAUNCH, "tw_async_status: device synchronisation failed");
  unsigned int w = 0;
  if (hipMemcpy(&w, p, sizeof(w), hipMemcpyDeviceToHost) != hipSuccess)
    return tw::fail(TW_ELAUNCH, "tw_async_status: reading the status word failed");
  if (clear && w) {
    const unsigned int z = 0;
    if (hipMemcpy(p, &z, sizeof(z), hipMemcpyHostToDevice) != hipSuccess)
      return tw::fail(TW_ELAUNCH, "tw_async_status: clearing the status word failed");
  }
  if (w & TW_STATUS_WAIT_GAVE_UP)
    return tw::fail(TW_EWAIT,
                    "a uDTW sweep split over several workgroups gave up waiting for a "
                    "neighbouring workgroup's boundary row; the outputs of that call are NaN");
  return TW_OK;
}

void tw_test_set_mw(int mode) { g_test_mw.store(mode >= 0 && mode <= 2 ? mode : -1); }

void tw_test_set_wait(int spins, int drop_handoff) {
  g_test_spins.store(spins > 0 ? spins : 0, std::memory_order_relaxed);
  g_test_drop.store(drop_handoff ? 1 : 0, std::memory_order_relaxed);
}

}  // extern "C"
