// FVM backward without any allocation by the caller or the library: its
// scratch (the temporal-cost adjoint [B, T*U] and, for sequences longer than
// one workgroup holds, the soft-DTW hand-off records) lives in a file-scope
// device array of kNoAllocScratchBytes, instead of the workspace argument of
// tw_fvm_cost_bwd_*.
//
// Each device holds its own copy of the array for the life of the process.
// In host code the array's name is only a host-side stand-in, so its device
// address is looked up once per device, with that device current, by
// hipGetSymbolAddress, and that address (never the name) is what the
// kernels receive. Every call on a device shares the array and leaves its
// contents behind; everything the kernels need cleared (the hand-off
// sentinels) is cleared by a fill kernel of the call itself. Calls that
// overlap on one device (on different streams, or from several host
// threads) race on the array.

#include <mutex>

#include "tw_capi.hpp"
#include "../../include/torchwarp_hip.h"

namespace {
constexpr size_t kNoAllocScratchBytes = 16u << 20;   // 16 MiB per device
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
int g_scratch_err[kMaxDevices];
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace tw {

template <typename T>
int fvm_bwd(const T* C, const T* tmp, const T* R, const T* gout, int B, int K, int Tn, int Un,
            double gamma, T* dC, T* ws, size_t ws_bytes, hipStream_t s, const char* what);
size_t fvm_workspace_bytes(int B, int Tn, int Un, int es);

// The device address of this device's scratch array (looked up on the first
// call per device), or null with the last error set.
static void* scratch_address(const char* what) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(TW_ELAUNCH, "%s: no current HIP device", what);
    return nullptr;
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_err[dev] = (int)e;
    g_scratch_ptr[dev] = e == hipSuccess ? p : nullptr;
  });
  if (!g_scratch_ptr[dev]) {
    fail(TW_ELAUNCH, "%s: hipGetSymbolAddress of the scratch array failed (%s)", what,
         hipGetErrorString((hipError_t)g_scratch_err[dev]));
    return nullptr;
  }
  return g_scratch_ptr[dev];
}

template <typename T>
static int fvm_bwd_noalloc(const T* C, const T* tmp, const T* R, const T* gout, int B, int K,
                           int Tn, int Un, double gamma, T* dC, hipStream_t s,
                           const char* what) {
  if (B < 0 || K <= 0 || Tn <= 0 || Un <= 0 || !(gamma > 0))
    return fail(TW_EINVAL, "%s: bad arguments", what);
  if (B == 0) return TW_OK;
  const size_t need = fvm_workspace_bytes(B, Tn, Un, (int)sizeof(T));
  if (need > kNoAllocScratchBytes)
    return fail(TW_ESIZE,
                "%s: this call needs %zu bytes of scratch; the entry point without allocation "
                "holds %zu (B*T*U elements plus, past one workgroup's rows, hand-off records): "
                "use tw_fvm_cost_bwd with a workspace",
                what, need, kNoAllocScratchBytes);
  void* p = scratch_address(what);
  if (!p) return TW_ELAUNCH;
  return fvm_bwd<T>(C, tmp, R, gout, B, K, Tn, Un, gamma, dC, static_cast<T*>(p),
                    kNoAllocScratchBytes, s, what);
}

}  // namespace tw

extern "C" {

size_t tw_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int tw_fvm_cost_bwd_noalloc_f32(const float* cost, const float* temporal, const float* R,
                                const float* grad_out, int B, int K, int T, int U, float gamma,
                                float* d_cost, hipStream_t stream) {
  return tw::fvm_bwd_noalloc<float>(cost, temporal, R, grad_out, B, K, T, U, gamma, d_cost,
                                    stream, "tw_fvm_cost_bwd_noalloc_f32");
}

int tw_fvm_cost_bwd_noalloc_f64(const double* cost, const double* temporal, const double* R,
                                const double* grad_out, int B, int K, int T, int U, double gamma,
                                double* d_cost, hipStream_t stream) {
  return tw::fvm_bwd_noalloc<double>(cost, temporal, R, grad_out, B, K, T, U, gamma, d_cost,
                                     stream, "tw_fvm_cost_bwd_noalloc_f64");
}

}  // extern "C"
