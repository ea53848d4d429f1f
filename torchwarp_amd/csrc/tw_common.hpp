// Shared device helpers for the torchwarp gfx950 kernels.
//
// Conventions used by every DP kernel in this library:
//  * Values are carried in the base-2 "scaled" domain: Rh = R * log2(e) / gamma.
//    softmin_g(a, b, c) = gamma * ln2 * (mh - log2(2^(mh-ah) + 2^(mh-bh) + 2^(mh-ch)))
//    with mh = min(ah, bh, ch); every exponent is an exact difference of two
//    neighbouring scaled values, so one v_exp_f32 / v_log_f32 per term and no
//    extra multiply on the dependency chain.
//  * One row of the DP grid per (thread, k) slot; neighbouring rows of
//    neighbouring threads exchange their boundary value with a DPP wave shift,
//    and neighbouring waves through a small LDS mailbox behind an LDS-only
//    barrier (never a wait on outstanding global stores).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tw {

template <typename T> __device__ __forceinline__ T inf_v();
template <> __device__ __forceinline__ float inf_v<float>() { return __builtin_inff(); }
template <> __device__ __forceinline__ double inf_v<double>() { return __builtin_inf(); }

// 2^x, log2(x), 1/x. float uses the hardware transcendental unit (1 ulp);
// double uses the device library.
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ double ex2(double x) { return exp2(x); }
__device__ __forceinline__ float lg2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ double lg2(double x) { return log2(x); }
__device__ __forceinline__ float rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ double rcp(double x) { return 1.0 / x; }
__device__ __forceinline__ float sqrt_v(float x) { return __builtin_sqrtf(x); }
__device__ __forceinline__ double sqrt_v(double x) { return __builtin_sqrt(x); }

template <typename T>
__device__ __forceinline__ T min3(T a, T b, T c) {
  return fmin(a, fmin(b, c));
}

// ---- cross-lane moves (DPP wave shifts; a 64-bit value moves as two dwords)
// lane l receives lane l-1's value; lane 0 receives `edge`.
__device__ __forceinline__ float from_prev_lane(float v, float edge) {
  int r = __builtin_amdgcn_update_dpp(__float_as_int(edge), __float_as_int(v), 0x138, 0xf, 0xf,
                                      false);
  return __int_as_float(r);
}
__device__ __forceinline__ double from_prev_lane(double v, double edge) {
  long long b = __double_as_longlong(v), e = __double_as_longlong(edge);
  int lo = __builtin_amdgcn_update_dpp((int)e, (int)b, 0x138, 0xf, 0xf, false);
  int hi = __builtin_amdgcn_update_dpp((int)(e >> 32), (int)(b >> 32), 0x138, 0xf, 0xf, false);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
// lane l receives lane l+1's value; lane 63 receives `edge`.
__device__ __forceinline__ float from_next_lane(float v, float edge) {
  int r = __builtin_amdgcn_update_dpp(__float_as_int(edge), __float_as_int(v), 0x130, 0xf, 0xf,
                                      false);
  return __int_as_float(r);
}
__device__ __forceinline__ double from_next_lane(double v, double edge) {
  long long b = __double_as_longlong(v), e = __double_as_longlong(edge);
  int lo = __builtin_amdgcn_update_dpp((int)e, (int)b, 0x130, 0xf, 0xf, false);
  int hi = __builtin_amdgcn_update_dpp((int)(e >> 32), (int)(b >> 32), 0x130, 0xf, 0xf, false);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// DPP wave shift with an explicit value for the lane that has no source:
// lane l takes lane l-1 (prev) / l+1 (next); lane 0 (prev) / 63 (next) keeps `edge`.
__device__ __forceinline__ int dpp_prev_i(int v, int edge) {
  return __builtin_amdgcn_update_dpp(edge, v, 0x138, 0xf, 0xf, false);
}
__device__ __forceinline__ int dpp_next_i(int v, int edge) {
  return __builtin_amdgcn_update_dpp(edge, v, 0x130, 0xf, 0xf, false);
}

// Raw buffer access with a 32-bit byte offset split in a per-lane part
// (voffset) and a wave-uniform part (soffset). A voffset of kOob is out of
// range: loads return 0 and stores are dropped by the hardware range check.
constexpr int kOob = 0x80000000;
constexpr int kRsrcWord3 = 0x00020000;  // gfx9-family raw buffer, dword format
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

struct Buf {
  __amdgpu_buffer_rsrc_t r;
  // The size and flags words pass through an empty asm, so descriptors of
  // equal size never share registers: a shared word would have to be copied
  // into each descriptor's aligned register quad before every access.
  template <typename T>
  __device__ __forceinline__ void init(const T* p, long long n) {
    int bytes = (int)(n * (long long)sizeof(T)), flags = kRsrcWord3;
    asm volatile("" : "+s"(bytes), "+s"(flags));
    r = __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, bytes, flags);
  }
  __device__ __forceinline__ float ldf(int v, int s) const {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, v, s, 0));
  }
  __device__ __forceinline__ double ldd(int v, int s) const {
    const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(r, v, s, 0);
    return __longlong_as_double((long long)(((unsigned long long)w.y << 32) | w.x));
  }
  __device__ __forceinline__ void st(float x, int v, int s) const {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, v, s, 0);
  }
  __device__ __forceinline__ void st(double x, int v, int s) const {
    const unsigned long long u = (unsigned long long)__double_as_longlong(x);
    u32x2 w;
    w.x = (unsigned int)u;
    w.y = (unsigned int)(u >> 32);
    __builtin_amdgcn_raw_buffer_store_b64(w, r, v, s, 0);
  }
  template <typename T>
  __device__ __forceinline__ T ld(int v, int s) const;
};
template <> __device__ __forceinline__ float Buf::ld<float>(int v, int s) const { return ldf(v, s); }
template <> __device__ __forceinline__ double Buf::ld<double>(int v, int s) const { return ldd(v, s); }

// Two consecutive elements x0 (at byte offset v + s, s wave-uniform) and x1
// as one store, which must be aligned to its size (8 bytes for float, 16 for
// double).
template <typename T>
__device__ __forceinline__ void st_pair(const Buf& b, int v, T x0, T x1, int s = 0) {
  if constexpr (sizeof(T) == 4) {
    const u32x2 w = {__float_as_uint(x0), __float_as_uint(x1)};
    __builtin_amdgcn_raw_buffer_store_b64(w, b.r, v, s, 0);
  } else {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const unsigned long long u0 = (unsigned long long)__double_as_longlong(x0);
    const unsigned long long u1 = (unsigned long long)__double_as_longlong(x1);
    const u4 w = {(unsigned)u0, (unsigned)(u0 >> 32), (unsigned)u1, (unsigned)(u1 >> 32)};
    __builtin_amdgcn_raw_buffer_store_b128(w, b.r, v, s, 0);
  }
}

template <typename T>
__device__ __forceinline__ T shift_prev(T v, T edge);
template <>
__device__ __forceinline__ float shift_prev<float>(float v, float edge) {
  return __int_as_float(dpp_prev_i(__float_as_int(v), __float_as_int(edge)));
}
template <>
__device__ __forceinline__ double shift_prev<double>(double v, double edge) {
  long long b = __double_as_longlong(v), e = __double_as_longlong(edge);
  int lo = dpp_prev_i((int)b, (int)e);
  int hi = dpp_prev_i((int)(b >> 32), (int)(e >> 32));
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
// A wave-uniform value, taken from the first active lane (into a scalar register).
__device__ __forceinline__ float uniform(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ double uniform(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readfirstlane((int)b);
  const int hi = __builtin_amdgcn_readfirstlane((int)(b >> 32));
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// lane l takes lane l-1's value; lane 0 takes 0 (DPP bound_ctrl zero fill)
__device__ __forceinline__ float shift_prev0(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x138, 0xf, 0xf, true));
}
__device__ __forceinline__ double shift_prev0(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)b, 0x138, 0xf, 0xf, true);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), 0x138, 0xf, 0xf, true);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

template <typename T>
__device__ __forceinline__ T shift_next(T v, T edge);
template <>
__device__ __forceinline__ float shift_next<float>(float v, float edge) {
  return __int_as_float(dpp_next_i(__float_as_int(v), __float_as_int(edge)));
}
template <>
__device__ __forceinline__ double shift_next<double>(double v, double edge) {
  long long b = __double_as_longlong(v), e = __double_as_longlong(edge);
  int lo = dpp_next_i((int)b, (int)e);
  int hi = dpp_next_i((int)(b >> 32), (int)(e >> 32));
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// lane l takes lane l+1's value; lane 63 takes 0 (DPP bound_ctrl zero fill)
__device__ __forceinline__ float shift_next0(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x130, 0xf, 0xf, true));
}
__device__ __forceinline__ double shift_next0(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)b, 0x130, 0xf, 0xf, true);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), 0x130, 0xf, 0xf, true);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// Workgroup barrier that orders LDS only: outstanding global stores are not
// waited for (the DP stores its R/P history every diagonal).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Barrier for lagged wavefront pipelines: waits for every LDS operation of
// this wave except the most recent one (the mailbox store just issued), then
// joins the workgroup barrier. A mailbox record stored before barrier k is
// therefore complete at barrier k+1; readers only touch it after that
// barrier. LDS operations of a wave complete in order, so lgkmcnt <= 1
// leaves at most the newest LDS operation pending even when scalar-memory
// loads share the counter. The asm's memory clobber keeps the compiler from
// moving memory operations across it.
__device__ __forceinline__ void lag_barrier() {
  asm volatile("s_waitcnt lgkmcnt(1)\n\ts_barrier" ::: "memory");
}

// Number of cells on anti-diagonals 0..d-1 of an N x M grid (N <= M not required).
__host__ __device__ __forceinline__ long long diag_offset(int d, int N, int M) {
  // cells (i, d' - i) with max(0, d'-M+1) <= i <= min(N-1, d'), summed over d' < d
  long long s = 0;
  const int a = N < M ? N : M;   // length of the plateau
  const int b = N < M ? M : N;
  // ramp up: diagonals 0..a-2 have lengths 1..a-1
  int ramp = d < a - 1 ? d : a - 1;
  s += (long long)ramp * (ramp + 1) / 2;
  if (d <= a - 1) return s;
  // plateau: diagonals a-1 .. b-1 have length a
  int plat = (d < b ? d : b) - (a - 1);
  s += (long long)plat * a;
  if (d <= b) return s;
  // ramp down: diagonals b .. d-1 have lengths a-1, a-2, ...
  int down = d - b;
  s += (long long)down * (a - 1) - (long long)down * (down - 1) / 2;
  return s;
}

}  // namespace tw
