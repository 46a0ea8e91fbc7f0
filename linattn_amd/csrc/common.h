// Shared device/host helpers for the gfx950 sparse-attention kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "linattn_hip.h"

namespace la {

// ---------------------------------------------------------------- errors ----
void set_error(const char *fmt, ...);
int fail(int code, const char *fmt, ...);
// compute units of the current device (cached per thread and device)
int num_cus();
// Status bits of prefill.hip's kernels on the current device (read after the
// caller synchronised), optionally cleared.
int prefill_status(uint32_t *bits, bool clear, hipStream_t st);
// The same for indexer.hip's kernels.
int indexer_status(uint32_t *bits, bool clear, hipStream_t st);

#define LA_REQUIRE(cond, ...)                               \
  do {                                                      \
    if (!(cond)) return ::la::fail(LA_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define LA_HIP(expr)                                                               \
  do {                                                                             \
    hipError_t _e = (expr);                                                        \
    if (_e != hipSuccess)                                                          \
      return ::la::fail(LA_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

// Check the launch that was just enqueued.
#define LA_LAUNCHED()                                                                \
  do {                                                                               \
    hipError_t _e = hipGetLastError();                                               \
    if (_e != hipSuccess)                                                            \
      return ::la::fail(LA_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(_e)); \
  } while (0)

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
inline int ilog2(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}

// ----------------------------------------------------- LDS and barriers ----
typedef __attribute__((address_space(3))) void lds_void_t;

// 16 bytes per lane from global memory straight into LDS (gfx950
// global_load_lds_dwordx4): lane i writes dst + 16 i, dst wave-uniform (M0).
// Issued as inline assembly so that the compiler neither waits for it (it
// treated the address registers as pending results) nor reorders it across
// the barriers; it counts in vmcnt, and the caller waits (wait_vmcnt) and
// synchronises the workgroup before reading the data.
__device__ __forceinline__ void dma16(const void *src, void *dst) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t *)dst);
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// Wait until at most N vector memory operations of this wave are
// outstanding (N < 64; the other counters are not waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier for LDS traffic only: this wave's LDS operations are
// complete, then s_barrier.  Unlike __syncthreads it does not wait for global
// memory operations (so loads issued earlier stay in flight).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// An empty use of a register value: the compiler waits here for a load of it
// still in flight.  Placed after the waits of inline-asm loads, it stops the
// compiler from waiting for its own earlier loads later (by then its counts
// would also cover the asm loads issued after them).
template <class T>
__device__ __forceinline__ void settle(const T &x) {
  asm volatile("" ::"v"(x));
}

// Wave-uniform 32-bit read through the scalar cache, waited for at once
// (lgkmcnt(0): LDS operations in flight are waited for as well).  For reads
// the compiler would otherwise issue as vector loads: after inline assembly
// that may write memory it no longer proves a pointer unclobbered, and a
// vector load's wait also waits for every load issued before it.
__device__ __forceinline__ int32_t sload_i32(const int32_t *p) {
  int32_t v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}

// --------------------------------------------------------- element loads ----
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 bits (finite inputs; NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// OCP e4m3fn byte pair -> two fp32 (gfx950 v_cvt_pk_f32_fp8 decodes OCP e4m3).
// HI selects bytes 2..3 of the word, otherwise bytes 0..1.
template <bool HI>
__device__ __forceinline__ float2 fp8x2_to_f32(uint32_t word) {
  auto r = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, HI);
  return make_float2(r[0], r[1]);
}

// Scalar load of one element of dtype `dt` as double (exact for f32/bf16/f16).
__device__ __forceinline__ double load_as_f64(const void *base, int64_t idx, int dt) {
  switch (dt) {
    case LA_F32:
      return (double)((const float *)base)[idx];
    case LA_BF16:
      return (double)bf16_bits_to_f32(((const uint16_t *)base)[idx]);
    case LA_F16:
      return (double)__half2float(((const __half *)base)[idx]);
    case LA_F64:
      return ((const double *)base)[idx];
    default:
      return 0.0;
  }
}
__device__ __forceinline__ float load_as_f32(const void *base, int64_t idx, int dt) {
  switch (dt) {
    case LA_F32:
      return ((const float *)base)[idx];
    case LA_BF16:
      return bf16_bits_to_f32(((const uint16_t *)base)[idx]);
    case LA_F16:
      return __half2float(((const __half *)base)[idx]);
    case LA_F64:
      return (float)((const double *)base)[idx];
    default:
      return 0.0f;
  }
}
__device__ __forceinline__ void store_from_f32(void *base, int64_t idx, int dt, float x) {
  if (dt == LA_BF16)
    ((uint16_t *)base)[idx] = f32_to_bf16_bits(x);
  else if (dt == LA_F16)
    ((__half *)base)[idx] = __float2half(x);
  else
    ((float *)base)[idx] = x;
}

// -------------------------------------------------------- ordering keys ----
// Monotone map fp64 -> uint64: a > b (as reals) <=> key(a) > key(b).  -0 and +0
// map to the same key so that equal scores tie exactly.
__device__ __forceinline__ uint64_t ord_key(double x) {
  if (x == 0.0) x = 0.0;
  uint64_t u = (uint64_t)__double_as_longlong(x);
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}
__device__ __forceinline__ double key_to_double(uint64_t u) {
  uint64_t b = (u >> 63) ? (u & 0x7fffffffffffffffull) : ~u;
  return __longlong_as_double((long long)b);
}
constexpr uint64_t KEY_FORCED = 0xffffffffffffffffull;  // above every finite score

// fl(acc + fl(a * b)): two roundings, never fused into an fma.
__device__ __forceinline__ double add_product(double acc, double a, double b) {
#pragma clang fp contract(off)
  return acc + a * b;
}

// ------------------------------------------------------------ wave utils ----
__device__ __forceinline__ float wave_xor_f32(float x, int m) { return __shfl_xor(x, m, 64); }

// DPP lane permutation within rows of 16 lanes (no LDS traffic).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// The values of lane l and its partner l ^ 16 (pair16) or l ^ 32 (pair32), in
// lane order: .x from the lower lane, .y from the upper one, the same pair on
// both partners.  gfx950 v_permlane16_swap / v_permlane32_swap are VALU lane
// swaps, so these cost no LDS round trip (unlike __shfl_xor's ds_bpermute).
__device__ __forceinline__ float2 pair16(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 pair32(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair16_sum(float x) { const float2 p = pair16(x); return p.x + p.y; }
__device__ __forceinline__ float pair32_sum(float x) { const float2 p = pair32(x); return p.x + p.y; }
__device__ __forceinline__ float pair16_max(float x) { const float2 p = pair16(x); return fmaxf(p.x, p.y); }
__device__ __forceinline__ float pair32_max(float x) { const float2 p = pair32(x); return fmaxf(p.x, p.y); }

// Sum over aligned groups of N lanes; every lane of a group gets the same sum
// (each step adds a value to its partner's, and fp addition is commutative).
// quad_perm [1,0,3,2] and [2,3,0,1], then row_half_mirror and row_mirror, then
// the 16- and 32-lane swaps.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp_f32<0xB1>(x);
  if constexpr (N >= 4) x += dpp_f32<0x4E>(x);
  if constexpr (N >= 8) x += dpp_f32<0x141>(x);
  if constexpr (N >= 16) x += dpp_f32<0x140>(x);
  if constexpr (N >= 32) x = pair16_sum(x);
  if constexpr (N >= 64) x = pair32_sum(x);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace la
