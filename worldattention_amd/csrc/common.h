// Shared device helpers for the gfx950 HSA/HKV kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/worldattention_amd.h"

typedef __bf16 bf16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define WA_LOG2E 1.4426950408889634f
#define WA_LN2 0.6931471805599453f

// Raw buffer descriptor word 3 for the gfx9 family (32-bit data format; untyped loads ignore it
// otherwise).
#define WA_BUF_DWORD3 0x00020000

// ---------------------------------------------------------------------------------------------
// Host-side error reporting (wa_last_error): one thread-local message per calling thread.
// ---------------------------------------------------------------------------------------------
void wa_set_error(const char* fmt, ...);
int wa_fail(int code, const char* fmt, ...);

#define WA_CHECK_ARG(cond, ...)                                  \
  do {                                                           \
    if (!(cond)) return wa_fail(WA_ERR_ARG, __VA_ARGS__);        \
  } while (0)

#define WA_CHECK_HIP(expr)                                                        \
  do {                                                                            \
    hipError_t _e = (expr);                                                       \
    if (_e != hipSuccess)                                                         \
      return wa_fail((int)_e, "%s failed: %s", #expr, hipGetErrorString(_e));     \
  } while (0)

// Returns the launch status of the most recent kernel launch as a wa status code.
int wa_launch_status(const char* what);

static inline bool wa_aligned16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }

// ---------------------------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float wa_bf16_round(float x) { return (float)(bf16_t)x; }

// The linear heads' feature map phi(x) = elu(x) + 1 (one definition for every kernel that forms it,
// so that they agree bit for bit).
__device__ __forceinline__ float elu1f(float x) { return x > 0.f ? x + 1.f : __expf(x); }

// Single-rounding fp32 operations that the compiler may not fuse with a neighbouring multiply or
// add: HIP's __fadd_rn / __fmul_rn are plain operators, which the default -ffp-contract=fast turns
// into fused multiply-adds (one rounding instead of two). Used where results must round as the
// reference's separate torch operations do.
__device__ __forceinline__ float wa_add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float wa_sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}
__device__ __forceinline__ float wa_mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float wa_div_rn(float a, float b) {
#pragma clang fp contract(off)
  return a / b;
}

__device__ __forceinline__ float wa_load_f(const void* p, int64_t i, int dtype) {
  return dtype == WA_BF16 ? (float)((const bf16_t*)p)[i] : ((const float*)p)[i];
}

__device__ __forceinline__ void wa_store_f(void* p, int64_t i, float x, int dtype) {
  if (dtype == WA_BF16) ((bf16_t*)p)[i] = (bf16_t)x;
  else ((float*)p)[i] = x;
}

template <typename T>
__device__ __forceinline__ T wa_shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, 64);
}

__device__ __forceinline__ float wa_wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ float wa_wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ double wa_wave_sum_d(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ f32x16 wa_mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float wa_sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Workgroups are dispatched round-robin over the 8 XCDs (id % 8). Remap so that each XCD gets a
// contiguous range of work items: neighbouring items (same head, adjacent blocks) then share the
// XCD's L2. Bijective on [0, n).
__device__ __forceinline__ int wa_xcd_remap(int id, int n) {
  const int per = (n + 7) / 8;
  int tall = n % 8;
  if (tall == 0) tall = 8;
  const int xcd = id % 8, local = id / 8;
  return xcd < tall ? xcd * per + local : tall * per + (xcd - tall) * (per - 1) + local;
}

// Order-preserving float -> uint32 key (larger float -> larger key); NaN sorts above +inf.
__device__ __forceinline__ uint32_t wa_float_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
