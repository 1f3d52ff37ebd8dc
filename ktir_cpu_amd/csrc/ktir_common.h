// Shared device helpers for the KTIR gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/ktir_hip.h"

namespace ktir {

// Status plumbing shared by every translation unit (defined in ktir_runtime.hip).
int set_error(int code, const char* fmt, ...);
hipStream_t stream();
int* device_error_flag();   // device int: 1 = negative indirect index seen
int rmw_scratch_setup(int device);   // ktir_init: per-device scratch of the allocation-free RMW

#define KTIR_HIP_CHECK(expr)                                                        \
  do {                                                                              \
    hipError_t _e = (expr);                                                         \
    if (_e != hipSuccess)                                                           \
      return ::ktir::set_error(KTIR_E_HIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

// ---- element conversions -------------------------------------------------

__device__ __forceinline__ float round_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return __uint_as_float(u | 0x400000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}

__device__ __forceinline__ float round_f16(float x) { return (float)(_Float16)x; }

// x * y in f32, for a product that may be rounded to f16 next.  The
// compiler turns an f32 product narrowed to f16 into one mixed-precision
// fused multiply-add with a +0 addend (v_fma_mix), which gives +0 for a
// product of -0: the empty asm keeps the product a separate f32 result, so
// the narrowing sees -0 and keeps its sign.
__device__ __forceinline__ float mul_keep(float x, float y) {
  float r = __fmul_rn(x, y);
  __asm__ volatile("" : "+v"(r));
  return r;
}

// Round a float result to the KTIR dtype it is declared with.
__device__ __forceinline__ float round_to(float x, int dt) {
  if (dt == KTIR_F16) return round_f16(x);
  if (dt == KTIR_BF16) return round_bf16(x);
  return x;
}

__device__ __forceinline__ bool is_float_dt(int dt) { return dt <= KTIR_F32; }

__device__ __forceinline__ int elem_bytes(int dt) {
  switch (dt) {
    case KTIR_F16: case KTIR_BF16: case KTIR_I16: return 2;
    case KTIR_F32: case KTIR_I32: return 4;
    case KTIR_I64: return 8;
    default: return 1;
  }
}

// Device buffers are global memory: accesses through address-space-1
// pointers compile to global_* instructions (flat_* ones would make the
// compiler wait for LDS traffic too).
#define KTIR_G(T) __attribute__((address_space(1))) T

// Read one element of dtype dt at element offset off from ptr, as a 32-bit
// register value (float bits for float types, int32 for integer types).
__device__ __forceinline__ float load_elem(uint64_t ptr, int64_t off, int dt) {
  switch (dt) {
    case KTIR_F16: return (float)((const KTIR_G(_Float16)*)ptr)[off];
    case KTIR_BF16: return __uint_as_float(((uint32_t)((const KTIR_G(uint16_t)*)ptr)[off]) << 16);
    case KTIR_F32: return ((const KTIR_G(float)*)ptr)[off];
    case KTIR_I1: return __int_as_float(((const KTIR_G(uint8_t)*)ptr)[off] ? 1 : 0);
    case KTIR_I8: return __int_as_float((int)((const KTIR_G(int8_t)*)ptr)[off]);
    case KTIR_I16: return __int_as_float((int)((const KTIR_G(int16_t)*)ptr)[off]);
    case KTIR_I32: return __int_as_float(((const KTIR_G(int32_t)*)ptr)[off]);
    case KTIR_I64: return __int_as_float((int32_t)((const KTIR_G(int64_t)*)ptr)[off]);
  }
  return 0.f;
}

__device__ __forceinline__ void store_elem(uint64_t ptr, int64_t off, int dt, float v) {
  switch (dt) {
    case KTIR_F16: ((KTIR_G(_Float16)*)ptr)[off] = (_Float16)v; break;
    case KTIR_BF16: ((KTIR_G(uint16_t)*)ptr)[off] = (uint16_t)(__float_as_uint(round_bf16(v)) >> 16); break;
    case KTIR_F32: ((KTIR_G(float)*)ptr)[off] = v; break;
    case KTIR_I1: ((KTIR_G(uint8_t)*)ptr)[off] = __float_as_int(v) ? 1 : 0; break;
    case KTIR_I8: ((KTIR_G(int8_t)*)ptr)[off] = (int8_t)__float_as_int(v); break;
    case KTIR_I16: ((KTIR_G(int16_t)*)ptr)[off] = (int16_t)__float_as_int(v); break;
    case KTIR_I32: ((KTIR_G(int32_t)*)ptr)[off] = __float_as_int(v); break;
    case KTIR_I64: ((KTIR_G(int64_t)*)ptr)[off] = (int64_t)__float_as_int(v); break;
  }
}

// a wavefront-uniform value (loaded through a pointer or from LDS) into scalar registers
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t uni(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x), hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ int64_t lane_offset(const ktir_leaf_t& L, int64_t lane) {
  return L.lane_base ? ((const KTIR_G(int64_t)*)L.lane_base)[lane] : L.base + lane * L.lane_stride;
}

}  // namespace ktir
