// Shared device/host definitions of the MI355X (gfx950) kernels behind include/kh.h.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kh.h"

namespace kh {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---- 16-bit conversions (round to nearest even, as the reference's bf16(x) / half(x)) ----
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);  // v_cvt_pk_bf16_f32: RNE, NaN stays NaN
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32: RNE under the default mode
}
template <int DT>
__device__ __forceinline__ uint16_t to16(float f) {
  return DT == KH_BF16 ? f32_to_bf16_bits(f) : f32_to_f16_bits(f);
}
// two f32 -> one dword of 16-bit values (a in the low half), round to nearest even; one instruction each
template <int DT>
__device__ __forceinline__ uint32_t pack16(float a, float b) {
  if constexpr (DT == KH_BF16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, (bf2){(__bf16)a, (__bf16)b});  // v_cvt_pk_bf16_f32
  } else {
    return __builtin_bit_cast(uint32_t, (f16x2){(_Float16)a, (_Float16)b});  // v_cvt_pk_f16_f32 / 2 cvt
  }
}
template <int DT>
__device__ __forceinline__ float from16(uint16_t h) {
  if (DT == KH_BF16) return __builtin_bit_cast(float, (uint32_t)h << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ float load_scale(const void* s, int s_dtype, size_t i) {
  if (s_dtype == KH_F16) return (float)((const _Float16*)s)[i];
  if (s_dtype == KH_BF16) return __builtin_bit_cast(float, (uint32_t)((const uint16_t*)s)[i] << 16);
  return ((const float*)s)[i];
}

// ---- epilogue math (engine/kernels/common.h:23-29) ----
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float gelu_tanh_f(float x) {
  const float k0 = 0.7978845608028654f, k1 = 0.044715f;
  return 0.5f * x * (1.0f + tanhf(k0 * (x + k1 * x * x * x)));
}
// Epilogue forms on the hardware exp2 / reciprocal (v_exp_f32, v_rcp_f32, ~1 ulp each):
//   gelu_tanh(x) = 0.5 x (1 + tanh(u)) = x / (1 + e^(-2u)),  u = k0 (x + k1 x^3)
//                = x / (1 + 2^(x (c0 + c1 x^2))),  c0 = -2 k0 log2(e), c1 = -2 k0 k1 log2(e)
//   silu(x) = x / (1 + e^(-x))
// Both saturate correctly: 2^(...) -> inf gives -0, 2^(...) -> 0 gives x.
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float gelu_fast(float x) {
  constexpr double k0 = 0.7978845608028654, k1 = 0.044715, log2e = 1.4426950408889634;
  constexpr float c0 = (float)(-2.0 * k0 * log2e), c1 = (float)(-2.0 * k0 * k1 * log2e);
  const float t = __builtin_fmaf(x * x, c1, c0);
  return x * rcp_fast(1.0f + __builtin_amdgcn_exp2f(t * x));
}
__device__ __forceinline__ float silu_fast(float x) { return x * rcp_fast(1.0f + __expf(-x)); }
__device__ __forceinline__ float sigmoid_fast(float x) { return rcp_fast(1.0f + __expf(-x)); }

// s_waitcnt immediate (gfx9 encoding): vmcnt <= vm, lgkmcnt <= lgkm, expcnt untouched.
__host__ __device__ constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8);
}

// Global loads the compiler does not track (inline asm): the caller orders them with explicit s_waitcnt and
// vm_ready(), which ties the destination registers to the wait so no use can be hoisted above it. Used where
// the compiler's own conservative vmcnt(0) (at loop back-edges) would cancel a multi-step prefetch.
__device__ __forceinline__ uint32_t vm_load_b32(const void* p) {
  uint32_t r;
  asm volatile("global_load_dword %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
__device__ __forceinline__ u32x2 vm_load_b64(const void* p) {
  u32x2 r;
  asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
__device__ __forceinline__ u32x4 vm_load_b128(const void* p) {
  u32x4 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
__device__ __forceinline__ uint32_t vm_load_u16(const void* p) {
  uint32_t r;
  asm volatile("global_load_ushort %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}
template <typename T>
__device__ __forceinline__ void vm_ready(T& r) {
  asm volatile("" : "+v"(r));
}

// Device-coherent 16-byte store / load (sc1: written through to / read from memory past L1 and L2, the
// encoding of the memory model's agent-scope atomic accesses), for data exchanged between workgroups that
// may run on different XCDs. Loads wait for themselves; stores are waited for by the caller.
__device__ __forceinline__ void st_coherent_b128(float* p, f32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
// eight device-coherent 16-byte loads at p + i * stride floats, completed before the statement ends
__device__ __forceinline__ void ld_coherent_8x_b128(const float* p, int stride, f32x4 (&r)[8]) {
  asm volatile(
      "global_load_dwordx4 %0, %8, off sc1\n\t"
      "global_load_dwordx4 %1, %9, off sc1\n\t"
      "global_load_dwordx4 %2, %10, off sc1\n\t"
      "global_load_dwordx4 %3, %11, off sc1\n\t"
      "global_load_dwordx4 %4, %12, off sc1\n\t"
      "global_load_dwordx4 %5, %13, off sc1\n\t"
      "global_load_dwordx4 %6, %14, off sc1\n\t"
      "global_load_dwordx4 %7, %15, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
      : "v"(p), "v"(p + stride), "v"(p + 2 * stride), "v"(p + 3 * stride), "v"(p + 4 * stride),
        "v"(p + 5 * stride), "v"(p + 6 * stride), "v"(p + 7 * stride)
      : "memory");
}

// Workgroup barrier that is also a compiler memory barrier, without the release fence of __syncthreads
// (which would also wait for LDS-direct loads still streaming in for later pipeline stages).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace kh
