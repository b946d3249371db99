// Shared helpers for the gfx950 kernels: element types, 16-byte vector access, wave reductions,
// and the thread-local error state behind edgerag_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>

#include <cstdint>

#include "../../include/edgerag_amd.h"

namespace edgerag {

// ---- error state (capi.cpp) -----------------------------------------------------------------
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Converts a pending launch error into EDGERAG_EHIP; returns EDGERAG_OK otherwise.
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kWave = 64;

// ---- element types ---------------------------------------------------------------------------
using f16 = __half;
using bf16 = __hip_bfloat16;

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<f16>(f16 v) { return __half2float(v); }
template <> __device__ __forceinline__ float to_f32<bf16>(bf16 v) { return __bfloat162float(v); }

// Round-to-nearest-even conversions, matching torch's Tensor.to(dtype).
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return __float2half_rn(v); }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return __float2bfloat16(v); }

template <typename T> struct Same { static constexpr bool value = false; };

// Compiler-only fence: keeps the loads issued above it from being sunk below it (next to their
// first use), which would serialise memory latency with the compute they are meant to overlap.
// The memory clobber stops IR-level code motion; the scheduling barrier stops the machine
// scheduler, which otherwise moves each load next to its first use to save registers.
__device__ __forceinline__ void issue_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// v, made opaque to the optimiser at this point of the program (a wave-uniform value kept in
// SGPRs): computations on it cannot be hoisted above the statement that uses pin_s.
template <class V>
__device__ __forceinline__ V pin_s(V v) {
  asm volatile("" : "+s"(v));
  return v;
}

// p as a global-memory pointer: loads through it are global_load instructions (a pointer that
// went through pin_s is a generic one, whose loads would be flat loads, which also count against
// lgkmcnt and make every later wait a full one).
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* as_global(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}

// A plain 16-byte register payload. Loads/stores through it compile to dwordx4 accesses.
struct alignas(16) Vec16 {
  uint32_t w[4];
};

template <typename T>
__device__ __forceinline__ Vec16 load16(const T* p) {
  return *reinterpret_cast<const Vec16*>(p);
}

// A 16-byte load marked non-temporal (its cache lines are the first to be evicted): for data a
// launch reads exactly once, so that streaming it does not push reused lines out of L2.
template <typename T>
__device__ __forceinline__ Vec16 load16_stream(const T* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return Vec16{{v.x, v.y, v.z, v.w}};
}

template <typename T>
__device__ __forceinline__ void store16(T* p, const Vec16& v) {
  *reinterpret_cast<Vec16*>(p) = v;
}

// Element i of a 16-byte payload viewed as an array of T, widened to fp32.
template <typename T>
__device__ __forceinline__ float vec_elem(const Vec16& v, int i) {
  const T* e = reinterpret_cast<const T*>(&v);
  return to_f32<T>(e[i]);
}

// ---- wave reductions (64 lanes) --------------------------------------------------------------
// Butterfly over lane-index bits [lo_bit, hi_bit): after the call every lane holds the reduction
// over the 2^(hi-lo) lanes that differ from it only in those bits.
template <int LO_BIT, int HI_BIT>
__device__ __forceinline__ float xor_sum(float v) {
#pragma unroll
  for (int b = LO_BIT; b < HI_BIT; ++b) v += __shfl_xor(v, 1 << b, kWave);
  return v;
}
template <int LO_BIT, int HI_BIT>
__device__ __forceinline__ float xor_max(float v) {
#pragma unroll
  for (int b = LO_BIT; b < HI_BIT; ++b) v = fmaxf(v, __shfl_xor(v, 1 << b, kWave));
  return v;
}

// SwiGLU's gate activation rounded as the reference's fp16 F.silu: fp16(g / (1 + exp(-g))), with
// the quotient and exp in fp32 (layers.py:341).
__device__ __forceinline__ float silu_rounded_f16(float g) {
  return __half2float(__float2half_rn(g / (1.f + expf(-g))));
}

constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v / 2); }

// log2 of a power of two, -1 for anything else.
inline int log2_exact(int v) {
  if (v <= 0) return -1;
  int s = 0;
  while ((1 << s) < v) ++s;
  return (1 << s) == v ? s : -1;
}

}  // namespace edgerag
