// Shared device/host helpers for the resihp HIP library (gfx950 / CDNA4).
//
// Storage types: fp32 (`float`) and bf16 (raw `uint16_t`, round-to-nearest-even
// on store, identical to torch's float->bfloat16 conversion for non-NaN values). Every kernel
// accumulates in fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include <type_traits>

#include "../../include/resihp_hip.h"

typedef uint16_t bf16_t;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8_t __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// scalar conversions
// ---------------------------------------------------------------------------
__device__ __host__ __forceinline__ float bf16_to_f32(bf16_t v) {
  uint32_t u = ((uint32_t)v) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// Round to nearest even with gfx950's v_cvt_pk_bf16_f32: the same bits as torch's
// float->bfloat16 conversion for every non-NaN value (NaNs stay NaNs).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

template <typename T> struct Storage;
template <> struct Storage<float> {
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
  __device__ __forceinline__ static float to_f32(float v) { return v; }
  __device__ __forceinline__ static float from_f32(float v) { return v; }
};
template <> struct Storage<bf16_t> {
  __device__ __forceinline__ static float load(const bf16_t* p) { return bf16_to_f32(*p); }
  __device__ __forceinline__ static void store(bf16_t* p, float v) { *p = f32_to_bf16(v); }
  __device__ __forceinline__ static float to_f32(bf16_t v) { return bf16_to_f32(v); }
  __device__ __forceinline__ static bf16_t from_f32(float v) { return f32_to_bf16(v); }
};

template <typename T> __device__ __forceinline__ float ld_f32(const T* p) { return Storage<T>::load(p); }
template <typename T> __device__ __forceinline__ void st_f32(T* p, float v) { Storage<T>::store(p, v); }

// ---------------------------------------------------------------------------
// GELU (exact, erf form) and its derivative.  HIP's own erff/expf are used.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float gelu_f(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}
__device__ __forceinline__ float gelu_grad_f(float x) {
  const float cdf = 0.5f * (1.0f + erff(x * 0.70710678118654752440f));
  const float pdf = expf(-0.5f * x * x) * 0.39894228040143267794f;
  return cdf + x * pdf;
}

// GELU for results that are rounded to bf16 (the bf16 GEMM epilogues and elementwise
// kernels).  The normal CDF uses Abramowitz & Stegun, Handbook of Mathematical Functions
// (1964), formula 7.1.26: for z >= 0, erf(z) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5)
// exp(-z^2) with t = 1/(1 + p z), |error| <= 1.5e-7 -- three orders of magnitude below bf16
// resolution.  With z = |x|/sqrt(2), exp(-z^2) = exp(-x^2/2) is also the Gaussian density's
// factor, so the value and the derivative share one exp and one reciprocal (hardware
// v_exp_f32 / v_rcp_f32) instead of an erf and an exp each.
struct GeluParts {
  float cdf;  // Phi(x)
  float pdf;  // phi(x)
};
__device__ __forceinline__ GeluParts gelu_parts_fast(float x) {
  constexpr float kP = 0.3275911f, kA1 = 0.254829592f, kA2 = -0.284496736f, kA3 = 1.421413741f,
                  kA4 = -1.453152027f, kA5 = 1.061405429f;
  const float ax = fabsf(x);
  const float e = __builtin_amdgcn_exp2f(x * x * (-0.5f * 1.4426950408889634074f));  // exp(-x^2/2)
  const float t = __builtin_amdgcn_rcpf(fmaf(kP * 0.70710678118654752440f, ax, 1.0f));
  const float poly = t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, kA5, kA4), kA3), kA2), kA1);
  const float tail = 0.5f * poly * e;  // = Phi(-|x|)
  return {x >= 0.f ? 1.0f - tail : tail, e * 0.39894228040143267794f};
}
__device__ __forceinline__ float gelu_fast_f(float x) { return x * gelu_parts_fast(x).cdf; }
__device__ __forceinline__ float gelu_grad_fast_f(float x) {
  const GeluParts g = gelu_parts_fast(x);
  return g.cdf + x * g.pdf;
}

// ---------------------------------------------------------------------------
// wavefront (64-lane) reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Block-wide sum for a 1-D block of `nthreads` (multiple of 64, <= 1024).
// `scratch` must hold nthreads/64 floats.  Result is broadcast to all threads.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float r = 0.f;
  for (int i = 0; i < nw; ++i) r += scratch[i];
  return r;
}
__device__ __forceinline__ float block_max(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float r = -INFINITY;
  for (int i = 0; i < nw; ++i) r = fmaxf(r, scratch[i]);
  return r;
}

// ---------------------------------------------------------------------------
// direct global->LDS loads (gfx950 global_load_lds_dwordx4)
// ---------------------------------------------------------------------------
// Direct global->LDS load of 16 bytes per lane: lane l of the wave writes LDS bytes
// lds_base + 16*l .. +15 (lds_base wave-uniform).  Issued through inline asm on purpose: the
// compiler cannot see that the asynchronous LDS write never aliases the stages being read, and
// with the builtin it waits for every outstanding load before each LDS read, serialising the
// pipeline.  Completion is tracked explicitly with wait_vm_le (these loads count in vmcnt).
// The LDS destination is a wave-uniform 32-bit LDS byte address: a generic-to-LDS pointer
// conversion per load would cost a null check in scalar instructions.
__device__ __forceinline__ void dma16(const bf16_t* src, uint32_t lds_dst) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_dst))
      : "memory", "m0");
}

// The same load in saddr form: lane l fetches the 16 bytes at sbase + voff (sbase wave-uniform,
// held in SGPRs; voff a 32-bit per-lane byte offset), so a stage of loads needs one 32-bit
// offset register per load instead of a 64-bit pointer.
// (the LDS destination is a wave-uniform byte address, as for dma16; s_nop 4: five wait states, so an
// SGPR base written by a VALU op (readfirstlane) just before this statement is settled when the
// load reads it, the M0 write needs one)
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_dst) {
  // (readfirstlane returns a signed int: widen through uint32_t, never by sign extension)
  const uint64_t b = (uint64_t)(uintptr_t)sbase;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
  const uint32_t lds = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_dst);
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 4\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(sb), "s"(lds)
      : "memory", "m0");
}

// The 4-byte form: lane l fetches the dword at sbase + voff into LDS byte lds_dst + 4*l.
__device__ __forceinline__ void dma4s(const void* sbase, uint32_t voff, uint32_t lds_dst) {
  const uint64_t b = (uint64_t)(uintptr_t)sbase;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
  const uint32_t lds = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_dst);
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 4\n\t"
      "global_load_lds_dword %0, %1"
      :
      : "v"(voff), "s"(sb), "s"(lds)
      : "memory", "m0");
}

// wait until at most N of this thread's vector-memory loads (direct-to-LDS ones included) are
// outstanding; they complete in issue order
template <int N>
__device__ __forceinline__ void wait_vm_le() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate out of range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}

// ---------------------------------------------------------------------------
// host-side error plumbing (defined in runtime.hip)
// ---------------------------------------------------------------------------
int rh_set_error(int code, const char* fmt, ...);
int rh_check_launch(const char* what);

#define RH_REQUIRE(cond, ...)                                   \
  do {                                                          \
    if (!(cond)) return rh_set_error(RH_ERR_INVALID, __VA_ARGS__); \
  } while (0)

static inline int64_t rh_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
static inline bool rh_aligned(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0;
}
