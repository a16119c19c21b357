// Shared device/host helpers for the gfx950 (MI355X) kernels of the Qwen3-VL
// operator layer. Everything here is CDNA4-specific: wave64, MFMA bf16
// builtins, 16-byte vector memory ops.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "q3vl.h"

typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define Q3_WAVE 64

// ------------------------------------------------------------------ host-side checks
// Every entry point validates its arguments on the host and returns a negative
// q3_status before touching the device; launch failures come back as the
// (positive) hipError_t.
#define Q3_REQUIRE(cond, code) \
  do {                         \
    if (!(cond)) return (code); \
  } while (0)

#define Q3_LAUNCH_CHECK()                      \
  do {                                         \
    hipError_t e__ = hipGetLastError();        \
    if (e__ != hipSuccess) return (int)e__;    \
  } while (0)

static inline bool q3_aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
static inline int64_t q3_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------------ conversions
__device__ __forceinline__ float bf2f(bf16 x) { return static_cast<float>(x); }
// Round-to-nearest-even float -> bf16 (gfx950 has a native conversion).
__device__ __forceinline__ bf16 f2bf(float x) { return static_cast<bf16>(x); }

template <typename T>
__device__ __forceinline__ float to_f(T x);
template <>
__device__ __forceinline__ float to_f<float>(float x) { return x; }
template <>
__device__ __forceinline__ float to_f<bf16>(bf16 x) { return bf2f(x); }

// gelu with the tanh approximation: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
__device__ __forceinline__ float gelu_tanh_f(float a) {
  const float k0 = 0.7978845608028654f;
  const float inner = k0 * (a + 0.044715f * a * a * a);
  return 0.5f * a * (1.0f + tanhf(inner));
}

template <typename T>
__device__ __forceinline__ T from_f(float x);
template <>
__device__ __forceinline__ float from_f<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 from_f<bf16>(float x) { return f2bf(x); }

// 16-byte vector of T: 8 bf16 or 4 fp32.
template <typename T>
struct Vec16;
template <>
struct Vec16<bf16> {
  static constexpr int N = 8;
  typedef bf16x8 type;
};
template <>
struct Vec16<float> {
  static constexpr int N = 4;
  typedef floatx4 type;
};

// ------------------------------------------------------------------ wave reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// gelu_tanh of the fused GEMM epilogue (vision fc1, patch mergers): tanh(u) =
// 1 - 2 / (exp(2u) + 1) with the fast exponential and the hardware reciprocal
// (absolute error ~1e-7 against tanhf, far below the bf16 rounding that
// follows), instead of the libm tanhf the op-level kernel keeps. exp(2u)
// overflowing to inf gives 1, underflowing to 0 gives -1.
__device__ __forceinline__ float gelu_tanh_fast(float a) {
  const float k0 = 0.7978845608028654f;
  const float inner = k0 * (a + 0.044715f * a * a * a);
  const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(__expf(2.0f * inner) + 1.0f);
  return 0.5f * a * (1.0f + t);
}

// silu(g) * u of the fused SwiGLU epilogues (GEMM tiles, decode GEMVs), in
// fp32 before the one rounding: the hardware reciprocal (v_rcp_f32, ~1 ulp)
// instead of an IEEE division, which cost ~1.8 us per wave of 256x256 tiles.
// Ordered g * rcp * u so that a reciprocal of 0 (exp overflow) gives a signed
// zero rather than inf * 0.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// Reduction over aligned groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = G / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = G / 2; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ------------------------------------------------------------------ MFMA wrappers
// D(32x32, fp32) += A(32x16, bf16) * B(16x32, bf16).
// Lane l supplies A[l%32][8*(l/32)+t] and B[8*(l/32)+t][l%32], t = 0..7 (the
// k index assignment is the same for A and B, so any consistent permutation of
// k between the two operands yields the same product).
// Accumulator register r of lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32].
__device__ __forceinline__ floatx16 mfma32x32x16(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// D(16x16, fp32) += A(16x32) * B(32x16): lane l supplies A[l%16][8*(l/16)+t],
// B[8*(l/16)+t][l%16]; register r holds D[4*(l/16)+r][l%16].
__device__ __forceinline__ floatx4 mfma16x16x32(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 pack8(const float* v) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = f2bf(v[i]);
  return r;
}

__device__ __forceinline__ uint32_t pack_bf16x2(bf16 lo, bf16 hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// Blocks are dealt round-robin to the 8 XCDs of an MI355X (block b runs on XCD
// b % 8). Remap so that consecutive logical tiles land on the same XCD and
// share its L2: logical = (b % 8) * (n / 8) + b / 8, valid when n % 8 == 0.
__device__ __forceinline__ int xcd_remap(int b, int n) {
  if ((n & 7) != 0) return b;
  return (b & 7) * (n >> 3) + (b >> 3);
}
