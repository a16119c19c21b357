// Shared pieces of the bf16 MFMA kernels for gfx950 (GEMM, GEMV, attention):
// buffer resources, direct-to-LDS loads, wait counters and the accumulator
// block of a wave.
//
// GEMM convention: Y[m, n] = sum_k X[m, k] * W[n, k], both operands
// K-contiguous (nn.Linear layout). The product is formed transposed
// (D = W_tile * X_tile^T), so accumulator register r of lane l holds output
// row m = l % 32 and column n = 8*(r/4) + 4*(l/32) + r%4: four consecutive
// columns per lane, which the epilogue writes as one 8-byte store.
#pragma once

#include "q3_common.h"

namespace q3 {

constexpr int kBK = 32;      // K elements per LDS stage (default GEMM configuration)
constexpr int kStages = 4;   // LDS ring depth (default GEMM configuration)

// Buffer resource over `bytes` bytes at `base`: loads at byte offsets >= bytes
// return zeros (branch-free edges: rows past the matrix, the K tail, stages
// past the end of the loop). `bytes` is clamped to [0, 2^31 - 1]: a
// non-positive size gives an empty range, never a wrapped huge one.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int32_t n = bytes <= 0 ? 0 : (bytes >= 0x7fffffffLL ? 0x7fffffff : (int32_t)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
constexpr uint32_t kOOB = 0x80000000u;  // a byte offset that is always out of range

__device__ __forceinline__ bf16x8 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0));
}

// 16 bytes per lane from the buffer at `voff` into LDS at byte address
// `lds_byte` + 16 * lane. Issued as inline asm (m0 holds the LDS address) so the
// compiler inserts no wait of its own; callers fence with vm_wait<N>(). The LDS
// address is wave-uniform by contract; it is pinned to a scalar register here,
// since the compiler can leave a uniform value in a vector register (the "s"
// constraint then fails to assemble).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds_byte) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_byte);
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(voff), "s"(m0v), "s"(r)
               : "memory");
}
// dma16 with the non-temporal hint, for data read exactly once (the KV cache
// in decode): streaming it past the caches keeps HBM reads near their peak.
__device__ __forceinline__ void dma16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds_byte) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_byte);
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen nt lds" ::"v"(voff), "s"(m0v), "s"(r)
               : "memory");
}
template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

// Accumulators of one wave: TN x TM 32x32 MFMA tiles (TN along n, TM along m).
template <int TN, int TM>
struct WaveAcc {
  floatx16 c[TN][TM];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) c[i][j] = floatx16{};
  }
};

}  // namespace q3
