// Block-tiled bf16 GEMM core for gfx950: Y[m, n] = sum_k X[m, k] * W[n, k].
//
// Both operands are K-contiguous (nn.Linear layout). A block stages BM x BK
// tiles of X and BN x BK tiles of W in a ring of kStages LDS buffers, filled by
// direct global->LDS loads (buffer_load_dwordx4 ... lds): no staging
// registers, and a prefetch distance of kStages - 1 tiles. Each wave runs
// v_mfma_f32_32x32x16_bf16 on its (WTM x WTN) sub-tile.
//
// The product is formed transposed (D = W_tile * X_tile^T), so accumulator
// register r of lane l holds output row m = l % 32 and column
// n = 8*(r/4) + 4*(l/32) + r%4: four consecutive columns per lane, which the
// epilogue writes as one 8-byte store.
//
// LDS rows are BK = 32 bf16 = 64 bytes = 4 chunks of 16 bytes; chunk c of row
// r sits at slot c ^ h(r), h(r) = ((r >> 1) & 3) ^ ((r >> 3) & 1). A fragment
// read (ds_read_b128) has 16 consecutive rows read one chunk each; with this h
// they land on 16 distinct 16-byte positions of a 256-byte window (and any 8
// consecutive rows on 8 distinct positions of a 128-byte window), so the reads
// are free of bank conflicts. A direct-to-LDS load writes 64 lanes x 16 bytes
// contiguously (16 rows), so each lane fetches the global chunk whose swizzled
// slot is its LDS position.
#pragma once

#include "q3_common.h"

namespace q3 {

constexpr int kBK = 32;           // K elements per LDS stage
constexpr int kChunks = kBK / 8;  // 16-byte chunks per LDS row
constexpr int kStages = 4;        // LDS ring depth

__device__ __forceinline__ int swz_slot(int row, int chunk) { return chunk ^ (((row >> 1) & 3) ^ ((row >> 3) & 1)); }
// Element offset of (row, chunk) in a tile.
__device__ __forceinline__ int swz(int row, int chunk) { return row * kBK + (swz_slot(row, chunk) << 3); }

// Buffer resource over `bytes` bytes at `base`: loads at byte offsets >= bytes
// return zeros (branch-free edges: rows past the matrix, the K tail, stages
// past the end of the loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int32_t n = bytes >= 0x7fffffffLL ? 0x7fffffff : (int32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
constexpr uint32_t kOOB = 0x80000000u;  // a byte offset that is always out of range

__device__ __forceinline__ bf16x8 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0));
}

// 16 bytes per lane from the buffer at `voff` into LDS at byte address
// `lds_byte` + 16 * lane. Issued as inline asm (m0 holds the LDS address) so the
// compiler inserts no wait of its own; callers fence with vm_wait<N>().
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds_byte) {
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(voff), "s"(lds_byte), "s"(r)
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
  // One BK stage: sX holds the block's X tile, sW the W tile. All fragment
  // reads of the stage are issued before its MFMAs, so the LDS latency of the
  // second K step hides behind the first step's MFMAs.
  __device__ __forceinline__ void mma_stage(const bf16* sX, const bf16* sW, int wrow_m, int wrow_n, int lane) {
    constexpr int KS = kBK / 16;
    const int l32 = lane & 31;
    const int h = lane >> 5;
    bf16x8 a[KS][TN], b[KS][TM];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int i = 0; i < TN; ++i)
        a[ks][i] = *reinterpret_cast<const bf16x8*>(sW + swz(wrow_n + i * 32 + l32, ks * 2 + h));
#pragma unroll
      for (int j = 0; j < TM; ++j)
        b[ks][j] = *reinterpret_cast<const bf16x8*>(sX + swz(wrow_m + j * 32 + l32, ks * 2 + h));
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) c[i][j] = mfma32x32x16(a[ks][i], b[ks][j], c[i][j]);
  }
};

}  // namespace q3
