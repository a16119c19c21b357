// Block-tiled bf16 GEMM core for gfx950: Y[m, n] = sum_k X[m, k] * W[n, k].
//
// Both operands are K-contiguous (nn.Linear layout), so each block stages a
// BM x BK tile of X and a BN x BK tile of W in LDS, double-buffered, and each
// wave runs v_mfma_f32_32x32x16_bf16 on its (WTM x WTN) sub-tile.
//
// The product is formed transposed (D = W_tile * X_tile^T), so accumulator
// register r of lane l holds output row m = l % 32 and column
// n = 8*(r/4) + 4*(l/32) + r%4: four consecutive columns per lane, which the
// epilogue writes as one 8-byte store.
//
// LDS rows are BK = 64 bf16 = 128 bytes = 8 chunks of 16 bytes; chunk c of row
// r is stored at chunk slot c ^ (r & 7), so the 8 lanes that share an LDS cycle
// on a ds_read_b128 (8 consecutive rows, same chunk) hit 8 different 16-byte
// slots and the row-wise global->LDS writes stay conflict-free as well.
#pragma once

#include "q3_common.h"

namespace q3 {

constexpr int kBK = 64;           // K elements per LDS stage
constexpr int kChunks = kBK / 8;  // 16-byte chunks per LDS row

__device__ __forceinline__ int swz(int row, int chunk) { return row * kBK + ((chunk ^ (row & 7)) << 3); }

// Where the rows of the X operand come from.
struct RowSource {
  const bf16* base;   // X
  int64_t ld;         // row stride (elements)
  const int* gather;  // optional: logical row -> physical row of X
};

// One stage of global loads for a ROWS x BK tile, held in registers between
// the global read and the LDS write (the double-buffer hand-off).
template <int ROWS, int NT>
struct TileLoader {
  static constexpr int kPer = ROWS * kChunks / NT;  // 16-byte chunks per thread
  static_assert(ROWS * kChunks % NT == 0, "tile not divisible by threads");
  bf16x8 v[kPer];

  // rows_valid: logical rows [0, rows_valid) of the tile exist.
  // row_ptr(i): pointer to the first element of logical tile row i.
  template <typename RowPtr>
  __device__ __forceinline__ void load(RowPtr row_ptr, int rows_valid, int k0, int K, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int id = tid + i * NT;
      const int r = id / kChunks;
      const int c = id % kChunks;
      const int k = k0 + c * 8;
      if (r < rows_valid && k < K) {
        v[i] = *reinterpret_cast<const bf16x8*>(row_ptr(r) + k);
      } else {
        v[i] = bf16x8{};
      }
    }
  }
  __device__ __forceinline__ void store(bf16* s, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int id = tid + i * NT;
      const int r = id / kChunks;
      const int c = id % kChunks;
      *reinterpret_cast<bf16x8*>(s + swz(r, c)) = v[i];
    }
  }
};

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
  // One BK stage: sX holds the block's X tile, sW the W tile.
  __device__ __forceinline__ void mma_stage(const bf16* sX, const bf16* sW, int wrow_m, int wrow_n, int lane) {
    const int l32 = lane & 31;
    const int h = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8 a[TN], b[TM];
#pragma unroll
      for (int i = 0; i < TN; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(sW + swz(wrow_n + i * 32 + l32, ks * 2 + h));
#pragma unroll
      for (int j = 0; j < TM; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(sX + swz(wrow_m + j * 32 + l32, ks * 2 + h));
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) c[i][j] = mfma32x32x16(a[i], b[j], c[i][j]);
    }
  }
};

}  // namespace q3
