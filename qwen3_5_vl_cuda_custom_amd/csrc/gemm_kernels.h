// MFMA GEMM kernels (dense, batched, dual-B SwiGLU, MoE-grouped) built on the
// tile core in gemm_tile.h. Host launchers live in gemm.hip and moe.hip.
#pragma once

#include "gemm_tile.h"

namespace q3 {

enum Epilogue : int {
  kEpiStore = 0,     // C = acc (+ bias[n]) (+ R[m, n]), rounded once
  kEpiSwiGLU = 1,    // C = silu(acc_gate) * acc_up, rounded once
  kEpiRowScale = 2,  // C = bf16(bf16(acc) * s[m])  (MoE expert output x routing weight)
  kEpiStoreF32 = 3,  // C (fp32, ld = ldc floats, batch stride bsC floats) = acc, not rounded (split-K partials)
};

// Up to 4 weight matrices stacked along N and computed in one launch (the
// q/k/v projections of one input): segment i covers output columns
// [start[i], start[i+1]) (the last one up to N), rows of w[i], bias b[i] (or
// null). n <= 1: the plain W / bias of the params.
struct WeightSegments {
  int n;
  int start[4];
  const bf16* w[4];
  const bf16* b[4];
};

template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const T*>(((uint64_t)hi << 32) | lo);
}

template <typename T>
__device__ __forceinline__ T pick4(int s, T a, T b, T c, T d) {
  return s == 0 ? a : s == 1 ? b : s == 2 ? c : d;
}

__device__ __forceinline__ int segment_of(const WeightSegments& s, int col) {
  int i = 0;
#pragma unroll
  for (int j = 1; j < 4; ++j)
    if (j < s.n && col >= s.start[j]) i = j;
  return i;
}

struct GemmParams {
  const bf16* X;     // (M, K) rows, ld = ldx
  const bf16* W;     // (N, K) rows, ld = ldw  (gate weight for SwiGLU)
  const bf16* W2;    // up weight for SwiGLU
  const bf16* bias;  // (N) or null
  const bf16* R;     // residual (M, N) or null, ld = ldr
  bf16* C;           // (M, N_out), ld = ldc
  const bf16* rowscale;  // kEpiRowScale: (rows) scale
  int M, N, K;       // N = output columns (SwiGLU: intermediate size)
  int M_src;         // rows of X addressable through `gather` (grouped problems)
  int64_t ldx, ldw, ldr, ldc;
  int64_t bsX, bsW, bsC;  // batch strides (blockIdx.z)
  int group_m;       // tile-order grouping along m
  // MoE-grouped problems: tiles come from a device-side table.
  const int* gather;      // logical row -> row of X (null: identity)
  const int* tile_table;  // per m-tile: (expert << 20) | start row ... see moe.hip
  const int* group_end;   // per expert: end row (exclusive) in the sorted order
  const int* n_tiles_total;  // device scalar: number of valid m-tiles
  int64_t expert_stride_w;   // elements between consecutive experts' weights
  WeightSegments seg;        // dense (non-grouped, batch 1) store epilogue only
  int act;                   // kEpiStore: 1 = gelu_tanh of (acc + bias), before the residual
};

// Where a block's tile sits: logical rows [m_begin, m_begin + rows_m), output
// columns from n0_out, and the (possibly re-based) operand pointers.
struct TileCtx {
  int m_begin, rows_m, n0_out, n_lim;
  const bf16* X;
  const bf16* W;
  const bf16* W2;
  const bf16* bias;
  bf16* C;
};

// Returns false when the block has no tile (grouped problems past the last
// valid m-tile).
template <int BM, int BN_OUT, int EPI, bool GROUPED>
__device__ __forceinline__ bool tile_ctx(const GemmParams& p, TileCtx& t) {
  const int n_tiles_n = (p.N + BN_OUT - 1) / BN_OUT;
  int tile_m, tile_n;
  int m_begin, m_end;  // logical rows of this tile: [m_begin, m_end)
  const bf16* W = p.W;
  const bf16* W2 = p.W2;
  const bf16* X = p.X;
  bf16* C = p.C;

  if constexpr (GROUPED) {
    // XCD-aware over the valid tiles (known on the device only): blocks are
    // dealt round-robin over the 8 XCDs, so XCD x takes the contiguous range
    // [x * per, (x + 1) * per) of the (m-tile, n-tile) order; the blocks that
    // share an expert's weight panels and its rows' activations then run on
    // one XCD at the same time. Surplus blocks exit.
    const int total = *p.n_tiles_total * n_tiles_n;
    const int per = (total + 7) / 8;
    const int b = blockIdx.x;
    if (b / 8 >= per) return false;
    const int L = (b % 8) * per + b / 8;
    if (L >= total) return false;
    const int tt = L / n_tiles_n;
    tile_n = L % n_tiles_n;
    const int entry = p.tile_table[tt];
    const int expert = entry >> 20;
    m_begin = entry & 0xFFFFF;
    m_end = min(m_begin + BM, p.group_end[expert]);
    W += (int64_t)expert * p.expert_stride_w;
    if (W2) W2 += (int64_t)expert * p.expert_stride_w;
    tile_m = 0;
  } else {
    const int n_tiles_m = (p.M + BM - 1) / BM;
    const int total = n_tiles_m * n_tiles_n;
    const int pid = xcd_remap(blockIdx.x, total);
    const int gm = p.group_m;
    const int per_group = gm * n_tiles_n;
    const int group = pid / per_group;
    const int first_m = group * gm;
    const int size_m = min(n_tiles_m - first_m, gm);
    tile_m = first_m + (pid % per_group) % size_m;
    tile_n = (pid % per_group) / size_m;
    m_begin = tile_m * BM;
    m_end = min(m_begin + BM, p.M);
    const int z = blockIdx.z;
    X += z * p.bsX;
    W += z * p.bsW;
    if constexpr (EPI == kEpiStoreF32)
      C = reinterpret_cast<bf16*>(reinterpret_cast<float*>(C) + z * p.bsC);
    else
      C += z * p.bsC;
  }
  const int rows_m = m_end - m_begin;
  const int n0_out = tile_n * BN_OUT;
  // Stacked weights (p.seg.n > 1): W and bias stay those of the params; the
  // kernel picks each loaded row's and each stored column's segment.
  int n_lim = p.N;
  const bf16* bias = p.bias;

  // Everything here is block-uniform; integer division may still have left it
  // in vector registers. Pin it to scalars so buffer resources stay scalar.
  t.m_begin = __builtin_amdgcn_readfirstlane(m_begin);
  t.rows_m = __builtin_amdgcn_readfirstlane(rows_m);
  t.n0_out = __builtin_amdgcn_readfirstlane(n0_out);
  t.n_lim = __builtin_amdgcn_readfirstlane(n_lim);
  t.X = uniform_ptr(X);
  t.W = uniform_ptr(W);
  t.W2 = W2 ? uniform_ptr(W2) : nullptr;
  t.bias = bias ? uniform_ptr(bias) : nullptr;
  t.C = const_cast<bf16*>(uniform_ptr(C));
  return true;
}

// Bias of the stacked-weight segment holding output column n (wave-uniform),
// re-based so that it is indexed by the column (null when the segment has no
// bias). Constant-index selects pinned to scalars: a dynamic index into the
// by-value params would move them to memory.
__device__ __forceinline__ const bf16* seg_bias(const WeightSegments& sg, int n) {
  const int s = __builtin_amdgcn_readfirstlane(segment_of(sg, n));
  const bf16* b = uniform_ptr(pick4(s, sg.b[0], sg.b[1], sg.b[2], sg.b[3]));
  const int st = __builtin_amdgcn_readfirstlane(pick4(s, sg.start[0], sg.start[1], sg.start[2], sg.start[3]));
  return b ? b - st : nullptr;
}

// Epilogue through LDS. Stored straight from the accumulators, one wave store
// instruction writes 32 rows x 16 bytes (a lane holds 4 consecutive columns of
// one row), which the memory system takes at ~1.2 TB/s: at S = 4096 that is
// ~80 us of the gate/up GEMM. Instead the accumulators (after the register-level
// part of the epilogue, SwiGLU) go to the LDS ring, free by then, as fp32 in
// passes of RP rows; every wave then reads whole rows back, 8 consecutive columns
// per lane, adds bias / applies gelu / adds the residual, rounds once and
// stores 16 bytes per lane (kEpiStoreF32: 32 bytes of fp32, not rounded):
// contiguous rows per instruction. LDS rows are BN_OUT fp32; 16-byte chunk c
// of row r sits at chunk c ^ (r & 15).
// Accumulator visitors for the epilogues: f(mr, lrow, col, v) for every group
// of 4 consecutive output columns a lane holds, where mr is the MFMA tile's
// first row in the block tile (wave-uniform), lrow the lane's row in that
// tile, col the group's first output column (block tile) and v its values
// (SwiGLU applied). 32x32x16 tiles: lane l holds row l % 32 and columns 8 g +
// 4 (l / 32) + q of register 4 g + q. SwiGLU pairs the gate / up 32-row W
// tiles 2 i, 2 i + 1.
template <int EPI, int WTM, int WTN, int TN, int TM, typename F>
__device__ __forceinline__ void visit_acc32(const floatx16 (&c)[TN][TM], int wm, int wn, int lane, F&& f) {
  constexpr int WTN_OUT = EPI == kEpiSwiGLU ? WTN / 2 : WTN;
  constexpr int TN_OUT = EPI == kEpiSwiGLU ? TN / 2 : TN;
  const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int j = 0; j < TM; ++j) {
#pragma unroll
    for (int i = 0; i < TN_OUT; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        floatx4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (EPI == kEpiSwiGLU)
            v[q] = silu_mul(c[2 * i][j][4 * g + q], c[2 * i + 1][j][4 * g + q]);
          else
            v[q] = c[i][j][4 * g + q];
        }
        f(wm * WTM + j * 32, l32, wn * WTN_OUT + i * 32 + 8 * g + 4 * h, v);
      }
    }
  }
}

// 16x16x32 tiles: lane l holds row l % 16 and columns 4 (l / 16) + q (register
// q). SwiGLU: the wave's W rows come in 64-row groups, 32 gate rows then the
// 32 up rows of the same output columns, so output tile o pairs W tiles
// 4 (o / 2) + o % 2 (gate) and that + 2 (up).
template <int EPI, int WTM, int WTN, int TN, int TM, typename F>
__device__ __forceinline__ void visit_acc16(const floatx4 (&c)[TN][TM], int wm, int wn, int lane, F&& f) {
  constexpr int WTN_OUT = EPI == kEpiSwiGLU ? WTN / 2 : WTN;
  constexpr int TN_OUT = EPI == kEpiSwiGLU ? TN / 2 : TN;
  static_assert(EPI != kEpiSwiGLU || WTN % 64 == 0, "SwiGLU: whole 64-row gate/up groups per wave");
  const int l16 = lane & 15, q4 = lane >> 4;
#pragma unroll
  for (int j = 0; j < TM; ++j) {
#pragma unroll
    for (int o = 0; o < TN_OUT; ++o) {
      floatx4 v;
      if constexpr (EPI == kEpiSwiGLU) {
        const int gi = 4 * (o / 2) + o % 2;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = silu_mul(c[gi][j][q], c[gi + 2][j][q]);
      } else {
        v = c[o][j];
      }
      f(wm * WTM + j * 16, l16, wn * WTN_OUT + o * 16 + 4 * q4, v);
    }
  }
}

template <int BM, int BN_OUT, int EPI, int NW, int LDS_BYTES, typename VISIT>
__device__ __forceinline__ void store_tile_lds(const GemmParams& p, const TileCtx& t, VISIT&& visit, float* lds) {
  constexpr int RP0 = LDS_BYTES / (BN_OUT * 4);
  constexpr int RP = RP0 >= 256 ? 256 : RP0 >= 128 ? 128 : RP0 >= 64 ? 64 : 32;  // rows per pass
  constexpr int NPASS = (BM + RP - 1) / RP;
  constexpr int C8 = BN_OUT / 8;                          // 8-column items per row
  static_assert(BN_OUT % 64 == 0 && RP % 32 == 0, "epilogue tiling");
  const int m_begin = t.m_begin, rows_m = t.rows_m, n0_out = t.n0_out;
  const int N = p.N;
  const bool vec_ok = ((p.ldc & 7) == 0) && (reinterpret_cast<uintptr_t>(t.C) & 15) == 0 &&
                      (p.R == nullptr || ((p.ldr & 7) == 0 && (reinterpret_cast<uintptr_t>(p.R) & 15) == 0));
  auto slot = [](int r, int col) { return r * BN_OUT + ((((col >> 2) ^ (r & 15))) << 2); };
  __syncthreads();  // every wave is done with the main loop's LDS
#pragma unroll
  for (int pass = 0; pass < NPASS; ++pass) {
    const int r0 = pass * RP;
    // 1. this wave's accumulator rows of the pass -> LDS (fp32)
    visit([&](int mr, int lrow, int col, floatx4 v) {
      if (mr < r0 || mr >= r0 + RP) return;  // wave-uniform
      *reinterpret_cast<floatx4*>(lds + slot(mr - r0 + lrow, col)) = v;
    });
    __syncthreads();
    // 2. rows of the pass, 8 columns per lane, finished and stored
    const int nrows = min(RP, rows_m - r0);
    for (int it = threadIdx.x; it < nrows * C8; it += NW * 64) {
      const int lr = it / C8, c8 = it - lr * C8;
      const int col = c8 * 8;
      const floatx4 a = *reinterpret_cast<const floatx4*>(lds + slot(lr, col));
      const floatx4 b = *reinterpret_cast<const floatx4*>(lds + slot(lr, col + 4));
      float o[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
      const int m = m_begin + r0 + lr;
      const int n = n0_out + col;
      bf16* crow = t.C + (int64_t)m * p.ldc;
      if constexpr (EPI == kEpiStore) {
        const bf16* bias = t.bias;
        if (p.seg.n > 1) {  // per lane: the lanes' columns may lie in different segments
          const int sgi = segment_of(p.seg, n);  // segment starts are multiples of 16
          const bf16* b = pick4(sgi, p.seg.b[0], p.seg.b[1], p.seg.b[2], p.seg.b[3]);
          bias = b ? b - pick4(sgi, p.seg.start[0], p.seg.start[1], p.seg.start[2], p.seg.start[3]) : nullptr;
        }
        if (bias) {
          if (vec_ok && n + 7 < N) {
            const bf16x8 bv = *reinterpret_cast<const bf16x8*>(bias + n);
#pragma unroll
            for (int q = 0; q < 8; ++q) o[q] += bf2f(bv[q]);
          } else {
#pragma unroll
            for (int q = 0; q < 8; ++q)
              if (n + q < N) o[q] += bf2f(bias[n + q]);
          }
        }
        if (p.act) {
#pragma unroll
          for (int q = 0; q < 8; ++q) o[q] = gelu_tanh_fast(o[q]);
        }
        if (p.R) {
          const bf16* rrow = p.R + (int64_t)m * p.ldr;
          if (vec_ok && n + 7 < N) {
            const bf16x8 rv = *reinterpret_cast<const bf16x8*>(rrow + n);
#pragma unroll
            for (int q = 0; q < 8; ++q) o[q] += bf2f(rv[q]);
          } else {
#pragma unroll
            for (int q = 0; q < 8; ++q)
              if (n + q < N) o[q] += bf2f(rrow[n + q]);
          }
        }
      }
      if constexpr (EPI == kEpiStoreF32) {
        float* frow = reinterpret_cast<float*>(t.C) + (int64_t)m * p.ldc;
        if (vec_ok && n + 7 < N) {
          *reinterpret_cast<floatx4*>(frow + n) = floatx4{o[0], o[1], o[2], o[3]};
          *reinterpret_cast<floatx4*>(frow + n + 4) = floatx4{o[4], o[5], o[6], o[7]};
        } else {
#pragma unroll
          for (int q = 0; q < 8; ++q)
            if (n + q < N) frow[n + q] = o[q];
        }
      } else if (vec_ok && n + 7 < N) {
        bf16x8 v;
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = f2bf(o[q]);
        *reinterpret_cast<bf16x8*>(crow + n) = v;
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (n + q < N) crow[n + q] = f2bf(o[q]);
      }
    }
    if (pass + 1 < NPASS) __syncthreads();  // the next pass overwrites the LDS
  }
}

// True when the stored value takes no fp32 arithmetic after its one rounding:
// SwiGLU, the row scale (whose first step rounds the accumulator), a plain
// store without bias, activation or residual.
template <int EPI>
__device__ __forceinline__ bool epi_rounds_first(const GemmParams& p, const TileCtx& t) {
  if constexpr (EPI == kEpiSwiGLU || EPI == kEpiRowScale) {
    return true;
  } else if constexpr (EPI == kEpiStoreF32) {
    return false;
  } else {
    bool bias = p.seg.n > 1 ? false : t.bias != nullptr;
#pragma unroll
    for (int i = 0; i < 4; ++i) bias = bias || (p.seg.n > 1 && i < p.seg.n && p.seg.b[i] != nullptr);
    return !bias && !p.act && p.R == nullptr;
  }
}

// The LDS epilogue for outputs that round first (epi_rounds_first): the
// accumulators go to LDS already rounded to bf16, half the bytes of the fp32
// staging (a 256x256 tile fits one pass), and every lane then moves whole
// 16-byte chunks from LDS to memory, with all of a full pass's LDS reads in
// flight before its stores. Values are those of store_tile_lds (one rounding,
// same arithmetic). LDS rows are BN_OUT bf16; 16-byte chunk c of row r sits
// at chunk c ^ (r & SWZ).
template <int BM, int BN_OUT, int EPI, int NW, int LDS_BYTES, typename VISIT>
__device__ __forceinline__ void store_tile_lds_bf16(const GemmParams& p, const TileCtx& t, VISIT&& visit, bf16* lds) {
  constexpr int RP0 = LDS_BYTES / (BN_OUT * 2);
  constexpr int RP1 = RP0 >= 256 ? 256 : RP0 >= 128 ? 128 : RP0 >= 64 ? 64 : 32;
  constexpr int RP = RP1 < BM ? RP1 : BM;  // rows per pass
  constexpr int NPASS = (BM + RP - 1) / RP;
  constexpr int C8 = BN_OUT / 8;  // 16-byte chunks per row
  // XOR swizzle over aligned blocks of chunks that divide the row (24 chunks:
  // blocks of 8), so a swizzled chunk stays in its row.
  constexpr int SWZ = C8 % 16 == 0 ? 15 : 7;
  static_assert(C8 % (SWZ + 1) == 0, "swizzle blocks must divide the row");
  constexpr int NT = NW * 64;
  static_assert(BN_OUT % 64 == 0 && RP % 32 == 0, "epilogue tiling");
  constexpr int ITEMS = (RP * C8) / NT;  // chunks per thread in a full pass
  static_assert(ITEMS >= 1 && (RP * C8) % NT == 0, "whole chunks per thread");
  const int m_begin = t.m_begin, rows_m = t.rows_m, n0_out = t.n0_out;
  const int N = p.N;
  const bool vec_ok = ((p.ldc & 7) == 0) && (reinterpret_cast<uintptr_t>(t.C) & 15) == 0;
  const bool full_n = vec_ok && n0_out + BN_OUT <= N;
  auto slot = [](int r, int c8) { return r * BN_OUT + ((c8 ^ (r & SWZ)) << 3); };
  // One finished chunk (8 columns) of tile row lr of the pass at r0.
  auto finish = [&](bf16x8 v, int r0, int lr, int c8, bool whole) {
    const int m = m_begin + r0 + lr;
    const int n = n0_out + c8 * 8;
    if constexpr (EPI == kEpiRowScale) {
      const float rs = bf2f(p.rowscale[m]);
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = f2bf(bf2f(v[q]) * rs);
    }
    bf16* crow = t.C + (int64_t)m * p.ldc;
    if (whole || (vec_ok && n + 7 < N)) {
      *reinterpret_cast<bf16x8*>(crow + n) = v;
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (n + q < N) crow[n + q] = v[q];
    }
  };
  __syncthreads();  // every wave is done with the main loop's LDS
#pragma unroll
  for (int pass = 0; pass < NPASS; ++pass) {
    const int r0 = pass * RP;
    // 1. this wave's accumulator rows of the pass -> LDS, rounded once
    visit([&](int mr, int lrow, int col, floatx4 v) {
      if (mr < r0 || mr >= r0 + RP) return;  // wave-uniform
      bf16x4 b;
#pragma unroll
      for (int q = 0; q < 4; ++q) b[q] = f2bf(v[q]);
      *reinterpret_cast<bf16x4*>(lds + slot(mr - r0 + lrow, col >> 3) + (col & 7)) = b;
    });
    __syncthreads();
    // 2. rows of the pass -> memory, one 16-byte chunk per lane and item
    const int nrows = min(RP, rows_m - r0);
    if (nrows == RP && full_n) {
      bf16x8 v[ITEMS];
#pragma unroll
      for (int u = 0; u < ITEMS; ++u) {
        const int it = threadIdx.x + u * NT;
        v[u] = *reinterpret_cast<const bf16x8*>(lds + slot(it / C8, it % C8));
      }
#pragma unroll
      for (int u = 0; u < ITEMS; ++u) {
        const int it = threadIdx.x + u * NT;
        finish(v[u], r0, it / C8, it % C8, true);
      }
    } else {
      for (int it = threadIdx.x; it < nrows * C8; it += NT)
        finish(*reinterpret_cast<const bf16x8*>(lds + slot(it / C8, it % C8)), r0, it / C8, it % C8, false);
    }
    if (pass + 1 < NPASS) __syncthreads();  // the next pass overwrites the LDS
  }
}

// Swizzle of a BKT-element LDS row (BKT / 8 chunks of 16 bytes): chunk c of
// row r sits at slot c ^ dma_swz<BKT>(r). For 32 or 16 consecutive rows read
// one chunk each (a fragment read), the slots land on distinct 16-byte
// positions of every 128-byte (8 rows) and 256-byte (16 rows) window, so
// ds_read_b128 is conflict-free.
template <int BKT>
__device__ __forceinline__ int dma_swz(int r) {
  if constexpr (BKT == 32) return ((r >> 1) & 3) ^ ((r >> 3) & 1);
  else return (r & 7) ^ ((r >> 3) & 1);
}

// The tile GEMM with direct-to-LDS operand loads: stage kt's X and W tiles
// (BKT-wide in K) go global -> LDS by buffer_load ... lds into a ring of NST
// slots, issued NST - 1 stages ahead, so neither staging registers nor LDS
// store instructions sit in the loop. One DMA instruction fills 64 / (BKT / 8)
// rows; the lane that lands at slot s of row r fetches chunk s ^ dma_swz(r)
// (an involution), which keeps fragment reads conflict-free.
//
// The loop is software-pipelined over 16-wide K steps: the fragments of step
// q + 1 are read while the MFMAs of step q run, and each stage's barrier sits
// before its last step's MFMAs (which overlap the first reads of the next
// stage), so no wave starts a stage waiting on LDS.
//
// MF16: the same ring with v_mfma_f32_16x16x32_bf16 instead of 32x32x16. For
// the same work it moves less data through the register file (operands 4 KB
// + accumulators 4 KB per 32K flops, against 2 KB + 8 KB): on random data
// under the power cap a pure MFMA loop sustains ~2.03 PFLOP/s with it against
// ~1.80 with 32x32x16 (MI355X), and these GEMMs run power-limited.
template <int BM, int BN, int WM, int WN, int EPI, bool GROUPED, int NST, int BKT, int NSTW = NST, bool MF16 = false>
__global__ __launch_bounds__(WM* WN * 64) void gemm_bf16_dma_kernel(const GemmParams p) {
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM;
  constexpr int WTN = BN / WN;
  constexpr int TM = WTM / 32;
  constexpr int TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile too small");
  static_assert(EPI != kEpiSwiGLU || (TN % 2 == 0), "SwiGLU pairs gate/up tiles");
  static_assert(BKT == 32 || BKT == 64, "stage width");
  constexpr int BN_OUT = (EPI == kEpiSwiGLU) ? BN / 2 : BN;
  constexpr int CH = BKT / 8;              // 16-byte chunks per LDS row
  constexpr int KS = BKT / 16;             // MFMA K steps per stage
  // X slots (NST) and W slots (NSTW, up to two more: weights come from HBM,
  // activations from L2, so W may be issued further ahead).
  static_assert(NSTW >= NST && NSTW <= NST + 2, "W ring depth");
  constexpr int kStageX = BM * BKT, kStageW = BN * BKT;  // elements per ring slot
  constexpr int kRing = NST * kStageX + NSTW * kStageW;
  constexpr int RPI = 64 / CH;             // rows per DMA instruction
  constexpr int DX = BM / RPI, DW = BN / RPI;
  static_assert((DX + DW) % NW == 0 && DX % NW == 0, "DMA instructions must split evenly over the waves");
  constexpr int PX = DX / NW, PW = DW / NW;  // per wave and stage
  static_assert(MF16 || TN * TM >= TN + TM, "the interleave needs more MFMAs than fragment reads");

  __shared__ __attribute__((aligned(1024))) bf16 smem[kRing];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Waves w and w + 4 share a SIMD; with wm = wave / WN each SIMD holds waves of
  // different m-ranges, so a tile whose last rows are empty (MoE remainders, M
  // edges) leaves no SIMD with all of its waves busy while others idle.
  const int wn = wave % WN;
  const int wm = wave / WN;

  TileCtx tc;
  if (!tile_ctx<BM, BN_OUT, EPI, GROUPED>(p, tc)) return;
  const int m_begin = tc.m_begin, rows_m = tc.rows_m, n0_out = tc.n0_out, n_lim = tc.n_lim;
  const int K = p.K;
  const int nk = (K + BKT - 1) / BKT;
  const int64_t ldx = p.ldx, ldw = p.ldw;

  // Lane geometry of instruction i of this wave: tile row, and the global
  // chunk that lands in the lane's LDS slot. The swizzle depends on the row
  // mod 16 only, and instruction i's rows are those of instruction 0 plus a
  // multiple of 16, so one chunk index serves every instruction.
  static_assert((NW * RPI) % 16 == 0, "one swizzle chunk per lane");
  const int lrow = lane / CH, lslot = lane % CH;
  const int dc = lslot ^ dma_swz<BKT>(wave * RPI + lrow);
  uint32_t xoff[PX], woff[PW];
  const bf16* wsrc[PW];  // weight matrix of each W instruction (its rows share one segment) ...
  int wrows[PW];         // ... and its rows
#pragma unroll
  for (int i = 0; i < PX; ++i) {
    const int r = (wave + NW * i) * RPI + lrow;
    if (r < rows_m) {
      const int lr = m_begin + r;
      const int64_t pr = p.gather ? (int64_t)p.gather[lr] : (int64_t)lr;
      xoff[i] = (uint32_t)(pr * ldx * 2);
    } else {
      xoff[i] = kOOB;
    }
  }
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int r = (wave + NW * i) * RPI + lrow;
    int n, rbase = 0, rlim;  // global row n; rows of the source matrix: [rbase, rbase + rlim)
    const bf16* wb;
    if constexpr (EPI == kEpiSwiGLU) {
      n = n0_out + (r >> 6) * 32 + (r & 31);  // 32-row groups alternate gate / up
      const bool up = (((wave + NW * i) * RPI) >> 5) & 1;  // the instruction's rows share one group
      wb = up ? tc.W2 : tc.W;
      rlim = p.N;
    } else {
      n = n0_out + r;
      wb = tc.W;
      rlim = n_lim;
      if (!GROUPED && p.seg.n > 1) {
        const int n_first = n0_out + (wave + NW * i) * RPI;  // host: segment starts are multiples of RPI
        const int sgi = __builtin_amdgcn_readfirstlane(segment_of(p.seg, n_first));
        wb = pick4(sgi, p.seg.w[0], p.seg.w[1], p.seg.w[2], p.seg.w[3]);
        rbase = pick4(sgi, p.seg.start[0], p.seg.start[1], p.seg.start[2], p.seg.start[3]);
        const int end = sgi + 1 < p.seg.n ? pick4(sgi, p.seg.start[1], p.seg.start[2], p.seg.start[3], p.N) : p.N;
        rlim = end - rbase;
      }
    }
    // Selects can leave uniform values in vector registers: pin them to scalars
    // so that the buffer resource is scalar.
    wb = uniform_ptr(wb);
    rbase = __builtin_amdgcn_readfirstlane(rbase);
    rlim = __builtin_amdgcn_readfirstlane(rlim);
    wsrc[i] = wb;
    wrows[i] = rlim;
    woff[i] = (n - rbase < rlim) ? (uint32_t)((int64_t)(n - rbase) * ldw * 2) : kOOB;
  }
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(tc.X, p.gather ? (int64_t)p.M_src * ldx * 2 : (int64_t)(m_begin + rows_m) * ldx * 2);
  const uint32_t lbase = lds_addr(smem);

  // LDS byte address of stage kt's X / W slot.
  auto xslot = [&](int kt) { return lbase + (uint32_t)((kt % NST) * kStageX * 2); };
  auto wslot = [&](int kt) { return lbase + (uint32_t)((NST * kStageX + (kt % NSTW) * kStageW) * 2); };
  auto issue_x = [&](int kt) {
    const int k = kt * BKT + dc * 8;
    const uint32_t sb = xslot(kt);
#pragma unroll
    for (int i = 0; i < PX; ++i) {
      const uint32_t off = (k < K && xoff[i] != kOOB) ? xoff[i] + (uint32_t)k * 2u : kOOB;
      dma16(rx, off, sb + (uint32_t)((wave + NW * i) * 1024));
    }
  };
  auto issue_w = [&](int kt) {
    const int k = kt * BKT + dc * 8;
    const uint32_t sb = wslot(kt);
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const uint32_t off = (k < K && woff[i] != kOOB) ? woff[i] + (uint32_t)k * 2u : kOOB;
      dma16(make_rsrc(wsrc[i], (int64_t)wrows[i] * ldw * 2), off, sb + (uint32_t)((wave + NW * i) * 1024));
    }
  };
  // The DMAs are issued in groups, one per stage: the group issued at the end
  // of stage j is X(j + NST) then W(j + NSTW) (each into the slot stage j has
  // just released). Stage kt + 1 has landed once every DMA up to X(kt + 1) has
  // (W(kt + 1) went out no later); the NST - 2 groups after it, and with
  // NSTW > NST the W of its own group, may still be in flight (vmcnt retires
  // in issue order).
  constexpr int kWait = (NST - 2) * (PX + PW) + (NSTW > NST ? PW : 0);
  auto issue_group = [&](int j) {
    if (j + NST >= 0) issue_x(j + NST);
    issue_w(j + NSTW);
  };

  if constexpr (MF16) {
    // 16x16x32 loop. Per wave and 32-wide K step: T16N W fragments (A) and
    // T16M X fragments (B), 16 rows x 32 k each (lane: row l % 16, 16-byte
    // chunk 4 ks + l / 16 of the 64-wide stage row), T16N x T16M MFMAs in
    // column order (X tile outer). W fragments are double-buffered; each X
    // fragment is re-read for the next step right after its column's last
    // MFMA (a single set: the accumulators take 128 registers at 128x64 per
    // wave). Two K steps per stage: the first carries W(kt + NST), the last
    // crosses the barrier as in the 32x32 loop (its first NQ MFMAs use every
    // fragment of the step) and carries X(kt + NST).
    static_assert(BKT == 64 && (NSTW == NST + 1 || (NSTW == NST + 2 && NST == 2)),
                  "16x16x32 loop: 64-wide stages, W ring one slot deeper (two with two X slots)");
    constexpr int T16N = WTN / 16, T16M = WTM / 16;
    constexpr int NQ = T16N > T16M ? T16N : T16M;
    constexpr int NM16 = T16N * T16M;
    floatx4 a16[T16N][T16M];
#pragma unroll
    for (int i = 0; i < T16N; ++i)
#pragma unroll
      for (int j = 0; j < T16M; ++j) a16[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    bf16x8 fw[2][T16N], fx[T16M];
    const int l16 = lane & 15, q4 = lane >> 4;
    const int rn = wn * WTN, rm = wm * WTM;
    auto rd_w = [&](int buf, int kt, int ks, int i) {
      const bf16* sw = smem + NST * kStageX + (kt % NSTW) * kStageW;
      const int r = rn + i * 16 + l16, c = ks * 4 + q4;
      fw[buf][i] = *reinterpret_cast<const bf16x8*>(sw + r * BKT + ((c ^ dma_swz<BKT>(r)) << 3));
    };
    auto rd_x = [&](int kt, int ks, int j) {
      const bf16* sx = smem + (kt % NST) * kStageX;
      const int r = rm + j * 16 + l16, c = ks * 4 + q4;
      fx[j] = *reinterpret_cast<const bf16x8*>(sx + r * BKT + ((c ^ dma_swz<BKT>(r)) << 3));
    };
    auto mf = [&](int buf, int i, int j) { a16[i][j] = mfma16x16x32(fw[buf][i], fx[j], a16[i][j]); };
    // MFMA (i, j) is among the last step's first NQ (before the barrier)
    auto pre = [](int i, int j) {
      bool in = false;
#pragma unroll
      for (int q = 0; q < NQ; ++q) in = in || (q % T16N == i && q % T16M == j);
      return in;
    };
    auto dma_x = [&](int kx_stage, int d) {
      const int k = kx_stage * BKT + dc * 8;
      const uint32_t off = (k < K && xoff[d] != kOOB) ? xoff[d] + (uint32_t)k * 2u : kOOB;
      dma16(rx, off, xslot(kx_stage) + (uint32_t)((wave + NW * d) * 1024));
    };
    auto dma_w16 = [&](int kw, int i) {
      const int k = kw * BKT + dc * 8;
      const uint32_t off = (k < K && woff[i] != kOOB) ? woff[i] + (uint32_t)k * 2u : kOOB;
      dma16(make_rsrc(wsrc[i], (int64_t)wrows[i] * ldw * 2), off, wslot(kw) + (uint32_t)((wave + NW * i) * 1024));
    };

#pragma unroll
    for (int j = 0; j < NST; ++j) {
      issue_w(j);
      issue_x(j);
    }
    if constexpr (NSTW == NST + 2) issue_w(NST);  // W one stage further ahead
    vm_wait<(NST - 1) * (PX + PW) + (NSTW - NST - 1) * PW>();  // stage 0 has landed
    __syncthreads();

    // Wave priority (256-row and 128x256 tiles), falling from one stage barrier to the
    // next: 2 after the barrier (the next stage's first reads, the remaining
    // MFMAs, X(kt + NST)), 1 for the first half of the next stage's first K
    // step, 0 from there to the barrier. The two waves of a SIMD run the same
    // schedule, so whichever has fallen behind issues first, and the pair
    // meets the next barrier closer together. Same instructions, same
    // results. Same-box A/Bs at S=4096, two levels (2 = 1 after the barrier,
    // 0 elsewhere) against none: gate/up 617 -> 604 and 620 -> 613 us, down
    // 311 -> 303 and 314 -> 307, the layer 1390.7 -> 1369.5 and 1404.2 ->
    // 1387.7 us; three levels against two: the layer 1340.6 -> 1334.4 and
    // 1421.4 -> 1409.8 us, C4 852 -> 846 us. The 128x128 ring (S=1024 o, C5)
    // was no faster with it. Prioritising only the post-barrier reads, or the
    // first half of the stage instead, gained nothing.
    constexpr bool kPrio = BM == 256 || BN == 256;  // the 256-row and 128x256 tiles
    auto main16 = [&](auto active_c) {
      constexpr bool A = decltype(active_c)::value;
      if constexpr (A) {
#pragma unroll
        for (int i = 0; i < T16N; ++i) rd_w(0, 0, 0, i);
#pragma unroll
        for (int j = 0; j < T16M; ++j) rd_x(0, 0, j);
      }
      for (int kt = 0; kt < nk; ++kt) {
        if constexpr (kPrio) __builtin_amdgcn_s_setprio(1);
        // step 0: W(kt + NSTW - 1) between the MFMAs, step 1's fragments read ahead
        constexpr int gw = (NM16 + PW - 1) / PW;
        int d = 0;
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (A) {
#pragma unroll
          for (int j = 0; j < T16M; ++j) {
#pragma unroll
            for (int i = 0; i < T16N; ++i) {
              const int m = j * T16N + i;
              mf(0, i, j);
              if (kPrio && m == NM16 / 2) __builtin_amdgcn_s_setprio(0);
              if (m < T16N) rd_w(1, kt, 1, m);
              if (i == T16N - 1) rd_x(kt, 1, j);
              if (d < PW && m % gw == gw - 1) dma_w16(kt + NSTW - 1, d++);
              __builtin_amdgcn_sched_barrier(0);
            }
          }
        }
#pragma unroll
        for (; d < PW; ++d) dma_w16(kt + NSTW - 1, d);
        __builtin_amdgcn_sched_barrier(0);
        // step 1: the NQ MFMAs that use every fragment, the barrier, then the
        // rest with stage kt + 1's first-step reads and X(kt + NST)
        if constexpr (A) {
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            mf(1, q % T16N, q % T16M);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        vm_wait<kWait>();                         // this wave's part of stage kt + 1 has landed
        asm volatile("s_barrier" ::: "memory");  // every wave's; no wave reads stage kt any more
        __builtin_amdgcn_sched_barrier(0);
        d = 0;
        if constexpr (kPrio) __builtin_amdgcn_s_setprio(2);
        if constexpr (A) {
#pragma unroll
          for (int i = 0; i < T16N; ++i) rd_w(0, kt + 1, 0, i);
          __builtin_amdgcn_sched_barrier(0);
          constexpr int gx = (NM16 - NQ + PX - 1) / PX;
          int m = 0;
#pragma unroll
          for (int j = 0; j < T16M; ++j) {
#pragma unroll
            for (int i = 0; i < T16N; ++i) {
              if (!pre(i, j)) {
                mf(1, i, j);
                if (d < PX && m % gx == gx - 1) dma_x(kt + NST, d++);
                ++m;
              }
              if (i == T16N - 1) rd_x(kt + 1, 0, j);
              __builtin_amdgcn_sched_barrier(0);
            }
          }
        }
#pragma unroll
        for (; d < PX; ++d) dma_x(kt + NST, d);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
    };
    if (rm < rows_m)
      main16(std::true_type{});
    else
      main16(std::false_type{});
    vm_wait<0>();  // the trailing zero-fill DMAs must land before the block's LDS is reused

    auto visit = [&](auto&& f) { visit_acc16<EPI, WTM, WTN, T16N, T16M>(a16, wm, wn, lane, f); };
    if (epi_rounds_first<EPI>(p, tc))
      store_tile_lds_bf16<BM, BN_OUT, EPI, NW, kRing * 2>(p, tc, visit, smem);
    else if constexpr (EPI == kEpiStore || EPI == kEpiStoreF32)
      store_tile_lds<BM, BN_OUT, EPI, NW, kRing * 2>(p, tc, visit, reinterpret_cast<float*>(smem));
  } else {
  WaveAcc<TN, TM> acc;
  acc.zero();
  const int l32 = lane & 31, h = lane >> 5;
  const int rn = wn * WTN, rm = wm * WTM;
  // A grouped tile's wave with fewer than WTM rows (an expert's last m-tile) runs the
  // partial form (active_c == 2): the MFMAs of its 32-row blocks past the rows are
  // skipped by uniform branches; the others run in the same order as in a full tile.
  const int nact = __builtin_amdgcn_readfirstlane(min(TM, max(0, (rows_m - rm + 31) / 32)));
  bf16x8 fa[2][TN], fb[2][TM];
  // ACTIVE: the wave's m-range holds rows of the tile. A wave without rows still
  // issues its share of the DMAs and joins every barrier, but reads no fragments
  // and issues no MFMAs (its accumulators stay zero and are never stored).
  auto read = [&](auto active_c, int buf, int kt, int ks) {
    if constexpr (!decltype(active_c)::value) return;
    const bf16* sx = smem + (kt % NST) * kStageX;
    const bf16* sw = smem + NST * kStageX + (kt % NSTW) * kStageW;
    const int c = ks * 2 + h;
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const int r = rn + i * 32 + l32;
      fa[buf][i] = *reinterpret_cast<const bf16x8*>(sw + r * BKT + ((c ^ dma_swz<BKT>(r)) << 3));
    }
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int r = rm + j * 32 + l32;
      fb[buf][j] = *reinterpret_cast<const bf16x8*>(sx + r * BKT + ((c ^ dma_swz<BKT>(r)) << 3));
    }
  };
  auto mma = [&](auto active_c, int buf) {
    if constexpr (!decltype(active_c)::value) return;
    constexpr bool kPart = decltype(active_c)::value == 2;
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j)
        if (!kPart || j < nact) acc.c[i][j] = mfma32x32x16(fa[buf][i], fb[buf][j], acc.c[i][j]);
  };
  // The stage's last k16 step with the next DMAs spread between its MFMAs
  // (one DMA after each MFMA, order pinned), so the matrix core is not idle
  // while a burst of DMA instructions issues after the barrier.
  auto last_step = [&](auto active_c, int buf, int kt) {  // issues the group of stage kt: X(kt + NST), W(kt + NSTW)
    constexpr bool kActive = decltype(active_c)::value;
    constexpr bool kPart = decltype(active_c)::value == 2;
    constexpr int ND = PX + PW;
    const int kx = (kt + NST) * BKT + dc * 8, kw = (kt + NSTW) * BKT + dc * 8;
    const uint32_t sbx = xslot(kt + NST), sbw = wslot(kt + NSTW);
    uint32_t doff[ND], dlds[ND];
#pragma unroll
    for (int i = 0; i < PX; ++i) {
      doff[i] = (kx < K && xoff[i] != kOOB) ? xoff[i] + (uint32_t)kx * 2u : kOOB;
      dlds[i] = sbx + (uint32_t)((wave + NW * i) * 1024);
    }
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      doff[PX + i] = (kw < K && woff[i] != kOOB) ? woff[i] + (uint32_t)kw * 2u : kOOB;
      dlds[PX + i] = sbw + (uint32_t)((wave + NW * i) * 1024);
    }
    auto dma = [&](int d) {
      if (d < PX)
        dma16(rx, doff[d], dlds[d]);
      else
        dma16(make_rsrc(wsrc[d - PX], (int64_t)wrows[d - PX] * ldw * 2), doff[d], dlds[d]);
    };
    __builtin_amdgcn_sched_barrier(0);
    int d = 0;
    if constexpr (kActive) {
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) {
          if (!kPart || j < nact) acc.c[i][j] = mfma32x32x16(fa[buf][i], fb[buf][j], acc.c[i][j]);
          if (d < ND) dma(d++);
          __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (; d < ND; ++d) dma(d);
  };
  auto interleave = [&]() {
    constexpr int NR = TN + TM, NM = TN * TM;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
  };

  // Spread schedule (W ring one slot deeper than the X ring). A stage's DMA
  // group is 64 KB at 256x256: issued within one K step it outruns the
  // texture path, and a wave whose next instruction is a DMA that cannot
  // issue stalls the MFMAs behind it. So stage j issues W(j + NST) during its
  // first K steps, into the W slot stage j - 1 released (its barrier is
  // behind us; the slot is next read in stage j + NST, so W keeps NST - 1
  // stages and a half of lead), and only X(j + NST) in its last step. Issue
  // order per wave: W(j + NST) then X(j + NST), stage by stage, so vmcnt
  // bookkeeping is that of the burst schedule: at stage kt's barrier X(kt + 1)
  // has landed once NST - 2 whole groups and W(kt + NST) remain, which is
  // kWait. Same MFMA order, same results.
  constexpr bool kSpreadW = NSTW == NST + 1;
  constexpr int kWSteps = KS - 1 < 2 ? KS - 1 : 2;  // K steps that carry W DMAs
  static_assert(!kSpreadW || kWSteps >= 1, "the spread schedule needs two K steps per stage");
  auto dma_w = [&](int kw, int i) {
    const int k = kw * BKT + dc * 8;
    const uint32_t off = (k < K && woff[i] != kOOB) ? woff[i] + (uint32_t)k * 2u : kOOB;
    dma16(make_rsrc(wsrc[i], (int64_t)wrows[i] * ldw * 2), off, wslot(kw) + (uint32_t)((wave + NW * i) * 1024));
  };
  auto read_one = [&](int buf, int kt, int ks, int f) {
    const int c = ks * 2 + h;
    if (f < TN) {
      const bf16* sw = smem + NST * kStageX + (kt % NSTW) * kStageW;
      const int r = rn + f * 32 + l32;
      fa[buf][f] = *reinterpret_cast<const bf16x8*>(sw + r * BKT + ((c ^ dma_swz<BKT>(r)) << 3));
    } else {
      const bf16* sx = smem + (kt % NST) * kStageX;
      const int r = rm + (f - TN) * 32 + l32;
      fb[buf][f - TN] = *reinterpret_cast<const bf16x8*>(sx + r * BKT + ((c ^ dma_swz<BKT>(r)) << 3));
    }
  };
  // K step ks of stage kt: its MFMAs, the fragment reads of step ks + 1
  // (one after each of the first TN + TM MFMAs) and this step's share of
  // W(kt + NST), evenly between the MFMAs; order pinned.
  auto step_w = [&](auto active_c, int buf, int kt, int ks) {
    constexpr bool kActive = decltype(active_c)::value;
    constexpr bool kPart = decltype(active_c)::value == 2;
    constexpr int NR = TN + TM, NM = TN * TM;
    const int d0 = ks * PW / kWSteps, d1 = (ks + 1) * PW / kWSteps;
    const int nd = d1 - d0;
    const int gap = nd > 0 ? (NM + nd - 1) / nd : NM + 1;
    int d = d0;
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kActive) {
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        if (!kPart || m % TM < nact)
          acc.c[m / TM][m % TM] = mfma32x32x16(fa[buf][m / TM], fb[buf][m % TM], acc.c[m / TM][m % TM]);
        if (m < NR) read_one(buf ^ 1, kt, ks + 1, m);
        if (d < d1 && m % gap == gap - 1) dma_w(kt + NST, d++);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (; d < d1; ++d) dma_w(kt + NST, d);
    __builtin_amdgcn_sched_barrier(0);
  };
  // The last K step of stage kt, which also crosses the stage's barrier. Its
  // MFMAs run in diagonal order, so the first NQ = max(TN, TM) of them use
  // every fragment of the step: once they have issued, this wave has no read
  // of stage kt's slots in flight (their results are in registers). Then the
  // wave waits for its own part of stage kt + 1 (vmcnt) and meets the other
  // waves at a plain s_barrier; no lgkmcnt(0) drain is needed before it, and
  // the MFMAs already issued keep the matrix core busy across the barrier.
  // After it: the reads of stage kt + 1's first step and X(kt + NST) (into
  // the X slot stage kt released) between the remaining MFMAs. Each
  // accumulator still takes exactly one MFMA per step: same results.
  auto last_step_x = [&](auto active_c, int buf, int kt) {
    constexpr bool kActive = decltype(active_c)::value;
    constexpr bool kPart = decltype(active_c)::value == 2;
    constexpr int NM = TN * TM, NR = TN + TM;
    constexpr int NQ = TN > TM ? TN : TM;
    const int kx = (kt + NST) * BKT + dc * 8;
    const uint32_t sbx = xslot(kt + NST);
    uint32_t doff[PX];
#pragma unroll
    for (int i = 0; i < PX; ++i) doff[i] = (kx < K && xoff[i] != kOOB) ? xoff[i] + (uint32_t)kx * 2u : kOOB;
    // q-th MFMA of the step: diagonal q / NQ, position q % NQ along the longer side.
    auto mfma_q = [&](int q) {
      const int a = q % NQ, dg = q / NQ;
      const int i = TN >= TM ? a : (a + dg) % TN;
      const int j = TN >= TM ? (a + dg) % TM : a;
      if (!kPart || j < nact) acc.c[i][j] = mfma32x32x16(fa[buf][i], fb[buf][j], acc.c[i][j]);
    };
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kActive) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        mfma_q(q);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    vm_wait<kWait>();                         // this wave's part of stage kt + 1 has landed
    asm volatile("s_barrier" ::: "memory");  // every wave's; no wave reads stage kt any more
    __builtin_amdgcn_sched_barrier(0);
    constexpr int NAFT = NM - NQ;
    constexpr int gap = NAFT >= PX ? NAFT / PX : 1;
    int d = 0;
    if constexpr (kActive) {
      // all of stage kt + 1's first-step reads at once, so the remaining
      // MFMAs of this step cover their latency
#pragma unroll
      for (int r = 0; r < NR; ++r) read_one(buf ^ 1, kt + 1, 0, r);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = NQ; q < NM; ++q) {
        mfma_q(q);
        if (d < PX && (q - NQ) % gap == gap - 1) {
          dma16(rx, doff[d], sbx + (uint32_t)((wave + NW * d) * 1024));
          ++d;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (; d < PX; ++d) dma16(rx, doff[d], sbx + (uint32_t)((wave + NW * d) * 1024));
    __builtin_amdgcn_sched_barrier(0);
  };

  if constexpr (kSpreadW) {
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      issue_w(j);
      issue_x(j);
    }
    vm_wait<(NST - 1) * (PX + PW)>();  // stage 0 has landed
    __syncthreads();
  } else {
#pragma unroll
    for (int j = -NSTW; j <= -2; ++j) issue_group(j);
    vm_wait<kWait>();  // stage 0 has landed
    __syncthreads();
    issue_group(-1);
  }
  auto main_loop = [&](auto active_c) {
    read(active_c, 0, 0, 0);
    for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) {
          if constexpr (kSpreadW) {
            if (ks < kWSteps) {
              step_w(active_c, ks & 1, kt, ks);
              continue;
            }
          }
          read(active_c, (ks + 1) & 1, kt, ks + 1);
          mma(active_c, ks & 1);
          if constexpr (decltype(active_c)::value == 1) interleave();
        } else if constexpr (kSpreadW) {
          last_step_x(active_c, ks & 1, kt);  // crosses the barrier; X(kt + NST) into the slot stage kt released
        } else {
          vm_wait<kWait>();                   // this wave's part of stage kt + 1 has landed
          __syncthreads();                    // every wave's; nobody reads stage kt any more
          read(active_c, (ks + 1) & 1, kt + 1, 0);
          last_step(active_c, ks & 1, kt);    // MFMAs with stage kt's DMA group (into the slots it released) between them
        }
      }
    }
  };
  if (rm >= rows_m)
    main_loop(std::false_type{});
  else if constexpr (GROUPED) {
    if (nact < TM)
      main_loop(std::integral_constant<int, 2>{});
    else
      main_loop(std::true_type{});
  } else
    main_loop(std::true_type{});
  vm_wait<0>();  // the trailing zero-fill DMAs must land before the block's LDS is reused

  auto visit = [&](auto&& f) { visit_acc32<EPI, WTM, WTN, TN, TM>(acc.c, wm, wn, lane, f); };
  if (epi_rounds_first<EPI>(p, tc))
    store_tile_lds_bf16<BM, BN_OUT, EPI, NW, kRing * 2>(p, tc, visit, smem);
  else if constexpr (EPI == kEpiStore || EPI == kEpiStoreF32)
    store_tile_lds<BM, BN_OUT, EPI, NW, kRing * 2>(p, tc, visit, reinterpret_cast<float*>(smem));
  }  // 32x32x16 loop
}

}  // namespace q3
