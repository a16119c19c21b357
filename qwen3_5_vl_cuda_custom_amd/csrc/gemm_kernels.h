// MFMA GEMM kernels (dense, batched, dual-B SwiGLU, MoE-grouped) built on the
// tile core in gemm_tile.h. Host launchers live in gemm.hip and moe.hip.
#pragma once

#include "gemm_tile.h"

namespace q3 {

enum Epilogue : int {
  kEpiStore = 0,     // C = acc (+ bias[n]) (+ R[m, n]), rounded once
  kEpiSwiGLU = 1,    // C = silu(acc_gate) * acc_up, rounded once
  kEpiRowScale = 2,  // C = bf16(bf16(acc) * s[m])  (MoE expert output x routing weight)
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
    const int tt = blockIdx.x / n_tiles_n;
    tile_n = blockIdx.x % n_tiles_n;
    if (tt >= *p.n_tiles_total) return false;
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
    C += z * p.bsC;
  }
  const int rows_m = m_end - m_begin;
  const int n0_out = tile_n * BN_OUT;
  // Stacked weights: a tile never straddles segments (the host checks that
  // every segment start is a multiple of BN). W and bias are re-based so that
  // output column n still addresses row n.
  int n_lim = p.N;
  const bf16* bias = p.bias;
  if constexpr (!GROUPED && EPI == kEpiStore) {
    if (p.seg.n > 1) {
      // Constant-index selects keep the segment's pointers in scalar registers
      // (a dynamic index into the by-value params would go through memory and
      // make the buffer resource per-lane).
      // Each field passes through readfirstlane before the select, so the
      // selects cannot be folded back into one dynamically indexed load.
      const int s = __builtin_amdgcn_readfirstlane(segment_of(p.seg, n0_out));
      const bf16* sw = pick4(s, uniform_ptr(p.seg.w[0]), uniform_ptr(p.seg.w[1]), uniform_ptr(p.seg.w[2]),
                             uniform_ptr(p.seg.w[3]));
      const bf16* sb = pick4(s, uniform_ptr(p.seg.b[0]), uniform_ptr(p.seg.b[1]), uniform_ptr(p.seg.b[2]),
                             uniform_ptr(p.seg.b[3]));
      const int st0 = pick4(s, __builtin_amdgcn_readfirstlane(p.seg.start[0]),
                            __builtin_amdgcn_readfirstlane(p.seg.start[1]),
                            __builtin_amdgcn_readfirstlane(p.seg.start[2]),
                            __builtin_amdgcn_readfirstlane(p.seg.start[3]));
      const int nxt = pick4(s, __builtin_amdgcn_readfirstlane(p.seg.start[1]),
                            __builtin_amdgcn_readfirstlane(p.seg.start[2]),
                            __builtin_amdgcn_readfirstlane(p.seg.start[3]), p.N);
      W = uniform_ptr(sw - (int64_t)st0 * p.ldw);
      bias = sb ? uniform_ptr(sb - st0) : nullptr;
      n_lim = s + 1 < p.seg.n ? nxt : p.N;
    }
  }

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

// Epilogue of one wave's (TN x TM) 32x32 accumulator tiles at wave offset
// (wm * WTM, wn * WTN) of the block tile.
template <int WTM, int WTN, int TN, int TM, int EPI>
__device__ __forceinline__ void store_tile(const GemmParams& p, const TileCtx& t, const floatx16 (&c)[TN][TM],
                                           int wm, int wn, int lane) {
  const int m_begin = t.m_begin, rows_m = t.rows_m, n0_out = t.n0_out;
  const bf16* bias = t.bias;
  bf16* C = t.C;
  const int l32 = lane & 31;
  const int h = lane >> 5;
  const int N = p.N;
  const bool vec_ok = ((p.ldc & 3) == 0) && (p.R == nullptr || (p.ldr & 3) == 0);

  if constexpr (EPI == kEpiSwiGLU) {
#pragma unroll
    for (int i = 0; i < TN / 2; ++i) {
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int mr = wm * WTM + j * 32 + l32;
        if (mr >= rows_m) continue;
        bf16* crow = C + (int64_t)(m_begin + mr) * p.ldc;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0_out + (wn * WTN) / 2 + i * 32 + 8 * g + 4 * h;
          float o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gt = c[2 * i][j][4 * g + q];
            const float up = c[2 * i + 1][j][4 * g + q];
            o[q] = gt / (1.0f + __expf(-gt)) * up;
          }
          if (vec_ok && n + 3 < N) {
            bf16x4 v = {f2bf(o[0]), f2bf(o[1]), f2bf(o[2]), f2bf(o[3])};
            *reinterpret_cast<bf16x4*>(crow + n) = v;
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (n + q < N) crow[n + q] = f2bf(o[q]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // one accumulator tile live at a time
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < TN; ++i) {
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int mr = wm * WTM + j * 32 + l32;
        if (mr >= rows_m) continue;
        const int m = m_begin + mr;
        bf16* crow = C + (int64_t)m * p.ldc;
        float rs = 1.0f;
        if constexpr (EPI == kEpiRowScale) rs = bf2f(p.rowscale[m]);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0_out + wn * WTN + i * 32 + 8 * g + 4 * h;
          float o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) o[q] = c[i][j][4 * g + q];
          if (vec_ok && n + 3 < N) {
            if (bias) {
              const bf16x4 b = *reinterpret_cast<const bf16x4*>(bias + n);
#pragma unroll
              for (int q = 0; q < 4; ++q) o[q] += bf2f(b[q]);
            }
            if (p.R) {
              const bf16x4 rv = *reinterpret_cast<const bf16x4*>(p.R + (int64_t)m * p.ldr + n);
#pragma unroll
              for (int q = 0; q < 4; ++q) o[q] += bf2f(rv[q]);
            }
            if constexpr (EPI == kEpiRowScale) {
#pragma unroll
              for (int q = 0; q < 4; ++q) o[q] = bf2f(f2bf(o[q])) * rs;
            }
            bf16x4 v = {f2bf(o[0]), f2bf(o[1]), f2bf(o[2]), f2bf(o[3])};
            *reinterpret_cast<bf16x4*>(crow + n) = v;
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if (n + q >= N) continue;
              float v = o[q];
              if (bias) v += bf2f(bias[n + q]);
              if (p.R) v += bf2f(p.R[(int64_t)m * p.ldr + n + q]);
              if constexpr (EPI == kEpiRowScale) v = bf2f(f2bf(v)) * rs;
              crow[n + q] = f2bf(v);
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // one accumulator tile live at a time
      }
    }
  }
}

// Instruction order for one phase of the register-staged loop (one stage of
// MFMAs, the next stage's global loads and the previous stage's LDS stores):
// all fragment reads first, then the global loads and LDS stores spread
// between MFMAs, so neither the memory pipes nor the MFMA pipe idle.
template <int BK, int TN, int TM, int NV>
__device__ __forceinline__ void sched_phase() {
  constexpr int NR = (BK / 16) * (TN + TM), NM = (BK / 16) * TN * TM;
  static_assert(NM >= 2 * NV, "not enough MFMAs to interleave the memory operations");
  __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);  // DS reads
#pragma unroll
  for (int r = 0; r < NV; ++r) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
  }
  __builtin_amdgcn_sched_group_barrier(0x008, NM - 2 * NV, 0);
}

template <int BM, int BN, int WM, int WN, int EPI, bool GROUPED>
__global__ __launch_bounds__(WM* WN * 64) void gemm_bf16_kernel(const GemmParams p) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM;
  constexpr int WTN = BN / WN;
  constexpr int TM = WTM / 32;
  constexpr int TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile too small");
  static_assert(EPI != kEpiSwiGLU || (TN % 2 == 0), "SwiGLU pairs gate/up tiles");
  constexpr int BN_OUT = (EPI == kEpiSwiGLU) ? BN / 2 : BN;

  __shared__ __attribute__((aligned(16))) bf16 smem[2 * (BM + BN) * kBK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int wm = wave % WM;
  const int wn = wave / WM;

  TileCtx tc;
  if (!tile_ctx<BM, BN_OUT, EPI, GROUPED>(p, tc)) return;
  const int m_begin = tc.m_begin, rows_m = tc.rows_m, n0_out = tc.n0_out, n_lim = tc.n_lim;
  const bf16* X = tc.X;
  const bf16* W = tc.W;
  const bf16* W2 = tc.W2;

  constexpr int kStage = (BM + BN) * kBK;
  // Register staging: thread t owns 16-byte chunks t + i*NT of the X tile
  // (PX of them) and of the W tile (PW).
  constexpr int PX = BM * kChunks / NT;
  constexpr int PW = BN * kChunks / NT;
  static_assert(BM * kChunks % NT == 0 && BN * kChunks % NT == 0, "tile not divisible by threads");

  const int K = p.K;
  const int nk = (K + kBK - 1) / kBK;
  const int64_t ldx = p.ldx, ldw = p.ldw;

  // Per chunk: byte offset of its global row (kOOB: no such row) and its K chunk.
  uint32_t xoff[PX], woff[PW];
#pragma unroll
  for (int i = 0; i < PX; ++i) {
    const int r = (tid + i * NT) / kChunks;
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
    const int r = (tid + i * NT) / kChunks;
    int n;
    if constexpr (EPI == kEpiSwiGLU) {
      n = n0_out + (r >> 6) * 32 + (r & 31);  // 32-row groups alternate gate / up
    } else {
      n = n0_out + r;
    }
    woff[i] = n < n_lim ? (uint32_t)((int64_t)n * ldw * 2) : kOOB;
  }
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(X, p.gather ? (int64_t)p.M_src * ldx * 2 : (int64_t)(m_begin + rows_m) * ldx * 2);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(W, (int64_t)n_lim * ldw * 2);
  const __amdgpu_buffer_rsrc_t rw2 = make_rsrc(EPI == kEpiSwiGLU ? W2 : W, (int64_t)p.N * ldw * 2);

  struct Stage {
    bf16x8 x[PX], w[PW];
  };
  // Loads of K-stage kt (zeros past the end: offsets resolve out of range).
  auto load = [&](Stage& st, int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < PX; ++i) {
      const int k = k0 + ((tid + i * NT) % kChunks) * 8;
      st.x[i] = buffer_load16(rx, (k < K && xoff[i] != kOOB) ? xoff[i] + (uint32_t)k * 2u : kOOB);
    }
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int id = tid + i * NT;
      const int k = k0 + (id % kChunks) * 8;
      const uint32_t off = (k < K && woff[i] != kOOB) ? woff[i] + (uint32_t)k * 2u : kOOB;
      if constexpr (EPI == kEpiSwiGLU) {
        // The 64 chunks of a wave lie in 16 consecutive rows, all of one
        // 32-row gate or up group: the choice is wave-uniform, so the buffer
        // resource stays scalar (no per-lane selection loop).
        const bool up = (((wave * 64 + i * NT) / kChunks) >> 5) & 1;
        st.w[i] = buffer_load16(up ? rw2 : rw, off);
      } else {
        st.w[i] = buffer_load16(rw, off);
      }
    }
  };
  auto store = [&](const Stage& st, int slot) {
    bf16* sx = smem + slot * kStage;
    bf16* sw = sx + BM * kBK;
#pragma unroll
    for (int i = 0; i < PX; ++i) {
      const int id = tid + i * NT;
      *reinterpret_cast<bf16x8*>(sx + swz(id / kChunks, id % kChunks)) = st.x[i];
    }
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int id = tid + i * NT;
      *reinterpret_cast<bf16x8*>(sw + swz(id / kChunks, id % kChunks)) = st.w[i];
    }
  };
  auto compute = [&](auto& acc, int slot) {
    const bf16* sx = smem + slot * kStage;
    acc.mma_stage(sx, sx + BM * kBK, wm * WTM, wn * WTN, lane);
  };

  WaveAcc<TN, TM> acc;
  acc.zero();

  // Two register stages in flight (prefetch distance 2): the loads of stage
  // kt+2 are issued before the MFMAs of stage kt, and stage kt+1 (issued one
  // phase earlier) is written to LDS after them.
  Stage sa, sb;
  load(sa, 0);
  load(sb, 1);
  store(sa, 0);
  __syncthreads();
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {  // slot 0 holds stage kt, sb stage kt+1 (in flight)
    load(sa, kt + 2);
    compute(acc, 0);
    store(sb, 1);
    sched_phase<kBK, TN, TM, PX + PW>();
    __syncthreads();
    load(sb, kt + 3);
    compute(acc, 1);
    store(sa, 0);
    sched_phase<kBK, TN, TM, PX + PW>();
    __syncthreads();
  }
  if (kt < nk) compute(acc, 0);  // odd number of stages: the last one is in slot 0

  store_tile<WTM, WTN, TN, TM, EPI>(p, tc, acc.c, wm, wn, lane);
}

}  // namespace q3
