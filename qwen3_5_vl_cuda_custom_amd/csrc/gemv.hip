// Weight-streaming GEMV for decode-shaped GEMMs (M <= 32 activation rows):
//
//   C[m, n] = sum_k X[m, k] * W[n, k] (+ bias[n]) (+ R[m, n])      plain
//   C[m, n] = silu(X . Wg[n]) * (X . Wu[n])                        SwiGLU
//
// At M <= 32 the GEMM moves N*K*2 bytes of weights for 2*M*N*K FLOP, so it is
// bound by HBM and the kernel is built to keep the weight stream at full rate:
//
//  * Work units are (tile, k-stage) pairs: a tile is 128 weight rows (plain:
//    128 output columns; SwiGLU: 32-row gate / up groups alternating, 64
//    output columns), a stage is 64 k (128 bytes of every row). One block
//    runs per CU and takes an equal contiguous range of the tile-major unit
//    order (stream-K), so every CU streams the same number of bytes whatever
//    N and K are.
//  * A stage (128 weight rows + the 32 X rows) goes global -> LDS with
//    buffer_load ... lds; a 4-stage ring keeps three stages in flight while
//    the MFMAs (v_mfma_f32_32x32x16_bf16, W rows as A, X rows as B) consume
//    the fourth. One DMA instruction fills 8 rows x 128 bytes; the lane that
//    lands at slot s of row r fetches chunk s ^ swz(r), so fragment reads are
//    bank-conflict free.
//  * A tile that lies inside one block's range is finished in that block. A
//    tile split between blocks is summed by the block that contributes its
//    last piece: each block writes its fp32 piece with device-coherent stores,
//    and bumps the tile's counter only once its own pipeline waits have shown
//    those stores complete (vmcnt retires in order, so the wait for a later
//    stage's DMA covers them); the counter's return values are read after the
//    loop, and the block that completes a count sums the pieces in piece
//    order (deterministic) and resets the counter to zero.
//
// The split-K reduction above costs a few microseconds of dependent memory
// round trips at the end of every call (piece stores, counter atomics, the
// last block's piece loads). Where that outweighs what split-K saves, a
// row-owned kernel runs instead: each block owns r consecutive weight rows of
// one segment over all of K, so nothing leaves the block before the epilogue:
//  * r is the smallest row count that gives every CU at most one block; the
//    rows form 16-row groups of v_mfma_f32_16x16x32_bf16 (W as A, X as B),
//    rows past r load as zeros (out-of-range offsets: no memory traffic).
//  * gemv_rows_dma_kernel (every plain form, and the fused norm up to K =
//    8192): weights and X rows go global -> LDS by direct-to-LDS loads in
//    whole row pieces through a ring of k-stages, one barrier per stage.
//  * gemv_rows_kernel (the fused norm beyond K = 8192): W straight into VGPRs
//    D k-steps (of 32) ahead of its MFMAs; X staged per 512-k chunk through
//    LDS in whole 1 KB row pieces (the L2 serves those ~3x faster per CU than
//    16-row fragment reads).
//  * The waves take the k-steps round robin and sum their fp32 partials
//    through LDS in wave order (deterministic); the epilogue adds bias and
//    residual or applies SwiGLU and rounds once.
#include "gemv.h"

namespace q3 {
namespace {

constexpr int kGvBK = 64;                     // k per stage
constexpr int kGvBN = 128;                    // weight rows per tile
constexpr int kGvRows = kGvBN + 32;           // rows per stage: W tile + X
constexpr int kGvStage = kGvRows * kGvBK;     // elements per stage
constexpr int kGvPerWave = kGvRows / 8 / 4;   // DMA instructions per wave per stage
constexpr int kGvStages = 4;                  // LDS ring depth
constexpr int kGvGrid = 256;                  // one block per CU (MI355X)
constexpr int kGvPiece = 32 * kGvBN;          // floats per partial piece: [m 32][tile row 128]
// The workspace starts with a counter region of fixed size, so calls of any
// shape that share a workspace never write partials over another shape's
// counters.
constexpr int kGvMaxTiles = 4096;
constexpr int64_t kGvCounterBytes = kGvMaxTiles * 4;

struct GemvParams {
  GemvArgs a;
  int* counters;
  float* partial;
  int n_tiles, k_stages, total, grid, max_pieces;
  int vec4, vec8;  // C (and R) rows allow 8-byte / 16-byte vector access
};

__device__ __forceinline__ int gv_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Block whose unit range [b*total/G, (b+1)*total/G) contains unit u.
__host__ __device__ inline int gv_block_of(int64_t u, int G, int64_t total) {
  return (int)(((u + 1) * G - 1) / total);
}

// Wave-uniform weight source of the plain tile starting at output column col.
struct SegPick {
  const bf16* w;
  const bf16* b;
  int start, end;
};
__device__ __forceinline__ SegPick seg_pick(const WeightSegments& sg, int N, int col) {
  const int s = __builtin_amdgcn_readfirstlane(segment_of(sg, col));
  SegPick r;
  r.w = pick4(s, uniform_ptr(sg.w[0]), uniform_ptr(sg.w[1]), uniform_ptr(sg.w[2]), uniform_ptr(sg.w[3]));
  r.b = pick4(s, uniform_ptr(sg.b[0]), uniform_ptr(sg.b[1]), uniform_ptr(sg.b[2]), uniform_ptr(sg.b[3]));
  r.start = pick4(s, __builtin_amdgcn_readfirstlane(sg.start[0]), __builtin_amdgcn_readfirstlane(sg.start[1]),
                  __builtin_amdgcn_readfirstlane(sg.start[2]), __builtin_amdgcn_readfirstlane(sg.start[3]));
  const int nxt = pick4(s, __builtin_amdgcn_readfirstlane(sg.start[1]), __builtin_amdgcn_readfirstlane(sg.start[2]),
                        __builtin_amdgcn_readfirstlane(sg.start[3]), N);
  r.end = s + 1 < sg.n ? nxt : N;
  return r;
}

template <bool SWIGLU>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvParams p) {
  constexpr int NST = kGvStages;
  __shared__ __attribute__((aligned(1024))) bf16 ring[NST * kGvStage];
  __shared__ float xbuf[2][32 * 33];  // SwiGLU: up accumulators handed to the gate waves
  __shared__ int s_last[2];

  const GemvArgs& a = p.a;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  const int G = p.grid, b = blockIdx.x;
  const int64_t total = p.total;
  const int u0 = (int)((int64_t)b * total / G), u1 = (int)((int64_t)(b + 1) * total / G);
  const int KS = p.k_stages, K = a.K, N = a.N, M = a.M;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.X, (int64_t)M * a.ldx * 2);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(a.seg.w[0], (int64_t)N * a.ldw * 2);           // SwiGLU gate
  const __amdgpu_buffer_rsrc_t ru = make_rsrc(SWIGLU ? a.W2 : a.seg.w[0], (int64_t)N * a.ldw * 2);  // SwiGLU up
  const uint32_t lbase = lds_addr(ring);

  // DMA of unit u's stage into ring slot u % NST (zeros past the range).
  auto issue = [&](int u) {
    const bool live = u < u1;
    const int t = u / KS;
    const int k0 = (u - t * KS) * kGvBK;
    const uint32_t sbase = lbase + (uint32_t)((u % NST) * kGvStage * 2);
    __amdgpu_buffer_rsrc_t rw = rg;
    int rowbase = 0, lim = 0;
    if constexpr (!SWIGLU) {
      const SegPick sp = seg_pick(a.seg, N, t * kGvBN);
      rw = make_rsrc(sp.w, (int64_t)(sp.end - sp.start) * a.ldw * 2);
      rowbase = t * kGvBN - sp.start;
      lim = sp.end - t * kGvBN;
    }
#pragma unroll
    for (int i = 0; i < kGvPerWave; ++i) {
      const int j = wave + 4 * i;  // stage rows 8j .. 8j+7
      const int r = 8 * j + (lane >> 3);
      const int k = k0 + 8 * ((lane & 7) ^ gv_swz(r));
      const uint32_t dst = sbase + (uint32_t)(j * 1024);
      if (i < 4) {  // weight rows
        if constexpr (SWIGLU) {
          const int grp = j >> 2;
          const int n = t * 64 + (grp >> 1) * 32 + (r & 31);
          const uint32_t off = (live && n < N && k < K) ? (uint32_t)(((int64_t)n * a.ldw + k) * 2) : kOOB;
          dma16_nt((grp & 1) ? ru : rg, off, dst);
        } else {
          const uint32_t off = (live && r < lim && k < K) ? (uint32_t)(((int64_t)(rowbase + r) * a.ldw + k) * 2) : kOOB;
          dma16_nt(rw, off, dst);
        }
      } else {  // X rows
        const int m = r - kGvBN;
        const uint32_t off = (live && m < M && k < K) ? (uint32_t)(((int64_t)m * a.ldx + k) * 2) : kOOB;
        dma16(rx, off, dst);
      }
    }
  };

  // Epilogue of a tile finished inside this block.
  auto store_whole = [&](int t, const floatx16& acc) {
    if constexpr (SWIGLU) {
      if (wave & 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) xbuf[wave >> 1][(8 * (r >> 2) + 4 * h + (r & 3)) * 33 + l32] = acc[r];
      }
      __syncthreads();
      if (!(wave & 1) && l32 < M) {
        bf16* crow = a.C + (int64_t)l32 * a.ldc;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int nn = 8 * g + 4 * h;
          const int n = t * 64 + (wave >> 1) * 32 + nn;
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = silu_mul(acc[4 * g + e], xbuf[wave >> 1][(nn + e) * 33 + l32]);
          if (p.vec4 && n + 3 < N) {
            *reinterpret_cast<bf16x4*>(crow + n) = bf16x4{f2bf(o[0]), f2bf(o[1]), f2bf(o[2]), f2bf(o[3])};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < N) crow[n + e] = f2bf(o[e]);
          }
        }
      }
      __syncthreads();
    } else {
      if (l32 >= M) return;
      const SegPick sp = seg_pick(a.seg, N, t * kGvBN);
      const bf16* bias = sp.b ? sp.b - sp.start : nullptr;
      bf16* crow = a.C + (int64_t)l32 * a.ldc;
      const bf16* rrow = a.R ? a.R + (int64_t)l32 * a.ldr : nullptr;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = t * kGvBN + 32 * wave + 8 * g + 4 * h;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = acc[4 * g + e];
        if (p.vec4 && n + 3 < N) {
          if (bias) {
            const bf16x4 bv = *reinterpret_cast<const bf16x4*>(bias + n);
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] += bf2f(bv[e]);
          }
          if (rrow) {
            const bf16x4 rv = *reinterpret_cast<const bf16x4*>(rrow + n);
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] += bf2f(rv[e]);
          }
          *reinterpret_cast<bf16x4*>(crow + n) = bf16x4{f2bf(o[0]), f2bf(o[1]), f2bf(o[2]), f2bf(o[3])};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (n + e >= N) continue;
            float v = o[e];
            if (bias) v += bf2f(bias[n + e]);
            if (rrow) v += bf2f(rrow[n + e]);
            crow[n + e] = f2bf(v);
          }
        }
      }
    }
  };

  // Sum of a split tile's pieces (in piece order) and its epilogue.
  constexpr int kBatch = 8;
  auto reduce_tile = [&](int t, int npieces) {
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(p.partial + (int64_t)t * p.max_pieces * kGvPiece, (int64_t)p.max_pieces * kGvPiece * 4);
    const int m = tid >> 3;
    if constexpr (SWIGLU) {
      const int cc0 = (tid & 7) * 8;
      const int nng = (cc0 >> 5) * 64 + (cc0 & 31);
      // Pieces in batches of kBatch with all their loads in flight (pieces past
      // the count load as zeros), summed in piece order.
      floatx4 g0 = {}, g1 = {}, v0 = {}, v1 = {};
      for (int pc0 = 0; pc0 < npieces; pc0 += kBatch) {
        floatx4 ld[kBatch][4];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
          const uint32_t o =
              pc0 + i < npieces ? (uint32_t)(((pc0 + i) * kGvPiece + m * kGvBN + nng) * 4) : kOOB - 256;
          ld[i][0] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rp, o, 0, 0));
          ld[i][1] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rp, o + 16, 0, 0));
          ld[i][2] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rp, o + 128, 0, 0));
          ld[i][3] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rp, o + 144, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
          g0 += ld[i][0];
          g1 += ld[i][1];
          v0 += ld[i][2];
          v1 += ld[i][3];
        }
      }
      if (m >= M) return;
      const int n0 = t * 64 + cc0;
      float f[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[e] = silu_mul(g0[e], v0[e]);
        f[4 + e] = silu_mul(g1[e], v1[e]);
      }
      bf16* crow = a.C + (int64_t)m * a.ldc;
      if (p.vec8 && n0 + 7 < N) {
        *reinterpret_cast<bf16x8*>(crow + n0) = pack8(f);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n0 + e < N) crow[n0 + e] = f2bf(f[e]);
      }
    } else {
      const int nn0 = (tid & 7) * 16;
      floatx4 s[4] = {};
      for (int pc0 = 0; pc0 < npieces; pc0 += kBatch) {
        floatx4 ld[kBatch][4];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
          const uint32_t o =
              pc0 + i < npieces ? (uint32_t)(((pc0 + i) * kGvPiece + m * kGvBN + nn0) * 4) : kOOB - 256;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            ld[i][q] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rp, o + 16 * q, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) s[q] += ld[i][q];
      }
      if (m >= M) return;
      const int n0 = t * kGvBN + nn0;
      const SegPick sp = seg_pick(a.seg, N, t * kGvBN);
      const bf16* bias = sp.b ? sp.b - sp.start : nullptr;
      float f[16];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) f[4 * q + e] = s[q][e];
      bf16* crow = a.C + (int64_t)m * a.ldc;
      const bf16* rrow = a.R ? a.R + (int64_t)m * a.ldr : nullptr;
      if (p.vec8 && n0 + 15 < N) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          if (bias) {
            const bf16x8 bv = *reinterpret_cast<const bf16x8*>(bias + n0 + 8 * hh);
#pragma unroll
            for (int e = 0; e < 8; ++e) f[8 * hh + e] += bf2f(bv[e]);
          }
          if (rrow) {
            const bf16x8 rv = *reinterpret_cast<const bf16x8*>(rrow + n0 + 8 * hh);
#pragma unroll
            for (int e = 0; e < 8; ++e) f[8 * hh + e] += bf2f(rv[e]);
          }
          *reinterpret_cast<bf16x8*>(crow + n0 + 8 * hh) = pack8(f + 8 * hh);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          if (n0 + e >= N) continue;
          float v = f[e];
          if (bias) v += bf2f(bias[n0 + e]);
          if (rrow) v += bf2f(rrow[n0 + e]);
          crow[n0 + e] = f2bf(v);
        }
      }
    }
  };

  // Split tiles this block contributes to (at most its first and its last).
  int np_ = 0;
  int pt0 = 0, pt1 = 0, pn0 = 0, pn1 = 0;
  int old0 = 0, old1 = 0;  // counter values returned to thread 0
  auto bump = [&](int idx) {
    if (tid == 0) {
      const int v = __hip_atomic_fetch_add(&p.counters[idx == 0 ? pt0 : pt1], 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
      if (idx == 0) old0 = v;
      else old1 = v;
    }
  };

  floatx16 acc = floatx16{};
#pragma unroll
  for (int s = 0; s < NST - 1; ++s) issue(u0 + s);

  for (int u = u0; u < u1; ++u) {
    vm_wait<(NST - 2) * kGvPerWave>();  // this wave's DMAs of stage u have landed
    __syncthreads();                     // ... and every wave's; slot (u - 1) % NST is free
    issue(u + NST - 1);
    const bf16* st = ring + (u % NST) * kGvStage;
    const int ra = 32 * wave + l32, rb = kGvBN + l32;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = 2 * q + h;
      const bf16x8 fa = *reinterpret_cast<const bf16x8*>(st + ra * kGvBK + ((c ^ gv_swz(ra)) << 3));
      const bf16x8 fb = *reinterpret_cast<const bf16x8*>(st + rb * kGvBK + ((c ^ gv_swz(rb)) << 3));
      acc = mfma32x32x16(fa, fb, acc);
    }
    const int t = u / KS;
    if (u - t * KS == KS - 1 || u == u1 - 1) {
      if (t * KS >= u0 && t * KS + KS <= u1) {
        store_whole(t, acc);
      } else {
        const int fb = gv_block_of((int64_t)t * KS, G, total);
        const int lb = gv_block_of((int64_t)t * KS + KS - 1, G, total);
        const int piece = b - fb;
        const __amdgpu_buffer_rsrc_t rp =
            make_rsrc(p.partial + (int64_t)t * p.max_pieces * kGvPiece, (int64_t)p.max_pieces * kGvPiece * 4);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int nn = 32 * wave + 8 * g + 4 * h;
          const floatx4 v = {acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp,
                                                 (uint32_t)((piece * kGvPiece + l32 * kGvBN + nn) * 4), 0, 0);
        }
        if (np_ == 0) {
          pt0 = t;
          pn0 = lb - fb + 1;
        } else {
          pt1 = t;
          pn1 = lb - fb + 1;
        }
        ++np_;
      }
      acc = floatx16{};
    }
  }

  // Cross-block hand-off of a split tile: every thread's piece stores are
  // released at agent scope (the fence writes them back past this XCD's L2)
  // before the barrier, so they are visible device-wide before thread 0
  // counts the block's arrival; the block that brings a tile's count to its
  // piece total reads the pieces only after an agent-scope acquire fence
  // (which invalidates stale cached lines). The counters themselves are
  // device-scope atomics.
  __threadfence();
  __syncthreads();
  if (np_ > 0) bump(0);
  if (np_ > 1) bump(1);
  if (tid == 0) {
    s_last[0] = np_ > 0 && old0 == pn0 - 1;
    s_last[1] = np_ > 1 && old1 == pn1 - 1;
  }
  __syncthreads();
  if (s_last[0] || s_last[1]) __threadfence();
  if (s_last[0]) {
    reduce_tile(pt0, pn0);
    if (tid == 0) __hip_atomic_store(&p.counters[pt0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (s_last[1]) {
    reduce_tile(pt1, pn1);
    if (tid == 0) __hip_atomic_store(&p.counters[pt1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}


// ------------------------------------------------------------ row-owned GEMV
constexpr int kRowsDirectMaxM = 8;   // up to this many rows the row-owned kernels take any K
constexpr int kRowsMaxK = 16384;     // staged-X kernel beats stream-K up to here (M > 8)
constexpr int kRowsMaxRG = 4;        // at most 64 weight rows per block
constexpr int kRowsKC = 512;         // staged X: k per LDS chunk (1 KB of each X row)

struct RowsParams {
  GemvArgs a;
  int r;          // weight rows per block
  int bstart[5];  // first block of each segment; bstart[seg.n] = grid
  int vec4;       // C (and R, bias) allow 8-byte access at 4-aligned columns
};

// Epilogue of the row-owned kernels: red holds each wave's fp32 partials,
// [wave][row group][X tile][lane] (accumulator register e of lane l in group
// (q, t) is weight row 16 q + 4 (l / 16) + e, X row 16 t + l % 16); they are
// summed in wave order, scaled by the row's rstd (NORM: rsum[m] = sum of x^2
// of X row m), then SwiGLU or bias + residual, and rounded once.
template <int RG, int MT, bool SW, bool NORM, int NW, int NT>
__device__ __forceinline__ void rows_epilogue(const RowsParams& p, const floatx4* red, const float* rsum, int s,
                                              int n0, int rows, int cbase) {
  constexpr int RGT = SW ? 2 * RG : RG;
  const GemvArgs& a = p.a;
  const int tid = threadIdx.x, K = a.K, M = a.M;
  auto at = [&](int w, int q, int t, int l) { return red[((w * RGT + q) * MT + t) * 64 + l]; };
  const bf16* bias = SW ? nullptr : pick4(s, a.seg.b[0], a.seg.b[1], a.seg.b[2], a.seg.b[3]);
  for (int it = tid; it < RG * MT * 64; it += NT) {
    const int q = it / (MT * 64), t = (it / 64) % MT, l = it & 63;
    const int m = 16 * t + (l & 15);
    const int row = 16 * q + 4 * (l >> 4);
    if (m >= M || row >= rows) continue;
    floatx4 v = at(0, q, t, l);
#pragma unroll
    for (int w = 1; w < NW; ++w) v += at(w, q, t, l);
    float rstd = 1.f;
    if constexpr (NORM) rstd = rsqrtf(rsum[m] / (float)K + a.eps);
    if constexpr (NORM) v *= rstd;
    float o[4];
    if constexpr (SW) {
      floatx4 u = at(0, RG + q, t, l);
#pragma unroll
      for (int w = 1; w < NW; ++w) u += at(w, RG + q, t, l);
      if constexpr (NORM) u *= rstd;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = silu_mul(v[e], u[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = v[e];
    }
    const int n = cbase + row;  // output column
    bf16* crow = a.C + (int64_t)m * a.ldc;
    const bf16* rrow = a.R ? a.R + (int64_t)m * a.ldr : nullptr;
    if (p.vec4 && row + 3 < rows && (n & 3) == 0) {
      if (bias) {
        const bf16x4 bv = *reinterpret_cast<const bf16x4*>(bias + n0 + row);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] += bf2f(bv[e]);
      }
      if (rrow) {
        const bf16x4 rv = *reinterpret_cast<const bf16x4*>(rrow + n);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] += bf2f(rv[e]);
      }
      *reinterpret_cast<bf16x4*>(crow + n) = bf16x4{f2bf(o[0]), f2bf(o[1]), f2bf(o[2]), f2bf(o[3])};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (row + e >= rows) continue;
        float v2 = o[e];
        if (bias) v2 += bf2f(bias[n0 + row + e]);
        if (rrow) v2 += bf2f(rrow[n + e]);
        crow[n + e] = f2bf(v2);
      }
    }
  }
}

// Row-owned GEMV with the RMSNorm fused (the form for K past the DMA ring's
// LDS copy of the norm weight): W straight into a VGPR ring D k-steps ahead;
// X staged per 512-k chunk through LDS, RMS-normalised on its way in. The LDS
// copy holds bf16(x * w_norm); each staging lane keeps its rows' partial sums
// of x^2 over the K it loads; the epilogue scales each row's dot products by
// rsqrt(sum / K + eps), which equals projecting the normalised rows.
template <int RG, int MT, bool SW, int D>
__global__ __launch_bounds__(256) void gemv_rows_kernel(const RowsParams p) {
  constexpr int NW = 4;
  constexpr int RGT = SW ? 2 * RG : RG;
  constexpr int XR = 16 * MT;              // X rows of the MFMA B operand
  constexpr int XPW = XR / NW;             // staged X rows loaded per wave
  constexpr int SPC = kRowsKC / 32;        // k-steps per chunk
  constexpr int SPW = SPC / NW;            // k-steps per wave per chunk
  __shared__ __attribute__((aligned(1024))) bf16 xs[2][XR * kRowsKC];
  __shared__ floatx4 red[NW][RGT][MT][64];
  __shared__ float rsum[XR];  // sum of x^2 of each X row
  const GemvArgs& a = p.a;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int b = blockIdx.x;
  int s = 0;
#pragma unroll
  for (int j = 1; j < 4; ++j)
    if (j < a.seg.n && b >= p.bstart[j]) s = j;
  const int n0 = (b - p.bstart[s]) * p.r;  // first row of the block within segment s
  const int seg_start = pick4(s, a.seg.start[0], a.seg.start[1], a.seg.start[2], a.seg.start[3]);
  const int seg_end = s + 1 < a.seg.n ? pick4(s, a.seg.start[1], a.seg.start[2], a.seg.start[3], a.N) : a.N;
  const int rows = min(p.r, seg_end - seg_start - n0);
  const int K = a.K, M = a.M;
  const bf16* wb = uniform_ptr(pick4(s, a.seg.w[0], a.seg.w[1], a.seg.w[2], a.seg.w[3]) + (int64_t)n0 * a.ldw);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(wb, (int64_t)rows * a.ldw * 2);
  const __amdgpu_buffer_rsrc_t ru =
      SW ? make_rsrc(uniform_ptr(a.W2 + (int64_t)n0 * a.ldw), (int64_t)rows * a.ldw * 2) : rw;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.X, (int64_t)M * a.ldx * 2);
  uint32_t woff[RG];
#pragma unroll
  for (int q = 0; q < RG; ++q) woff[q] = 16 * q + i < rows ? (uint32_t)((16 * q + i) * a.ldw * 2) : kOOB;

  const int NC = (K + kRowsKC - 1) / kRowsKC;
  // Wave step j -> k-step: chunk j / SPW, in-chunk step wave + NW * (j % SPW)
  // (every wave has NC * SPW steps; those past K load zeros).
  const int nsw = NC * SPW;
  auto kstep = [&](int j) __attribute__((always_inline)) { return (j / SPW) * SPC + wave + NW * (j % SPW); };

  bf16x8 wf[D][RGT];
  floatx4 acc[RGT][MT];
#pragma unroll
  for (int q = 0; q < RGT; ++q)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[q][t] = floatx4{};

  // W of wave step j into ring slot `slot`; k >= K loads zeros.
  auto load = [&](int j, int slot) __attribute__((always_inline)) {
    const int kk = 32 * kstep(j) + 8 * g;
    const uint32_t kmask = (uint32_t)((K - 1 - kk) >> 31) << 31;
#pragma unroll
    for (int q = 0; q < RG; ++q) {
      const uint32_t o = (woff[q] + (uint32_t)kk * 2u) | kmask;
      wf[slot][q] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, 0));
      if constexpr (SW)
        wf[slot][RG + q] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(ru, o, 0, 0));
    }
  };
  // X, chunk c: wave loads rows wave * XPW .. + XPW; lane l loads chunk l of
  // every row and stores it at slot l ^ (row & 15), so the fragment reads (16
  // rows, one chunk) hit 16 different bank groups and one norm-weight piece
  // per lane and chunk (wn) serves all of the lane's rows. Two register
  // buffers: chunk c's rows sit in xr[c & 1] from two chunks before their LDS
  // store, so the W loads issued in between stay in flight.
  bf16x8 xr[2][XPW];
  bf16x8 wn[2];
  float ss[XPW];
#pragma unroll
  for (int e = 0; e < XPW; ++e) ss[e] = 0.f;
  const __amdgpu_buffer_rsrc_t rn = make_rsrc(a.nw, (int64_t)K * 2);
  auto xload = [&](int c, int rb) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < XPW; ++e) {
      const int m = wave * XPW + e;
      const int kk = c * kRowsKC + 8 * lane;
      const uint32_t o = (m < M && kk < K) ? (uint32_t)((m * a.ldx + kk) * 2) : kOOB;
      xr[rb][e] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0));
    }
    const int kk = c * kRowsKC + 8 * lane;
    wn[rb] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rn, kk < K ? (uint32_t)kk * 2u : kOOB, 0, 0));
  };
  auto xstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < XPW; ++e) {
      const int m = wave * XPW + e;
      bf16x8 y;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float f = bf2f(xr[buf][e][q]);
        ss[e] += f * f;
        y[q] = f2bf(f * bf2f(wn[buf][q]));
      }
      *reinterpret_cast<bf16x8*>(&xs[buf][m * kRowsKC + 8 * (lane ^ (m & 15))]) = y;
    }
  };
  auto comp = [&](int j, int slot) __attribute__((always_inline)) {
    bf16x8 xf[MT];
    const bf16* xb = xs[(j / SPW) & 1];
    const int ch = 4 * (wave + NW * (j % SPW)) + g;  // 16-byte chunk of the row piece
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = 16 * t + i;
      xf[t] = *reinterpret_cast<const bf16x8*>(xb + m * kRowsKC + 8 * (ch ^ (m & 15)));
    }
#pragma unroll
    for (int q = 0; q < RGT; ++q)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[q][t] = mfma16x16x32(wf[slot][q], xf[t], acc[q][t]);
  };

  // Chunk c (in registers xr[c & 1] since two chunks ago) goes to LDS buffer
  // c & 1, which last held chunk c - 2 (finished by every wave before the
  // barrier of chunk c - 1); chunk c + 2 is loaded into the freed registers
  // (zeros past K). `cb` = c & 1, static in the unrolled loops below.
  auto chunk = [&](int c, int cb) __attribute__((always_inline)) {
    xstore(cb);
    xload(c + 2, cb);
    __syncthreads();
  };
  xload(0, 0);
  xstore(0);
  xload(1, 1);
  xload(2, 0);
  // Loads sit outside any branch (only loop back-edges), so the compiler's
  // per-register waits keep D steps of loads in flight. The unrolled block is
  // U steps (two chunks, so chunk parities are static); the first and last
  // blocks are peeled.
  constexpr int U = 2 * SPW;
  static_assert(U % D == 0, "the unrolled block holds whole register rings");
  const int nfull = nsw / U;
  if (nfull >= 2) {
#pragma unroll
    for (int jj = 0; jj < D; ++jj) load(jj, jj);
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < U; ++jj) {
      if (jj % SPW == 0 && jj > 0) chunk(jj / SPW, (jj / SPW) & 1);
      comp(jj, jj % D);
      load(D + jj, jj % D);
      __builtin_amdgcn_sched_barrier(0);  // keep each step's loads beside its MFMAs
    }
    for (int j0 = U; j0 < (nfull - 1) * U; j0 += U) {
#pragma unroll
      for (int jj = 0; jj < U; ++jj) {
        if (jj % SPW == 0) chunk((j0 + jj) / SPW, (jj / SPW) & 1);
        comp(j0 + jj, jj % D);
        load(j0 + D + jj, jj % D);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    const int jl = (nfull - 1) * U;
#pragma unroll
    for (int jj = 0; jj < U; ++jj) {
      if (jj % SPW == 0) chunk((jl + jj) / SPW, (jj / SPW) & 1);
      comp(jl + jj, jj % D);
      if (jj + D < U) load(jl + D + jj, (jj + D) % D);  // jj static: no runtime branch
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    __syncthreads();
  }
  // Steps past the last full block (all of them for short K), unpipelined.
  for (int j = nfull >= 2 ? nfull * U : 0; j < nsw; ++j) {
    if (j % SPW == 0 && j > 0) {
      const int c = j / SPW;
      if (c & 1) chunk(c, 1);
      else chunk(c, 0);
    }
    load(j, 0);
    comp(j, 0);
  }

  // Cross-wave sum in wave order, then the epilogue. Accumulator register e of
  // lane l in group (q, t) holds row 16 q + 4 (l / 16) + e, X row 16 t + l % 16.
#pragma unroll
  for (int q = 0; q < RGT; ++q)
#pragma unroll
    for (int t = 0; t < MT; ++t) red[wave][q][t][lane] = acc[q][t];
  // The wave's rows: partial sums over its 64 lanes (each lane saw 8 of every
  // 512 k of the row).
#pragma unroll
  for (int e = 0; e < XPW; ++e) {
    float v = ss[e];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    if (lane == 0) rsum[wave * XPW + e] = v;
  }
  __syncthreads();
  rows_epilogue<RG, MT, SW, true, NW, 64 * NW>(p, &red[0][0][0][0], rsum, s, n0, rows, seg_start + n0);
}

// ------------------------------------------------------------ row-owned GEMV, DMA ring
// The row-owned GEMV with both operands streamed global -> LDS by direct-to-LDS
// loads (buffer_load ... lds) in whole contiguous pieces. A stage is KS k of
// the block's weight rows and of the X rows: each row's piece is KS * 2 bytes
// of one row, and one DMA instruction (64 lanes x 16 bytes) fills 1024 / (KS * 2)
// whole pieces, so the weight stream reaches HBM as runs of whole cache lines
// rather than the 16-rows x 64-byte pattern of MFMA fragments, which a CU
// issues at about half the rate. NS stages in a ring keep NS - 1 of them in
// flight; no VGPRs hold in-flight data. The lane that lands at 16-byte slot c
// of row r fetches chunk c ^ (r & 15), so the 16 rows of a fragment read hit
// 16 different bank groups. The 4 waves of a group take the stage's k-steps
// round robin (8 waves: two groups, one per X tile), one barrier per stage,
// and sum their fp32 partials in wave order.
// NORM: the RMSNorm weight sits in LDS for the whole call (K <= 8192); each
// X fragment becomes bf16(x * w_norm) on its way into the MFMA, the lane keeps
// the sum of x^2 over the k it sees, and the epilogue scales the row's dot
// products by rsqrt(sum / K + eps).
constexpr int kRowsDmaNormMaxK = 8192;

template <int RG, int MT, bool SW, bool NORM, int KS, int NS, int NW>
__global__ __launch_bounds__(64 * NW) void gemv_rows_dma_kernel(const RowsParams p) {
  constexpr int NG = NW / 4;          // wave groups: with 2, group h computes X tile h only
  constexpr int TT = MT / NG;         // X tiles per wave
  constexpr int RGT = SW ? 2 * RG : RG;
  constexpr int RB = KS * 2;          // bytes of one row piece
  constexpr int CPR = KS / 8;         // 16-byte chunks per row piece
  constexpr int RPI = 1024 / RB;      // row pieces per DMA instruction
  constexpr int WI = 16 * RGT / RPI;  // DMA instructions per stage: weight rows
  constexpr int XI = 16 * MT / RPI;   //                              X rows
  constexpr int IPW = (WI + XI) / NW; // per wave
  constexpr int SLOT = (WI + XI) * 1024;
  constexpr int SPW = KS / 128;       // k-steps per wave per stage (4 waves of a group share them)
  constexpr int WNB = NORM ? kRowsDmaNormMaxK * 2 : 0;
  static_assert((NW == 4 || (NW == 8 && MT == 2)) && KS % 128 == 0 && KS <= 512 && (WI + XI) % NW == 0,
                "whole pieces, whole k-steps per wave");
  static_assert(NS >= 2 && NS * SLOT + WNB <= 160 * 1024 - 1024, "ring fits LDS");
  static_assert(4 * RGT * MT * 1024 <= NS * SLOT, "partials fit the ring");
  __shared__ __attribute__((aligned(1024))) char lds[NS * SLOT + WNB];
  __shared__ float rs[NORM ? 4 * 16 * MT : 1];
  __shared__ float rsum[NORM ? 16 * MT : 1];
  const GemvArgs& a = p.a;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wg = wave & 3, h = wave >> 2;  // wave within its group, group
  const int i = lane & 15, g = lane >> 4;
  const int b = blockIdx.x;
  int s = 0;
#pragma unroll
  for (int j = 1; j < 4; ++j)
    if (j < a.seg.n && b >= p.bstart[j]) s = j;
  s = __builtin_amdgcn_readfirstlane(s);
  const int n0 = (b - p.bstart[s]) * p.r;
  const int seg_start = pick4(s, a.seg.start[0], a.seg.start[1], a.seg.start[2], a.seg.start[3]);
  const int seg_end = s + 1 < a.seg.n ? pick4(s, a.seg.start[1], a.seg.start[2], a.seg.start[3], a.N) : a.N;
  const int rows = min(p.r, seg_end - seg_start - n0);
  const int K = a.K, M = a.M;
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(uniform_ptr(pick4(s, a.seg.w[0], a.seg.w[1], a.seg.w[2], a.seg.w[3]) + (int64_t)n0 * a.ldw),
                (int64_t)rows * a.ldw * 2);
  const __amdgpu_buffer_rsrc_t ru =
      SW ? make_rsrc(uniform_ptr(a.W2 + (int64_t)n0 * a.ldw), (int64_t)rows * a.ldw * 2) : rw;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.X, (int64_t)M * a.ldx * 2);
  const uint32_t lbase = lds_addr(lds);

  // Instruction d = wave + NW * u of a stage fills slot bytes [1024 d, 1024 d + 1024):
  // weight row pieces first (16 RGT rows: the gate rows, then for SwiGLU the up
  // rows), then the X rows. Per lane: the piece's byte offset at k = 0 and the
  // chunk it fetches. Rows past the block's rows or past M load zeros.
  uint32_t off[IPW];
  int kc[IPW];  // the lane's k within a stage
#pragma unroll
  for (int u = 0; u < IPW; ++u) {
    const int d = wave + NW * u;
    const int r = (d < WI ? d : d - WI) * RPI + lane / CPR;  // row within its section
    const int c = (lane % CPR) ^ (r & 15);
    kc[u] = 8 * c;
    const int wr = r < 16 * RG ? r : r - 16 * RG;
    off[u] = d < WI ? (wr < rows ? (uint32_t)(wr * a.ldw * 2 + 16 * c) : kOOB)
                    : (r < M ? (uint32_t)(r * a.ldx * 2 + 16 * c) : kOOB);
  }
  auto issue = [&](int st, int slot) __attribute__((always_inline)) {
    const int k0 = st * KS;
    const uint32_t sb = lbase + (uint32_t)(slot * SLOT);
#pragma unroll
    for (int u = 0; u < IPW; ++u) {
      const int d = wave + NW * u;
      const uint32_t kmask = (uint32_t)((K - 1 - (k0 + kc[u])) >> 31) << 31;  // k >= K: out of range
      const uint32_t o = (off[u] + (uint32_t)k0 * 2u) | kmask;
      const uint32_t dst = sb + (uint32_t)(d * 1024);
      // The source is wave-uniform: where the section boundaries are multiples
      // of NW it is static in u, otherwise a scalar branch picks it.
      // Weights are read once per call: non-temporal (gate/up 46.1 -> 41.4 us, down 27.1 -> 26.1).
      if (d >= WI) dma16(rx, o, dst);
      else if (SW && d * RPI >= 16 * RG) dma16_nt(ru, o, dst);
      else dma16_nt(rw, o, dst);
    }
  };
  if constexpr (NORM) {
    // The norm weight, K * 2 bytes (zeros past K), before the first stage: the
    // first stage's wait covers it (loads retire in order).
    const __amdgpu_buffer_rsrc_t rn = make_rsrc(a.nw, (int64_t)K * 2);
    const uint32_t wb = lbase + (uint32_t)(NS * SLOT);
    for (int d = wave; d < (K + 511) / 512; d += NW) dma16(rn, (uint32_t)(d * 1024 + 16 * lane), wb + (uint32_t)(d * 1024));
  }

  floatx4 acc[RGT][TT];
#pragma unroll
  for (int q = 0; q < RGT; ++q)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[q][t] = floatx4{};
  float ss[TT];  // NORM: sum of x^2 of the lane's X rows over the k it sees
#pragma unroll
  for (int t = 0; t < TT; ++t) ss[t] = 0.f;
  const int t0 = NG == 1 ? 0 : h;  // first X tile of the wave

  // Only stages below nst are issued, so at stage st at most one later stage
  // (NS <= 3) is in flight, none at the last.
  static_assert(NS <= 3, "the waits below count at most one stage in flight after st");
  const int nst = (K + KS - 1) / KS;
#pragma unroll
  for (int st = 0; st < NS - 1; ++st)
    if (st < nst) issue(st, st);
  int cs = 0;  // ring slot of stage st
  for (int st = 0; st < nst; ++st) {
    if (st == nst - 1) vm_wait<0>();      // this wave's pieces of stage st have landed
    else vm_wait<(NS - 2) * IPW>();
    __syncthreads();  // everyone's have; everyone is done with stage st - 1
    if (st + NS - 1 < nst) issue(st + NS - 1, cs == 0 ? NS - 1 : cs - 1);
    const char* sb = lds + cs * SLOT;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int c = 4 * (wg + 4 * j) + g;  // the lane's 16-byte chunk of every row piece
      const int pc = 16 * (c ^ i);         // its slot in rows 16 q + i
      bf16x8 wf[RGT], xf[TT];
#pragma unroll
      for (int q = 0; q < RGT; ++q) wf[q] = *reinterpret_cast<const bf16x8*>(sb + (16 * q + i) * RB + pc);
#pragma unroll
      for (int t = 0; t < TT; ++t)
        xf[t] = *reinterpret_cast<const bf16x8*>(sb + WI * 1024 + (16 * (t0 + t) + i) * RB + pc);
      if constexpr (NORM) {
        const bf16x8 wn = *reinterpret_cast<const bf16x8*>(lds + NS * SLOT + 2 * (st * KS + 8 * c));
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float f = bf2f(xf[t][e]);
            ss[t] += f * f;
            xf[t][e] = f2bf(f * bf2f(wn[e]));
          }
        }
      }
#pragma unroll
      for (int q = 0; q < RGT; ++q)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[q][t] = mfma16x16x32(wf[q], xf[t], acc[q][t]);
    }
    cs = cs + 1 == NS ? 0 : cs + 1;
  }

  // The ring becomes the partials' buffer once every wave is past its last
  // fragment read (no load is outstanding after the last stage's wait). Partials are
  // laid out [wave of the group][q][X tile][lane] and summed over the group's
  // 4 waves in order.
  vm_wait<0>();
  __syncthreads();
  floatx4* red = reinterpret_cast<floatx4*>(lds);
#pragma unroll
  for (int q = 0; q < RGT; ++q)
#pragma unroll
    for (int t = 0; t < TT; ++t) red[((wg * RGT + q) * MT + t0 + t) * 64 + lane] = acc[q][t];
  if constexpr (NORM) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      float v = ss[t];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (g == 0) rs[wg * 16 * MT + 16 * (t0 + t) + i] = v;
    }
    __syncthreads();
    if (tid < 16 * MT) {
      float v = rs[tid];
#pragma unroll
      for (int w = 1; w < 4; ++w) v += rs[w * 16 * MT + tid];
      rsum[tid] = v;
    }
  }
  __syncthreads();
  rows_epilogue<RG, MT, SW, NORM, 4, 64 * NW>(p, red, rsum, s, n0, rows, seg_start + n0);
}

bool rows_selected(int64_t M, int64_t K) { return M <= kRowsDirectMaxM || K <= kRowsMaxK; }

int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int RG, int MT, bool SW>
void rows_launch_d(const RowsParams& p, int grid, hipStream_t st) {
  constexpr int RGT = SW ? 2 * RG : RG;
  constexpr int D = RGT <= 4 ? 8 : 4;  // register ring: ~32-48 KB of W in flight per CU
  hipLaunchKernelGGL((gemv_rows_kernel<RG, MT, SW, D>), dim3(grid), dim3(256), 0, st, p);
}
// DMA-ring form. Longer row pieces stream faster from HBM (measured, M = 32:
// gate/up with 512-byte pieces in 2 slots 38.2 us against 41.4 with 256-byte
// pieces in 5; down, K = 12288, with 1 KB pieces 25.0 against 26.1 with 512
// bytes), so a stage takes the longest k that leaves at least two slots in
// 144 KB: 512 for one plain row group over K >= 8192, else 256, else 128. As
// many slots as fit, at most 3 (deeper rings were no faster: the B=32 decode
// step 209.3 us with at most 3, 209.7 with 4, 210.2 with 6); 8 waves (two per
// SIMD) where the DMA count splits evenly.
template <int RG, int MT, bool SW, bool NORM, int KS>
void rows_dma_launch_ks(const RowsParams& p, int grid, hipStream_t st) {
  constexpr int RGT = SW ? 2 * RG : RG;
  constexpr int RPI = 512 / KS;
  constexpr int SLOT = (16 * RGT / RPI + 16 * MT / RPI) * 1024;
  constexpr int WNB = NORM ? kRowsDmaNormMaxK * 2 : 0;
  constexpr int NS0 = (144 * 1024 - WNB) / SLOT;
  constexpr int NS = NS0 > 3 ? 3 : NS0;
  constexpr int NW = MT == 2 && (16 * RGT / RPI + 16 * MT / RPI) % 8 == 0 ? 8 : 4;  // 8: 2 waves per SIMD
  hipLaunchKernelGGL((gemv_rows_dma_kernel<RG, MT, SW, NORM, KS, NS, NW>), dim3(grid), dim3(64 * NW), 0, st, p);
}
template <int RG, int MT, bool SW, bool NORM>
void rows_dma_launch(const RowsParams& p, int grid, hipStream_t st) {
  constexpr int RGT = SW ? 2 * RG : RG;
  constexpr int WNB = NORM ? kRowsDmaNormMaxK * 2 : 0;
  constexpr bool fits256 = (144 * 1024 - WNB) / ((16 * RGT + 16 * MT) / 2 * 1024) >= 2;
  if constexpr (RGT == 1 && !NORM) {
    if (p.a.K >= 8192) {
      rows_dma_launch_ks<RG, MT, SW, NORM, 512>(p, grid, st);
      return;
    }
  }
  rows_dma_launch_ks<RG, MT, SW, NORM, fits256 ? 256 : 128>(p, grid, st);
}
// Every plain form runs the DMA ring (at M <= 8 too: M = 1 / 8 down 20.9 ->
// 18.1 / 23.4 -> 18.4 us, gate/up 43.3 -> 35.8 / 43.7 -> 34.9, o and q/k/v
// 0.5-2 us faster than the register ring, outputs bit-identical); the
// register ring stays for the fused norm past the LDS copy of its weight.
template <int RG, int MT, bool SW>
void rows_launch_x(const RowsParams& p, int grid, hipStream_t st) {
  if (p.a.nw && p.a.K > kRowsDmaNormMaxK) rows_launch_d<RG, MT, SW>(p, grid, st);
  else if (p.a.nw) rows_dma_launch<RG, MT, SW, true>(p, grid, st);
  else rows_dma_launch<RG, MT, SW, false>(p, grid, st);
}
template <bool SW>
void rows_launch_rg(const RowsParams& p, int rg, int grid, hipStream_t st) {
  const bool mt2 = p.a.M > 16;
  switch (rg) {
    case 1: mt2 ? rows_launch_x<1, 2, SW>(p, grid, st) : rows_launch_x<1, 1, SW>(p, grid, st); break;
    case 2: mt2 ? rows_launch_x<2, 2, SW>(p, grid, st) : rows_launch_x<2, 1, SW>(p, grid, st); break;
    case 3: mt2 ? rows_launch_x<3, 2, SW>(p, grid, st) : rows_launch_x<3, 1, SW>(p, grid, st); break;
    default: mt2 ? rows_launch_x<4, 2, SW>(p, grid, st) : rows_launch_x<4, 1, SW>(p, grid, st); break;
  }
}

int rows_launch(const GemvArgs& a, hipStream_t st) {
  RowsParams p{};
  p.a = a;
  const int nseg = a.seg.n;
  int64_t len[4] = {};
  for (int i = 0; i < nseg; ++i) len[i] = (i + 1 < nseg ? a.seg.start[i + 1] : a.N) - a.seg.start[i];
  const int cus = device_cus();
  auto blocks_for = [&](int64_t r) {
    int64_t n = 0;
    for (int i = 0; i < nseg; ++i) n += q3_cdiv(len[i], r);
    return n;
  };
  // Smallest r that gives every CU at most one block, at most 64 (beyond
  // 64 * CUs rows the grid takes several blocks per CU).
  int64_t r = std::min<int64_t>(16 * kRowsMaxRG, std::max<int64_t>(1, q3_cdiv(a.N, cus)));
  while (r < 16 * kRowsMaxRG && blocks_for(r) > cus) ++r;
  p.r = (int)r;
  int64_t acc = 0;
  for (int i = 0; i < nseg; ++i) {
    p.bstart[i] = (int)acc;
    acc += q3_cdiv(len[i], r);
  }
  for (int i = nseg; i < 5; ++i) p.bstart[i] = (int)acc;
  const bool r_ok = a.R == nullptr || (q3_aligned(a.R, 8) && a.ldr % 4 == 0);
  bool b_ok = true;
  for (int i = 0; i < nseg; ++i) b_ok = b_ok && (!a.seg.b[i] || q3_aligned(a.seg.b[i], 8));
  p.vec4 = q3_aligned(a.C, 8) && a.ldc % 4 == 0 && r_ok && b_ok;
  const int rg = (int)q3_cdiv(r, 16);
  if (a.W2) rows_launch_rg<true>(p, rg, (int)acc, st);
  else rows_launch_rg<false>(p, rg, (int)acc, st);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

struct GemvPlan {
  int n_tiles, k_stages, total, grid, max_pieces;
  int64_t counter_bytes, bytes;
};

GemvPlan gemv_plan(int64_t N, int64_t K, bool swiglu) {
  GemvPlan pl{};
  pl.n_tiles = (int)q3_cdiv(N, swiglu ? 64 : kGvBN);
  pl.k_stages = (int)q3_cdiv(K, kGvBK);
  const int64_t total = (int64_t)pl.n_tiles * pl.k_stages;
  pl.total = (int)total;
  pl.grid = (int)std::min<int64_t>(kGvGrid, total);
  int mp = 0;
  for (int t = 0; t < pl.n_tiles; ++t) {
    const int fb = gv_block_of((int64_t)t * pl.k_stages, pl.grid, total);
    const int lb = gv_block_of((int64_t)t * pl.k_stages + pl.k_stages - 1, pl.grid, total);
    if (lb > fb) mp = std::max(mp, lb - fb + 1);
  }
  pl.max_pieces = mp;
  pl.counter_bytes = kGvCounterBytes;
  pl.bytes = pl.counter_bytes + (int64_t)pl.n_tiles * mp * kGvPiece * 4;
  return pl;
}

}  // namespace

bool gemv_eligible(const GemvArgs& a) {
  if (a.M < 1 || a.M > kGemvMaxRows || a.N < 1 || a.K < 8 || (a.K % 8) != 0) return false;
  // Tile count and segment alignment bound the stream-K kernel only; a fused
  // norm always runs the row-owned one.
  const bool sk = a.nw == nullptr && !rows_selected(a.M, a.K);
  if (sk && q3_cdiv(a.N, a.W2 ? 64 : kGvBN) > kGvMaxTiles) return false;
  if (a.seg.n < 1 || a.seg.n > 4) return false;
  if (!q3_aligned(a.X, 16) || (a.ldx % 8) != 0 || (a.ldw % 8) != 0) return false;
  if ((int64_t)a.M * a.ldx * 2 >= 0x7fffffffLL) return false;
  const bool swiglu = a.W2 != nullptr;
  if (swiglu) {
    if (a.seg.n != 1 || !q3_aligned(a.W2, 16)) return false;
    if (!q3_aligned(a.seg.w[0], 16) || (int64_t)a.N * a.ldw * 2 >= 0x7fffffffLL) return false;
    return true;
  }
  for (int i = 0; i < a.seg.n; ++i) {
    const int64_t end = i + 1 < a.seg.n ? a.seg.start[i + 1] : a.N;
    if (!a.seg.w[i] || !q3_aligned(a.seg.w[i], 16) || (sk && (a.seg.start[i] % kGvBN) != 0)) return false;
    if ((end - a.seg.start[i]) * a.ldw * 2 >= 0x7fffffffLL) return false;
  }
  return true;
}

int64_t gemv_workspace_bytes(int64_t M, int64_t N, int64_t K, bool swiglu) {
  if (M <= 0 || N <= 0 || K <= 0 || rows_selected(M, K)) return 0;
  return gemv_plan(N, K, swiglu).bytes;
}

int gemv_launch(const GemvArgs& a, void* ws, int64_t ws_bytes, hipStream_t st) {
  if (a.nw || rows_selected(a.M, a.K)) return rows_launch(a, st);
  const bool swiglu = a.W2 != nullptr;
  const GemvPlan pl = gemv_plan(a.N, a.K, swiglu);
  Q3_REQUIRE(ws != nullptr && ws_bytes >= pl.bytes, Q3_ERR_WORKSPACE);
  Q3_REQUIRE(q3_aligned(ws, 256), Q3_ERR_ALIGN);
  GemvParams p{};
  p.a = a;
  p.counters = static_cast<int*>(ws);
  p.partial = reinterpret_cast<float*>(static_cast<char*>(ws) + pl.counter_bytes);
  p.n_tiles = pl.n_tiles;
  p.k_stages = pl.k_stages;
  p.total = pl.total;
  p.grid = pl.grid;
  p.max_pieces = pl.max_pieces;
  const bool r_ok4 = a.R == nullptr || (q3_aligned(a.R, 8) && a.ldr % 4 == 0);
  const bool r_ok8 = a.R == nullptr || (q3_aligned(a.R, 16) && a.ldr % 8 == 0);
  bool b_ok4 = true, b_ok8 = true;
  for (int i = 0; i < a.seg.n; ++i) {
    if (!a.seg.b[i]) continue;
    b_ok4 = b_ok4 && q3_aligned(a.seg.b[i], 8);
    b_ok8 = b_ok8 && q3_aligned(a.seg.b[i], 16);
  }
  p.vec4 = q3_aligned(a.C, 8) && a.ldc % 4 == 0 && r_ok4 && b_ok4;
  p.vec8 = q3_aligned(a.C, 16) && a.ldc % 8 == 0 && r_ok8 && b_ok8;
  if (swiglu)
    hipLaunchKernelGGL(gemv_kernel<true>, dim3(pl.grid), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(gemv_kernel<false>, dim3(pl.grid), dim3(256), 0, st, p);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

}  // namespace q3
