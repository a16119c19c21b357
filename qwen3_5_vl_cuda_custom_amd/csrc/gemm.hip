// GEMM entry points of the C-ABI: q3_matmul, q3_matmul_swiglu, q3_matmul_segments,
// q3_rmsnorm_matmul_segments, q3_rmsnorm_matmul_swiglu, q3_batched_gemm.
//
//   Y[m, n] = sum_k X[m, k] * W[n, k] (+ bias[n]) (+ R[m, n])   (nn.Linear layout)
//
// Three device paths, chosen on the host from the shape:
//  * tiled   : bf16, M > 32     -> 32x32x16 MFMA over a ring of direct-to-LDS tiles
//  * gemv    : bf16, M <= 32    -> weight-streaming stream-K kernel (gemv.hip)
//  * generic : fp32, or bf16 whose rows are not 16-byte aligned -> SIMT fp32
#include "gemm_kernels.h"
#include "gemv.h"

using namespace q3;

namespace {

// =====================================================================
// Generic SIMT path (fp32 operands, or bf16 with unaligned rows): 64x64 tiles,
// 256 threads, 4x4 outputs per thread, fp32 accumulation.
// =====================================================================
template <typename T>
__global__ __launch_bounds__(256) void gemm_generic_kernel(const T* __restrict__ X, const T* __restrict__ W,
                                                           const T* __restrict__ bias, const T* __restrict__ R,
                                                           T* __restrict__ C, int M, int N, int K, int64_t ldx,
                                                           int64_t ldw, int64_t ldr, int64_t ldc, int64_t bsX,
                                                           int64_t bsW, int64_t bsC, int swiglu,
                                                           const T* __restrict__ W2, int act) {
  __shared__ float xs[16][65];
  __shared__ float ws[16][65];
  __shared__ float ws2[16][65];
  const int z = blockIdx.z;
  X += z * bsX;
  W += z * bsW;
  C += z * bsC;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4] = {}, acc2[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int i = threadIdx.x; i < 16 * 64; i += 256) {
      const int kk = i % 16, rr = i / 16;
      const int m = m0 + rr, n = n0 + rr, k = k0 + kk;
      xs[kk][rr] = (m < M && k < K) ? to_f(X[(int64_t)m * ldx + k]) : 0.f;
      ws[kk][rr] = (n < N && k < K) ? to_f(W[(int64_t)n * ldw + k]) : 0.f;
      if (swiglu) ws2[kk][rr] = (n < N && k < K) ? to_f(W2[(int64_t)n * ldw + k]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4], b2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = xs[kk][ty * 4 + i];
        b[i] = ws[kk][tx * 4 + i];
        b2[i] = swiglu ? ws2[kk][tx * 4 + i] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
          acc2[i][j] = fmaf(a[i], b2[j], acc2[i][j]);
        }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
      if (m >= M || n >= N) continue;
      float v = acc[i][j];
      if (swiglu) {
        v = v / (1.0f + expf(-v)) * acc2[i][j];
      } else {
        if (bias) v += to_f(bias[n]);
        if (act) v = gelu_tanh_f(v);
        if (R) v += to_f(R[(int64_t)m * ldr + n]);
      }
      C[(int64_t)m * ldc + n] = from_f<T>(v);
    }
}

template <typename T>
int launch_generic(const void* x, const void* w, const void* w2, const void* bias, const void* r, void* y, int64_t M,
                   int64_t N, int64_t K, int64_t batch, int64_t ldx, int64_t ldw, int64_t ldr, int64_t ldc,
                   int64_t bsX, int64_t bsW, int64_t bsC, bool swiglu, hipStream_t st, int act = 0) {
  dim3 grid((unsigned)q3_cdiv(N, 64), (unsigned)q3_cdiv(M, 64), (unsigned)batch);
  hipLaunchKernelGGL(gemm_generic_kernel<T>, grid, dim3(256), 0, st, static_cast<const T*>(x),
                     static_cast<const T*>(w), static_cast<const T*>(bias), static_cast<const T*>(r),
                     static_cast<T*>(y), (int)M, (int)N, (int)K, ldx, ldw, ldr, ldc, bsX, bsW, bsC, swiglu ? 1 : 0,
                     static_cast<const T*>(w2), act);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

// =====================================================================
// Tiled MFMA path.
// =====================================================================
template <int BM, int BN, int WM, int WN, int EPI, int NST, int BKT, int NSTW = NST, bool MF16 = false>
int launch_tiled_cfg(GemmParams p, int64_t batch, hipStream_t st) {
  constexpr int BN_OUT = (EPI == kEpiSwiGLU) ? BN / 2 : BN;
  const int64_t tiles = q3_cdiv(p.M, BM) * q3_cdiv(p.N, BN_OUT);
  p.group_m = 4;  // 4 along M: S=4096 gate/up 587 -> 582 us, o 112 -> 110, S=1024 layer 430.6 -> 425.4 (8 and 16: slower)
  hipLaunchKernelGGL((gemm_bf16_dma_kernel<BM, BN, WM, WN, EPI, false, NST, BKT, NSTW, MF16>),
                     dim3((unsigned)tiles, 1, (unsigned)batch), dim3(WM * WN * 64), 0, st, p);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

// Tile configuration by estimated time: full waves of blocks over 256 CUs,
// times the block's work over its relative MFMA efficiency (measured on
// MI355X): 256x256 (8 waves, 64-wide K stages: 2 X slots, 3 W slots, the
// whole 160 KB of LDS; 1 block per CU) 1.0,
// 128x256 (8 waves, 64-wide K stages; over K >= 2048 the 16x16x32 loop with
// 2 X and 4 W slots and the wave priority of the 256-row tiles, else the
// 32x32x16 loop with 3 stages, 144 KB. The third stage hides the HBM latency
// of weights read once per layer: with weights rotated past the MALL, M=1024
// gate/up 243 -> 189 us, M=4096 o 165 -> 131 us. The 16x16x32 form with the
// priority: M=1024 gate/up 184-185 -> 173-174 us, q/k/v 59-61 -> 58, the
// S=1024 layer 464-466 -> 451-456 us, bit-identical) 0.9, 256x192 (8 waves, 64-wide K
// stages, 2 X and 3 W slots; plain epilogue only) 0.95, 128x128 (4 waves; 2
// blocks per CU) 0.75. The third W slot (weights are read from HBM once per
// layer, activations from L2): M=4096 q/k/v 181 -> 170 us, gate/up 650 ->
// 633 us with weights rotated past the MALL.
//
// When the 128x128 tiles fit one block per CU (at most 256 of them) they take
// a deeper ring instead: 64-wide K stages in 4 X and 5 W slots (147 KB).
// Measured against the 2-blocks-per-CU ring (32-wide stages x 4): M=3136 N=1152
// K=4304 60.9 -> 49.3 us, M=1024 N=4096 K=12288 147.7 -> 120.1 us, K=4096
// 48.1 -> 43.7 us, shorter K unchanged; such a wave of tiles takes 0.46-0.56
// of the time of one wave of 256x256 tiles (estimate: 128 * 128 / 0.47).
// Rings of 6 or 8 32-wide stages were no faster than 4.
//
// The 256x256 tiles, and the 256x192 ones over K >= 2048, run the kernel's
// 16x16x32 loop (MF16): these long K loops are power-limited, and for the same
// work that instruction moves less data through the register file, so the
// chip holds a higher clock. Same-box A/B, bit-identical outputs: the S=4096
// decoder layer 1464.9 -> 1395.1 us (gate/up 633 -> 608, down 326 -> 307, o
// 121 -> 116, q/k/v on 256x192); S=1024 475.7 -> 469.2 us. The MoE expert
// tiles stay on 32x32x16: no faster with it. (The 128x128 deep ring and the
// 128x256 tiles take it in their own forms: launch_c, launch_d.)
//
// The 128x256 tiles on that loop keep a fourth W slot (2 X + 4 W slots of 64-wide
// stages, 160 KB): M=1024 gate/up 185.1 -> 181.5 us, q/k/v 56.6 -> 55.2 us, the
// S=1024 layer 461 -> 450 us, bit-identical. A fourth W slot for the 256x192
// tiles (also 160 KB) measured no faster: M=4096 q/k/v 166.0 -> 166.7 us.
template <int EPI>
int launch_tiled(GemmParams p, int64_t batch, hipStream_t st) {
  constexpr int kCUs = 256;
  auto waves = [](int64_t tiles, int64_t slots) { return (double)q3_cdiv(tiles, slots); };
  const int bo = EPI == kEpiSwiGLU ? 128 : 256;
  const double cost_a = waves(q3_cdiv(p.M, 256) * q3_cdiv(p.N, bo) * batch, kCUs) * 256.0 * 256.0;
  const int64_t tiles_c = q3_cdiv(p.M, 128) * q3_cdiv(p.N, bo / 2) * batch;
  const bool c_deep = tiles_c <= kCUs;  // one 128x128 block per CU: the deep ring
  const double cost_c = c_deep ? 128.0 * 128.0 / 0.47 : waves(tiles_c, 2 * kCUs) * 2.0 * 128.0 * 128.0 / 0.75;
  // 128x256 only when it fills at least 3/4 of the CUs: with fewer tiles the
  // 128x128 tiles, one per CU, run faster.
  const int64_t tiles_d = q3_cdiv(p.M, 128) * q3_cdiv(p.N, bo) * batch;
  const double cost_d = 4 * tiles_d >= 3 * kCUs ? waves(tiles_d, kCUs) * 128.0 * 256.0 / 0.9 : 1e300;
  auto launch_c = [&]() {
    // The deep ring's tiles, but for SwiGLU (which pairs 64-row gate/up groups
    // within a wave), run 8 waves of 64x32 on the 16x16x32 loop, two waves per
    // SIMD instead of one: C5 patch embed + vision block 230.1 -> 219.2 us,
    // S=1024 and C4 unchanged, bit-identical (same-box A/B).
    if constexpr (EPI != kEpiSwiGLU) {
      if (c_deep) return launch_tiled_cfg<128, 128, 2, 4, EPI, 4, 64, 5, true>(p, batch, st);
    }
    return c_deep ? launch_tiled_cfg<128, 128, 2, 2, EPI, 4, 64, 5>(p, batch, st)
                  : launch_tiled_cfg<128, 128, 2, 2, EPI, 4, 32>(p, batch, st);
  };
  auto launch_d = [&]() {
    return p.K >= 2048 ? launch_tiled_cfg<128, 256, 2, 4, EPI, 2, 64, 4, true>(p, batch, st)
                       : launch_tiled_cfg<128, 256, 2, 4, EPI, 3, 64>(p, batch, st);
  };
  if constexpr (EPI == kEpiSwiGLU) {
    if (cost_c < cost_a && cost_c < cost_d) return launch_c();
    if (cost_d < cost_a) return launch_d();
    return launch_tiled_cfg<256, 256, 2, 4, EPI, 2, 64, 3, true>(p, batch, st);
  } else {
    const double cost_b = waves(q3_cdiv(p.M, 256) * q3_cdiv(p.N, 192) * batch, kCUs) * 256.0 * 192.0 / 0.95;
    const double best = std::min(std::min(cost_a, cost_b), std::min(cost_c, cost_d));
    if (cost_c == best) return launch_c();
    if (cost_b == best)  // long K loops: the 16x16x32 loop (power-limited); short ones the 32x32x16 loop
      return p.K >= 2048 ? launch_tiled_cfg<256, 192, 4, 2, EPI, 2, 64, 3, true>(p, batch, st)
                         : launch_tiled_cfg<256, 192, 4, 2, EPI, 2, 64, 3>(p, batch, st);
    if (cost_d == best) return launch_d();
    return launch_tiled_cfg<256, 256, 2, 4, EPI, 2, 64, 3, true>(p, batch, st);
  }
}

// ---------------------------------------------------------------- split over K
// A plain store (bias and residual allowed, no activation, batch 1) whose
// 256x256 tiles would leave most CUs idle and whose fallback, the one-wave
// 128x128 ring, is bound by each CU's operand stream over a long K (M=1024,
// N=4096, K=12288: 6.3 MB per tile, 135 us) runs as S splits of 256x256 tiles
// (the tile GEMM's batch dimension: split z reads X and W columns
// [z K/S, (z + 1) K/S) and writes fp32 partial plane z), then one kernel sums
// the planes in split order, adds bias and residual and rounds once, the
// order of the unsplit epilogue. Chosen by estimates from measured rates: a
// wave of 256x256 tiles takes ~9.8 + 0.0243 K us, +4 us for an fp32 epilogue;
// the 128x128 ring ~0.45 of that at full K; the reduction moves its bytes
// (planes, residual, output) at ~5 TB/s after a ~4 us launch (the estimate
// counts a residual, so the plan and workspace size depend on M, N, K only). The partial planes follow the GEMM
// workspace's 16 KiB counter region, which they never touch.
constexpr int64_t kSplitWsOffset = 16 << 10;

int split_k_plan(int64_t M, int64_t N, int64_t K) {
  if (M <= kGemvMaxRows || K < 2048 || M >= (1 << 20) || N >= (1 << 20)) return 1;
  const int64_t tiles_a = q3_cdiv(M, 256) * q3_cdiv(N, 256);
  if (q3_cdiv(M, 128) * q3_cdiv(N, 128) > 256) return 1;  // not the one-wave 128x128 case
  const double t_c = 0.45 * (9.8 + 0.0243 * (double)K);
  int best = 1;
  double t_best = t_c;
  for (int s = 2; s <= 8; s *= 2) {
    if (tiles_a * s > 256 || K % (64 * s) != 0) continue;
    const double bytes = (double)s * M * N * 4 + (double)M * N * 4;  // planes, residual in, C out
    const double t = 9.8 + 0.0243 * (double)(K / s) + 4.0 + bytes / 5e6 + 4.0;
    if (t < t_best) {
      t_best = t;
      best = s;
    }
  }
  return best;
}

int64_t split_k_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  const int s = split_k_plan(M, N, K);
  return s > 1 ? kSplitWsOffset + (int64_t)s * M * N * 4 : 0;
}

// One thread per 8 output columns: C = bf16(sum_z P[z] + bias + R).
__global__ __launch_bounds__(256) void split_k_reduce_kernel(const float* __restrict__ parts, int S, int64_t M,
                                                             int64_t N, const bf16* __restrict__ bias,
                                                             const bf16* __restrict__ R, int64_t ldr,
                                                             bf16* __restrict__ C, int64_t ldc, int vec) {
  const int64_t n8 = (N + 7) / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * n8) return;
  const int64_t m = i / n8, n = (i % n8) * 8;
  const int64_t plane = M * N;
  float o[8];
  if (vec && n + 7 < N) {
#pragma unroll
    for (int q = 0; q < 8; ++q) o[q] = 0.f;
    for (int z = 0; z < S; ++z) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(parts + z * plane + m * N + n);
      const floatx4 b = *reinterpret_cast<const floatx4*>(parts + z * plane + m * N + n + 4);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        o[q] += a[q];
        o[4 + q] += b[q];
      }
    }
    if (bias) {
      const bf16x8 bv = *reinterpret_cast<const bf16x8*>(bias + n);
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] += bf2f(bv[q]);
    }
    if (R) {
      const bf16x8 rv = *reinterpret_cast<const bf16x8*>(R + m * ldr + n);
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] += bf2f(rv[q]);
    }
    bf16x8 v;
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = f2bf(o[q]);
    *reinterpret_cast<bf16x8*>(C + m * ldc + n) = v;
  } else {
    for (int q = 0; q < 8 && n + q < N; ++q) {
      float acc = 0.f;
      for (int z = 0; z < S; ++z) acc += parts[z * plane + m * N + n + q];
      if (bias) acc += bf2f(bias[n + q]);
      if (R) acc += bf2f(R[m * ldr + n + q]);
      C[m * ldc + n + q] = f2bf(acc);
    }
  }
}

int launch_split_k(const GemmParams& p0, int S, void* ws, hipStream_t st) {
  GemmParams p = p0;
  float* parts = reinterpret_cast<float*>(static_cast<char*>(ws) + kSplitWsOffset);
  const int64_t ks = p0.K / S;
  p.C = reinterpret_cast<bf16*>(parts);
  p.K = (int)ks;
  p.ldc = p0.N;
  p.bsX = ks;
  p.bsW = ks;
  p.bsC = (int64_t)p0.M * p0.N;
  p.bias = nullptr;
  p.R = nullptr;
  p.act = 0;
  p.seg.n = 1;
  p.seg.w[0] = p.W;
  const int rc = launch_tiled_cfg<256, 256, 2, 4, kEpiStoreF32, 2, 64, 3, true>(p, S, st);
  if (rc != Q3_OK) return rc;
  const bool vec = p0.N % 8 == 0 && p0.ldc % 8 == 0 && q3_aligned(p0.C, 16) &&
                   (!p0.bias || q3_aligned(p0.bias, 16)) && (!p0.R || (q3_aligned(p0.R, 16) && p0.ldr % 8 == 0));
  const int64_t items = (int64_t)p0.M * q3_cdiv(p0.N, 8);
  hipLaunchKernelGGL(split_k_reduce_kernel, dim3((unsigned)q3_cdiv(items, 256)), dim3(256), 0, st, parts, S,
                     (int64_t)p0.M, (int64_t)p0.N, p0.bias, p0.R, p0.ldr, p0.C, p0.ldc, vec ? 1 : 0);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

bool bf16_rows_ok(const void* base, int64_t ld, int64_t K) {
  return q3_aligned(base, 16) && (ld % 8 == 0) && (K % 8 == 0);
}

int matmul_impl(const void* x, const void* w, const void* w2, const void* bias, const void* residual, void* y,
                int64_t M, int64_t N, int64_t K, int64_t batch, int64_t ldx, int64_t ldw, int64_t ldr, int64_t ldc,
                int64_t bsX, int64_t bsW, int64_t bsC, int dtype, bool swiglu, void* ws, int64_t ws_bytes,
                hipStream_t st, int act = 0) {
  Q3_REQUIRE(x && w && y, Q3_ERR_NULL);
  Q3_REQUIRE(!swiglu || w2, Q3_ERR_NULL);
  Q3_REQUIRE(M >= 0 && N >= 0 && K >= 0 && batch >= 1, Q3_ERR_SHAPE);
  Q3_REQUIRE(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31), Q3_ERR_SHAPE);
  Q3_REQUIRE(ldx >= K && ldw >= K && ldc >= N && (!residual || ldr >= N), Q3_ERR_SHAPE);
  Q3_REQUIRE(dtype == Q3_F32 || dtype == Q3_BF16, Q3_ERR_DTYPE);
  Q3_REQUIRE(!(swiglu && (bias || residual)), Q3_ERR_UNSUPPORTED);
  if (M == 0 || N == 0) return Q3_OK;
  if (dtype == Q3_F32)
    return launch_generic<float>(x, w, w2, bias, residual, y, M, N, K, batch, ldx, ldw, ldr, ldc, bsX, bsW, bsC,
                                 swiglu, st, act);
  const bool rows_ok = bf16_rows_ok(x, ldx, K) && bf16_rows_ok(w, ldw, K) && (!w2 || bf16_rows_ok(w2, ldw, K)) &&
                       (bsX % 8 == 0) && (bsW % 8 == 0);
  if (!rows_ok || K == 0)
    return launch_generic<bf16>(x, w, w2, bias, residual, y, M, N, K, batch, ldx, ldw, ldr, ldc, bsX, bsW, bsC,
                                swiglu, st, act);
  if (M <= kGemvMaxRows && batch == 1 && !act) {
    GemvArgs ga{};
    ga.X = static_cast<const bf16*>(x);
    ga.ldx = ldx;
    ga.seg.n = 1;
    ga.seg.w[0] = static_cast<const bf16*>(w);
    ga.seg.b[0] = static_cast<const bf16*>(bias);
    ga.W2 = static_cast<const bf16*>(w2);
    ga.R = static_cast<const bf16*>(residual);
    ga.ldr = ldr;
    ga.C = static_cast<bf16*>(y);
    ga.ldc = ldc;
    ga.M = (int)M;
    ga.N = (int)N;
    ga.K = (int)K;
    ga.ldw = ldw;
    if (gemv_eligible(ga)) return gemv_launch(ga, ws, ws_bytes, st);
  }
  GemmParams p{};
  p.X = static_cast<const bf16*>(x);
  p.W = static_cast<const bf16*>(w);
  p.W2 = static_cast<const bf16*>(w2);
  p.bias = static_cast<const bf16*>(bias);
  p.R = static_cast<const bf16*>(residual);
  p.C = static_cast<bf16*>(y);
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldr = ldr;
  p.ldc = ldc;
  p.bsX = bsX;
  p.bsW = bsW;
  p.bsC = bsC;
  p.act = act;
  if (!swiglu && !act && batch == 1) {
    const int S = split_k_plan(M, N, K);
    if (S > 1 && ws != nullptr && q3_aligned(ws, 16) && ws_bytes >= split_k_workspace_bytes(M, N, K))
      return launch_split_k(p, S, ws, st);
  }
  return swiglu ? launch_tiled<kEpiSwiGLU>(p, batch, st) : launch_tiled<kEpiStore>(p, batch, st);
}

int segments_impl(const void* x, const void* const* w, const void* const* bias, const int64_t* n, int64_t nseg,
                  void* y, int64_t M, int64_t K, int64_t ldx, int64_t ldw, int64_t ldc, int dtype, void* ws,
                  int64_t ws_bytes, hipStream_t st) {
  Q3_REQUIRE(x && w && n && y, Q3_ERR_NULL);
  Q3_REQUIRE(nseg >= 1 && nseg <= 4, Q3_ERR_SHAPE);
  int64_t N = 0;
  bool tiled_ok = true;
  for (int64_t i = 0; i < nseg; ++i) {
    Q3_REQUIRE(w[i], Q3_ERR_NULL);
    Q3_REQUIRE(n[i] >= 0, Q3_ERR_SHAPE);
    // Each DMA instruction of the tiled kernels loads 16 (or 8) weight rows
    // of one segment.
    tiled_ok = tiled_ok && (N % 16 == 0) && bf16_rows_ok(w[i], ldw, K);
    N += n[i];
  }
  Q3_REQUIRE(M >= 0 && K >= 0 && N < (1ll << 31) && ldx >= K && ldw >= K && ldc >= N, Q3_ERR_SHAPE);
  Q3_REQUIRE(dtype == Q3_F32 || dtype == Q3_BF16, Q3_ERR_DTYPE);
  if (M == 0 || N == 0) return Q3_OK;
  // One launch per segment, into its column slice of y.
  auto per_segment = [&]() -> int {
    const size_t esz = dtype == Q3_BF16 ? 2 : 4;
    int64_t col = 0;
    for (int64_t i = 0; i < nseg; ++i) {
      const int rc = matmul_impl(x, w[i], nullptr, bias ? bias[i] : nullptr, nullptr,
                                 static_cast<char*>(y) + col * esz, M, n[i], K, 1, ldx, ldw, 0, ldc, 0, 0, 0, dtype,
                                 false, ws, ws_bytes, st);
      if (rc != Q3_OK) return rc;
      col += n[i];
    }
    return Q3_OK;
  };
  const bool one = dtype == Q3_BF16 && K > 0 && bf16_rows_ok(x, ldx, K) && (M <= kGemvMaxRows || tiled_ok);
  if (!one || nseg == 1) return per_segment();
  WeightSegments seg{};
  seg.n = (int)nseg;
  int64_t col = 0;
  for (int64_t i = 0; i < nseg; ++i) {
    seg.start[i] = (int)col;
    seg.w[i] = static_cast<const bf16*>(w[i]);
    seg.b[i] = bias ? static_cast<const bf16*>(bias[i]) : nullptr;
    col += n[i];
  }
  if (M <= kGemvMaxRows) {
    GemvArgs ga{};
    ga.X = static_cast<const bf16*>(x);
    ga.ldx = ldx;
    ga.seg = seg;
    ga.C = static_cast<bf16*>(y);
    ga.ldc = ldc;
    ga.M = (int)M;
    ga.N = (int)N;
    ga.K = (int)K;
    ga.ldw = ldw;
    if (gemv_eligible(ga)) return gemv_launch(ga, ws, ws_bytes, st);
    return per_segment();
  }
  GemmParams p{};
  p.X = static_cast<const bf16*>(x);
  p.W = seg.w[0];
  p.C = static_cast<bf16*>(y);
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldc = ldc;
  p.seg = seg;
  return launch_tiled<kEpiStore>(p, 1, st);
}

// Decode-shaped RMSNorm fused into the projection that consumes it (row-owned
// GEMV, staged X path). Only bf16, 1 <= M <= 32; no workspace.
int rmsnorm_gemv_impl(const void* x, const void* norm_w, float eps, WeightSegments seg, const void* w_up, void* y,
                      int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldc, int dtype,
                      hipStream_t st) {
  Q3_REQUIRE(x && norm_w && y, Q3_ERR_NULL);
  Q3_REQUIRE(M >= 0 && N >= 0 && K >= 0 && ldx >= K && ldw >= K && ldc >= N && N < (1ll << 31), Q3_ERR_SHAPE);
  Q3_REQUIRE(M <= kGemvMaxRows, Q3_ERR_UNSUPPORTED);
  Q3_REQUIRE(dtype == Q3_BF16, Q3_ERR_DTYPE);
  Q3_REQUIRE(eps >= 0.f, Q3_ERR_SHAPE);
  if (M == 0 || N == 0) return Q3_OK;
  Q3_REQUIRE(K > 0, Q3_ERR_SHAPE);
  Q3_REQUIRE(q3_aligned(norm_w, 16), Q3_ERR_ALIGN);
  GemvArgs ga{};
  ga.X = static_cast<const bf16*>(x);
  ga.ldx = ldx;
  ga.seg = seg;
  ga.W2 = static_cast<const bf16*>(w_up);
  ga.C = static_cast<bf16*>(y);
  ga.ldc = ldc;
  ga.M = (int)M;
  ga.N = (int)N;
  ga.K = (int)K;
  ga.ldw = ldw;
  ga.nw = static_cast<const bf16*>(norm_w);
  ga.eps = eps;
  Q3_REQUIRE(gemv_eligible(ga), Q3_ERR_ALIGN);
  return gemv_launch(ga, nullptr, 0, st);
}

}  // namespace

extern "C" {

int64_t q3_matmul_segments_workspace_bytes(int64_t M, const int64_t* n, int64_t nseg, int64_t K, int dtype) {
  if (!n || nseg < 1 || nseg > 4 || dtype != Q3_BF16 || M > kGemvMaxRows || M <= 0 || K <= 0) return 0;
  // Enough for the one-launch form and for the per-segment fallback.
  int64_t N = 0, need = 0;
  for (int64_t i = 0; i < nseg; ++i) {
    if (n[i] <= 0) continue;
    N += n[i];
    need = std::max(need, gemv_workspace_bytes(M, n[i], K, false));
  }
  return N > 0 ? std::max(need, gemv_workspace_bytes(M, N, K, false)) : 0;
}

int q3_matmul_segments(const void* x, const void* const* w, const void* const* bias, const int64_t* n, int64_t nseg,
                       void* y, int64_t M, int64_t K, int64_t ldx, int64_t ldw, int64_t ldc, int dtype,
                       void* workspace, int64_t workspace_bytes, void* stream) {
  return segments_impl(x, w, bias, n, nseg, y, M, K, ldx, ldw, ldc, dtype, workspace, workspace_bytes,
                       static_cast<hipStream_t>(stream));
}

int64_t q3_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K, int dtype, int swiglu) {
  if (dtype != Q3_BF16 || M <= 0 || N <= 0 || K <= 0) return 0;
  if (M > kGemvMaxRows) return swiglu ? 0 : split_k_workspace_bytes(M, N, K);
  return gemv_workspace_bytes(M, N, K, swiglu != 0);
}

int q3_matmul(const void* x, const void* w, const void* bias, const void* residual, void* y, int64_t M, int64_t N,
              int64_t K, int64_t ldx, int64_t ldw, int64_t ldr, int64_t ldc, int dtype, void* workspace,
              int64_t workspace_bytes, void* stream) {
  return matmul_impl(x, w, nullptr, bias, residual, y, M, N, K, 1, ldx, ldw, ldr, ldc, 0, 0, 0, dtype, false,
                     workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int q3_matmul_gelu(const void* x, const void* w, const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                   int64_t ldx, int64_t ldw, int64_t ldc, int dtype, void* stream) {
  return matmul_impl(x, w, nullptr, bias, nullptr, y, M, N, K, 1, ldx, ldw, 0, ldc, 0, 0, 0, dtype, false, nullptr,
                     0, static_cast<hipStream_t>(stream), 1);
}

int q3_matmul_swiglu(const void* x, const void* w_gate, const void* w_up, void* y, int64_t M, int64_t N, int64_t K,
                     int64_t ldx, int64_t ldw, int64_t ldc, int dtype, void* workspace, int64_t workspace_bytes,
                     void* stream) {
  return matmul_impl(x, w_gate, w_up, nullptr, nullptr, y, M, N, K, 1, ldx, ldw, 0, ldc, 0, 0, 0, dtype, true,
                     workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int q3_rmsnorm_matmul_segments(const void* x, const void* norm_w, float eps, const void* const* w,
                               const void* const* bias, const int64_t* n, int64_t nseg, void* y, int64_t M, int64_t K,
                               int64_t ldx, int64_t ldw, int64_t ldc, int dtype, void* stream) {
  Q3_REQUIRE(w && n, Q3_ERR_NULL);
  Q3_REQUIRE(nseg >= 1 && nseg <= 4, Q3_ERR_SHAPE);
  WeightSegments seg{};
  seg.n = (int)nseg;
  int64_t N = 0;
  for (int64_t i = 0; i < nseg; ++i) {
    Q3_REQUIRE(w[i], Q3_ERR_NULL);
    Q3_REQUIRE(n[i] >= 0, Q3_ERR_SHAPE);
    seg.start[i] = (int)N;
    seg.w[i] = static_cast<const bf16*>(w[i]);
    seg.b[i] = bias ? static_cast<const bf16*>(bias[i]) : nullptr;
    N += n[i];
  }
  return rmsnorm_gemv_impl(x, norm_w, eps, seg, nullptr, y, M, N, K, ldx, ldw, ldc, dtype,
                           static_cast<hipStream_t>(stream));
}

int q3_rmsnorm_matmul_swiglu(const void* x, const void* norm_w, float eps, const void* w_gate, const void* w_up,
                             void* y, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldc,
                             int dtype, void* stream) {
  Q3_REQUIRE(w_gate && w_up, Q3_ERR_NULL);
  WeightSegments seg{};
  seg.n = 1;
  seg.w[0] = static_cast<const bf16*>(w_gate);
  return rmsnorm_gemv_impl(x, norm_w, eps, seg, w_up, y, M, N, K, ldx, ldw, ldc, dtype,
                           static_cast<hipStream_t>(stream));
}

int q3_batched_gemm(const void* x, const void* w, void* y, int64_t E, int64_t M, int64_t N, int64_t K, int dtype,
                    void* stream) {
  Q3_REQUIRE(E >= 1, Q3_ERR_SHAPE);
  // Batched problems always use the tiled (or generic) path: no workspace.
  if (M <= 32 && dtype == Q3_BF16 && M > 0) {
    // Route small per-batch M through the tiled kernel (it masks rows).
    GemmParams p{};
    Q3_REQUIRE(x && w && y, Q3_ERR_NULL);
    if (!(bf16_rows_ok(x, K, K) && bf16_rows_ok(w, K, K)))
      return launch_generic<bf16>(x, w, nullptr, nullptr, nullptr, y, M, N, K, E, K, K, 0, N, M * K, N * K, M * N,
                                  false, static_cast<hipStream_t>(stream));
    p.X = static_cast<const bf16*>(x);
    p.W = static_cast<const bf16*>(w);
    p.C = static_cast<bf16*>(y);
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.ldx = K;
    p.ldw = K;
    p.ldc = N;
    p.bsX = M * K;
    p.bsW = N * K;
    p.bsC = M * N;
    return launch_tiled_cfg<128, 128, 2, 2, kEpiStore, 4, 32>(p, E, static_cast<hipStream_t>(stream));
  }
  return matmul_impl(x, w, nullptr, nullptr, nullptr, y, M, N, K, E, K, K, 0, N, M * K, N * K, M * N, dtype, false,
                     nullptr, 0, static_cast<hipStream_t>(stream));
}

}  // extern "C"
