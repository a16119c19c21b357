// GEMM entry points of the C-ABI: q3_matmul, q3_matmul_swiglu, q3_batched_gemm.
//
//   Y[m, n] = sum_k X[m, k] * W[n, k] (+ bias[n]) (+ R[m, n])   (nn.Linear layout)
//
// Three device paths, chosen on the host from the shape:
//  * tiled   : bf16, M > 32     -> 32x32x16 MFMA, LDS double-buffered tiles
//  * skinny  : bf16, M <= 32    -> weight-streaming MFMA kernel (decode GEMV-like
//                                  shapes), optional deterministic split-K
//  * generic : fp32, or bf16 whose rows are not 16-byte aligned -> SIMT fp32
#include "gemm_kernels.h"

using namespace q3;

// =====================================================================
// Skinny path: M <= 32. One block = 4 waves = 32 output columns over a K range;
// each wave streams its quarter of the K range in steps of 64. A lane reads
// 64 contiguous bytes of one weight row (and of one X row) per step and feeds
// them to 4 MFMAs: in step s, element t of MFMA v is k = s*64 + 32*(lane/32) +
// 8*v + t for both operands, a consistent k permutation.
// =====================================================================
namespace {

constexpr int kSkinnyWaves = 4;
constexpr int kSkinnyUnroll = 2;  // k steps per wave iteration (loads in flight)

struct SkinnyParams {
  const bf16* X;    // (M <= 32, K)
  const bf16* W;    // gate / plain weight (N, K)
  const bf16* W2;   // up weight for SwiGLU, or null
  const bf16* bias;
  const bf16* R;
  bf16* C;
  float* partial;   // (ksplit, 32, n_acc) fp32 when ksplit > 1
  int M, N, K;
  int64_t ldx, ldw, ldr, ldc;
  int ksplit;
  int k_per_split;  // multiple of 64*kSkinnyWaves except possibly the last
  WeightSegments seg;  // stacked weights (plain store only); starts are multiples of 32
};

// Bias of output column n, re-based like the weights of its segment.
__device__ __forceinline__ const bf16* skinny_bias(const SkinnyParams& p, int n) {
  if (p.seg.n <= 1) return p.bias;
  const int s = segment_of(p.seg, n);
  return p.seg.b[s] ? p.seg.b[s] - p.seg.start[s] : nullptr;
}

template <bool SWIGLU>
__device__ __forceinline__ void skinny_epilogue(const SkinnyParams& p, const bf16* bias, int m, int n, float g,
                                                float u) {
  if (m >= p.M || n >= p.N) return;
  float v;
  if constexpr (SWIGLU) {
    v = g / (1.0f + __expf(-g)) * u;
  } else {
    v = g;
    if (bias) v += bf2f(bias[n]);
    if (p.R) v += bf2f(p.R[(int64_t)m * p.ldr + n]);
  }
  p.C[(int64_t)m * p.ldc + n] = f2bf(v);
}

template <bool SWIGLU>
__global__ __launch_bounds__(kSkinnyWaves * 64) void gemm_skinny_kernel(const SkinnyParams p) {
  constexpr int NACC = SWIGLU ? 2 : 1;
  __shared__ float red[kSkinnyWaves][NACC][32 * 32 + 32];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int h = lane >> 5;
  const int n0 = blockIdx.x * 32;
  const int split = blockIdx.y;

  const int kb = split * p.k_per_split;
  const int ke = min(p.K, kb + p.k_per_split);

  // Stacked weights: re-base W so that column n addresses row n of its segment.
  const bf16* Wp = p.W;
  int n_base = 0, n_lim = p.N;
  if (!SWIGLU && p.seg.n > 1) {
    const int s = segment_of(p.seg, n0);
    n_base = p.seg.start[s];
    n_lim = s + 1 < p.seg.n ? p.seg.start[s + 1] : p.N;
    Wp = p.seg.w[s] - (int64_t)n_base * p.ldw;
  }
  const bf16* bias = skinny_bias(p, n0);
  const int n = n0 + l32;
  const bool nvalid = n < n_lim;
  const bool mvalid = l32 < p.M;
  const bf16* wrow = Wp + (int64_t)(nvalid ? n : n_base) * p.ldw;
  const bf16* wrow2 = SWIGLU ? p.W2 + (int64_t)(nvalid ? n : 0) * p.ldw : nullptr;
  const bf16* xrow = p.X + (int64_t)(mvalid ? l32 : 0) * p.ldx;

  floatx16 acc[NACC];
#pragma unroll
  for (int a = 0; a < NACC; ++a) acc[a] = floatx16{};

  // Wave w handles steps w, w + 4, w + 8, ... of 64 elements in [kb, ke),
  // kSkinnyUnroll steps per iteration with all their loads issued up front.
  constexpr int U = kSkinnyUnroll;
  for (int k = kb + wave * 64; k < ke; k += 64 * kSkinnyWaves * U) {
    bf16x8 wa[U][4], wb[U][4], xb[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k + u * 64 * kSkinnyWaves + 32 * h;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int kv = kk + 8 * v;
        const bool kin = kv < ke;
        wa[u][v] = (nvalid && kin) ? *reinterpret_cast<const bf16x8*>(wrow + kv) : bf16x8{};
        if constexpr (SWIGLU) wb[u][v] = (nvalid && kin) ? *reinterpret_cast<const bf16x8*>(wrow2 + kv) : bf16x8{};
        xb[u][v] = (mvalid && kin) ? *reinterpret_cast<const bf16x8*>(xrow + kv) : bf16x8{};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        acc[0] = mfma32x32x16(wa[u][v], xb[u][v], acc[0]);
        if constexpr (SWIGLU) acc[1] = mfma32x32x16(wb[u][v], xb[u][v], acc[1]);
      }
  }

  // Cross-wave reduction through LDS. Register r of lane l holds output
  // (m = l % 32, n = 8*(r/4) + 4*(l/32) + r%4); stored as red[n][m] with a
  // 33-float row pitch.
#pragma unroll
  for (int a = 0; a < NACC; ++a)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int nn = 8 * (r >> 2) + 4 * h + (r & 3);
      red[wave][a][nn * 33 + l32] = acc[a][r];
    }
  __syncthreads();
  // 1024 outputs, 4 per thread.
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int idx = tid + e * 256;
    const int nn = idx >> 5;
    const int m = idx & 31;
    float s[NACC];
#pragma unroll
    for (int a = 0; a < NACC; ++a) {
      s[a] = 0.f;
#pragma unroll
      for (int w = 0; w < kSkinnyWaves; ++w) s[a] += red[w][a][nn * 33 + m];
    }
    if (p.ksplit == 1) {
      skinny_epilogue<SWIGLU>(p, bias, m, n0 + nn, s[0], NACC > 1 ? s[NACC - 1] : 0.f);
    } else {
      const int ncols = p.N * NACC;
      float* dst = p.partial + ((int64_t)split * 32 + m) * ncols;
#pragma unroll
      for (int a = 0; a < NACC; ++a)
        if (n0 + nn < p.N) dst[(int64_t)a * p.N + n0 + nn] = s[a];
    }
  }
}

template <bool SWIGLU>
__global__ void gemm_skinny_finalize(const SkinnyParams p) {
  const int NACC = SWIGLU ? 2 : 1;
  const int64_t total = (int64_t)p.M * p.N;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(i / p.N);
    const int n = (int)(i % p.N);
    float s[2] = {0.f, 0.f};
    for (int sp = 0; sp < p.ksplit; ++sp) {
      const float* src = p.partial + ((int64_t)sp * 32 + m) * (int64_t)p.N * NACC;
      s[0] += src[n];
      if (SWIGLU) s[1] += src[p.N + n];
    }
    skinny_epilogue<SWIGLU>(p, skinny_bias(p, n), m, n, s[0], s[1]);
  }
}

int skinny_ksplit(int64_t N, int64_t K) {
  const int64_t blocks = q3_cdiv(N, 32);
  int ks = 1;
  // Aim for >= 512 blocks (2 per CU) while each wave keeps >= 256 elements of K.
  while (blocks * ks < 512 && K / (ks * 2) >= 256 * kSkinnyWaves / 2 && ks < 16) ks *= 2;
  return ks;
}

int64_t skinny_workspace_bytes(int64_t N, int64_t K, bool swiglu) {
  const int ks = skinny_ksplit(N, K);
  if (ks == 1) return 0;
  return (int64_t)ks * 32 * N * (swiglu ? 2 : 1) * (int64_t)sizeof(float);
}

template <bool SWIGLU>
int launch_skinny(SkinnyParams p, void* ws, int64_t ws_bytes, hipStream_t st) {
  const int ks = skinny_ksplit(p.N, p.K);
  p.ksplit = ks;
  // Split boundaries on multiples of 64 so every wave step is whole.
  int64_t kps = q3_cdiv(p.K, ks);
  kps = q3_cdiv(kps, 64) * 64;
  p.k_per_split = (int)kps;
  p.partial = nullptr;
  if (ks > 1) {
    Q3_REQUIRE(ws != nullptr && ws_bytes >= skinny_workspace_bytes(p.N, p.K, SWIGLU), Q3_ERR_WORKSPACE);
    p.partial = static_cast<float*>(ws);
  }
  dim3 grid((unsigned)q3_cdiv(p.N, 32), (unsigned)ks);
  hipLaunchKernelGGL(gemm_skinny_kernel<SWIGLU>, grid, dim3(kSkinnyWaves * 64), 0, st, p);
  Q3_LAUNCH_CHECK();
  if (ks > 1) {
    const int64_t total = (int64_t)p.M * p.N;
    const unsigned blocks = (unsigned)std::min<int64_t>(q3_cdiv(total, 256), 2048);
    hipLaunchKernelGGL(gemm_skinny_finalize<SWIGLU>, dim3(blocks), dim3(256), 0, st, p);
    Q3_LAUNCH_CHECK();
  }
  return Q3_OK;
}

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
                                                           const T* __restrict__ W2) {
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
        if (R) v += to_f(R[(int64_t)m * ldr + n]);
      }
      C[(int64_t)m * ldc + n] = from_f<T>(v);
    }
}

template <typename T>
int launch_generic(const void* x, const void* w, const void* w2, const void* bias, const void* r, void* y, int64_t M,
                   int64_t N, int64_t K, int64_t batch, int64_t ldx, int64_t ldw, int64_t ldr, int64_t ldc,
                   int64_t bsX, int64_t bsW, int64_t bsC, bool swiglu, hipStream_t st) {
  dim3 grid((unsigned)q3_cdiv(N, 64), (unsigned)q3_cdiv(M, 64), (unsigned)batch);
  hipLaunchKernelGGL(gemm_generic_kernel<T>, grid, dim3(256), 0, st, static_cast<const T*>(x),
                     static_cast<const T*>(w), static_cast<const T*>(bias), static_cast<const T*>(r),
                     static_cast<T*>(y), (int)M, (int)N, (int)K, ldx, ldw, ldr, ldc, bsX, bsW, bsC, swiglu ? 1 : 0,
                     static_cast<const T*>(w2));
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

// =====================================================================
// Tiled MFMA path.
// =====================================================================
template <int BM, int BN, int WM, int WN, int EPI>
int launch_tiled_cfg(GemmParams p, int64_t batch, hipStream_t st) {
  constexpr int BN_OUT = (EPI == kEpiSwiGLU) ? BN / 2 : BN;
  const int64_t tiles = q3_cdiv(p.M, BM) * q3_cdiv(p.N, BN_OUT);
  p.group_m = 8;
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, EPI, false>), dim3((unsigned)tiles, 1, (unsigned)batch),
                     dim3(WM * WN * 64), 0, st, p);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

template <int EPI>
int launch_tiled(GemmParams p, int64_t batch, hipStream_t st) {
  // Big tiles when they still give at least one full wave of 256 CUs.
  const int64_t big = q3_cdiv(p.M, 256) * q3_cdiv(p.N, EPI == kEpiSwiGLU ? 128 : 256) * batch;
  if (big >= 256) return launch_tiled_cfg<256, 256, 2, 4, EPI>(p, batch, st);
  return launch_tiled_cfg<128, 128, 2, 2, EPI>(p, batch, st);
}

bool bf16_rows_ok(const void* base, int64_t ld, int64_t K) {
  return q3_aligned(base, 16) && (ld % 8 == 0) && (K % 8 == 0);
}

int matmul_impl(const void* x, const void* w, const void* w2, const void* bias, const void* residual, void* y,
                int64_t M, int64_t N, int64_t K, int64_t batch, int64_t ldx, int64_t ldw, int64_t ldr, int64_t ldc,
                int64_t bsX, int64_t bsW, int64_t bsC, int dtype, bool swiglu, void* ws, int64_t ws_bytes,
                hipStream_t st) {
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
                                 swiglu, st);
  const bool rows_ok = bf16_rows_ok(x, ldx, K) && bf16_rows_ok(w, ldw, K) && (!w2 || bf16_rows_ok(w2, ldw, K)) &&
                       (bsX % 8 == 0) && (bsW % 8 == 0);
  if (!rows_ok || K == 0)
    return launch_generic<bf16>(x, w, w2, bias, residual, y, M, N, K, batch, ldx, ldw, ldr, ldc, bsX, bsW, bsC,
                                swiglu, st);
  if (M <= 32 && batch == 1) {
    SkinnyParams sp{};
    sp.X = static_cast<const bf16*>(x);
    sp.W = static_cast<const bf16*>(w);
    sp.W2 = static_cast<const bf16*>(w2);
    sp.bias = static_cast<const bf16*>(bias);
    sp.R = static_cast<const bf16*>(residual);
    sp.C = static_cast<bf16*>(y);
    sp.M = (int)M;
    sp.N = (int)N;
    sp.K = (int)K;
    sp.ldx = ldx;
    sp.ldw = ldw;
    sp.ldr = ldr;
    sp.ldc = ldc;
    return swiglu ? launch_skinny<true>(sp, ws, ws_bytes, st) : launch_skinny<false>(sp, ws, ws_bytes, st);
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
  return swiglu ? launch_tiled<kEpiSwiGLU>(p, batch, st) : launch_tiled<kEpiStore>(p, batch, st);
}

int segments_impl(const void* x, const void* const* w, const void* const* bias, const int64_t* n, int64_t nseg,
                  void* y, int64_t M, int64_t K, int64_t ldx, int64_t ldw, int64_t ldc, int dtype, void* ws,
                  int64_t ws_bytes, hipStream_t st) {
  Q3_REQUIRE(x && w && n && y, Q3_ERR_NULL);
  Q3_REQUIRE(nseg >= 1 && nseg <= 4, Q3_ERR_SHAPE);
  int64_t N = 0;
  bool tiled_ok = true, skinny_ok = true;
  for (int64_t i = 0; i < nseg; ++i) {
    Q3_REQUIRE(w[i], Q3_ERR_NULL);
    Q3_REQUIRE(n[i] >= 0, Q3_ERR_SHAPE);
    tiled_ok = tiled_ok && (N % 256 == 0) && bf16_rows_ok(w[i], ldw, K);
    skinny_ok = skinny_ok && (N % 32 == 0) && bf16_rows_ok(w[i], ldw, K);
    N += n[i];
  }
  Q3_REQUIRE(M >= 0 && K >= 0 && N < (1ll << 31) && ldx >= K && ldw >= K && ldc >= N, Q3_ERR_SHAPE);
  Q3_REQUIRE(dtype == Q3_F32 || dtype == Q3_BF16, Q3_ERR_DTYPE);
  if (M == 0 || N == 0) return Q3_OK;
  const bool one = dtype == Q3_BF16 && K > 0 && bf16_rows_ok(x, ldx, K) && (M <= 32 ? skinny_ok : tiled_ok);
  if (!one || nseg == 1) {
    // One launch per segment, into its column slice of y.
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
  }
  WeightSegments seg{};
  seg.n = (int)nseg;
  int64_t col = 0;
  for (int64_t i = 0; i < nseg; ++i) {
    seg.start[i] = (int)col;
    seg.w[i] = static_cast<const bf16*>(w[i]);
    seg.b[i] = bias ? static_cast<const bf16*>(bias[i]) : nullptr;
    col += n[i];
  }
  if (M <= 32) {
    SkinnyParams sp{};
    sp.X = static_cast<const bf16*>(x);
    sp.W = seg.w[0];
    sp.C = static_cast<bf16*>(y);
    sp.M = (int)M;
    sp.N = (int)N;
    sp.K = (int)K;
    sp.ldx = ldx;
    sp.ldw = ldw;
    sp.ldc = ldc;
    sp.seg = seg;
    return launch_skinny<false>(sp, ws, ws_bytes, st);
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

}  // namespace

extern "C" {

int64_t q3_matmul_segments_workspace_bytes(int64_t M, const int64_t* n, int64_t nseg, int64_t K, int dtype) {
  if (!n || nseg < 1 || nseg > 4 || dtype != Q3_BF16 || M > 32 || M <= 0 || K <= 0) return 0;
  int64_t N = 0, need = 0;
  for (int64_t i = 0; i < nseg; ++i) {
    if (n[i] <= 0) continue;
    N += n[i];
    need = std::max(need, skinny_workspace_bytes(n[i], K, false));
  }
  return N > 0 ? std::max(need, skinny_workspace_bytes(N, K, false)) : 0;
}

int q3_matmul_segments(const void* x, const void* const* w, const void* const* bias, const int64_t* n, int64_t nseg,
                       void* y, int64_t M, int64_t K, int64_t ldx, int64_t ldw, int64_t ldc, int dtype,
                       void* workspace, int64_t workspace_bytes, void* stream) {
  return segments_impl(x, w, bias, n, nseg, y, M, K, ldx, ldw, ldc, dtype, workspace, workspace_bytes,
                       static_cast<hipStream_t>(stream));
}

int64_t q3_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K, int dtype, int swiglu) {
  if (dtype != Q3_BF16 || M > 32 || M <= 0 || N <= 0 || K <= 0) return 0;
  return skinny_workspace_bytes(N, K, swiglu != 0);
}

int q3_matmul(const void* x, const void* w, const void* bias, const void* residual, void* y, int64_t M, int64_t N,
              int64_t K, int64_t ldx, int64_t ldw, int64_t ldr, int64_t ldc, int dtype, void* workspace,
              int64_t workspace_bytes, void* stream) {
  return matmul_impl(x, w, nullptr, bias, residual, y, M, N, K, 1, ldx, ldw, ldr, ldc, 0, 0, 0, dtype, false,
                     workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int q3_matmul_swiglu(const void* x, const void* w_gate, const void* w_up, void* y, int64_t M, int64_t N, int64_t K,
                     int64_t ldx, int64_t ldw, int64_t ldc, int dtype, void* workspace, int64_t workspace_bytes,
                     void* stream) {
  return matmul_impl(x, w_gate, w_up, nullptr, nullptr, y, M, N, K, 1, ldx, ldw, 0, ldc, 0, 0, 0, dtype, true,
                     workspace, workspace_bytes, static_cast<hipStream_t>(stream));
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
    return launch_tiled_cfg<128, 128, 2, 2, kEpiStore>(p, E, static_cast<hipStream_t>(stream));
  }
  return matmul_impl(x, w, nullptr, nullptr, nullptr, y, M, N, K, E, K, K, 0, N, M * K, N * K, M * N, dtype, false,
                     nullptr, 0, static_cast<hipStream_t>(stream));
}

}  // extern "C"
