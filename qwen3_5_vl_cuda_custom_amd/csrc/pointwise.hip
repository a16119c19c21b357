// Elementwise and row-reduction kernels: residual_add, swiglu, gelu_tanh,
// rmsnorm, layernorm, softmax, top-k. All are HBM-bound; rows are handled by
// aligned groups of G lanes of a wave64 (G = 8..64), each lane holding VPT
// 16-byte vectors in registers, so a row is read once and written once and
// reductions are lane shuffles with no LDS and no barriers.
#include <algorithm>

#include "q3_common.h"

namespace {

// ===================================================================== elementwise
enum EwOp : int { kAdd = 0, kSwiGLU = 1, kGelu = 2 };

template <int OP>
__device__ __forceinline__ float ew_apply(float a, float b) {
  if constexpr (OP == kAdd) {
    return a + b;
  } else if constexpr (OP == kSwiGLU) {
    return a / (1.0f + expf(-a)) * b;
  } else {
    return gelu_tanh_f(a);
  }
}

template <typename T, int OP, bool VEC>
__global__ __launch_bounds__(256) void ew_kernel(const T* __restrict__ a, const T* __restrict__ b, T* __restrict__ y,
                                                 int64_t n) {
  constexpr int V = Vec16<T>::N;
  typedef typename Vec16<T>::type VT;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i0 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if constexpr (VEC) {
    const int64_t nv = n / V;
    for (int64_t i = i0; i < nv; i += stride) {
      const VT va = reinterpret_cast<const VT*>(a)[i];
      VT vb{};
      if constexpr (OP != kGelu) vb = reinterpret_cast<const VT*>(b)[i];
      VT vy;
#pragma unroll
      for (int j = 0; j < V; ++j) vy[j] = from_f<T>(ew_apply<OP>(to_f<T>(va[j]), to_f<T>(vb[j])));
      reinterpret_cast<VT*>(y)[i] = vy;
    }
    for (int64_t i = nv * V + i0; i < n; i += stride) {
      const float vb = (OP != kGelu) ? to_f<T>(b[i]) : 0.f;
      y[i] = from_f<T>(ew_apply<OP>(to_f<T>(a[i]), vb));
    }
  } else {
    for (int64_t i = i0; i < n; i += stride) {
      const float vb = (OP != kGelu) ? to_f<T>(b[i]) : 0.f;
      y[i] = from_f<T>(ew_apply<OP>(to_f<T>(a[i]), vb));
    }
  }
}

template <typename T, int OP>
int launch_ew(const void* a, const void* b, void* y, int64_t n, hipStream_t st) {
  constexpr int V = Vec16<T>::N;
  const bool vec = q3_aligned(a, 16) && q3_aligned(y, 16) && (OP == kGelu || q3_aligned(b, 16));
  const int64_t work = vec ? q3_cdiv(n, V) : n;
  const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(q3_cdiv(work, 256), 256 * 16));
  if (vec)
    hipLaunchKernelGGL((ew_kernel<T, OP, true>), dim3(blocks), dim3(256), 0, st, static_cast<const T*>(a),
                       static_cast<const T*>(b), static_cast<T*>(y), n);
  else
    hipLaunchKernelGGL((ew_kernel<T, OP, false>), dim3(blocks), dim3(256), 0, st, static_cast<const T*>(a),
                       static_cast<const T*>(b), static_cast<T*>(y), n);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

template <int OP>
int ew_entry(const void* a, const void* b, void* y, int64_t n, int dtype, void* stream) {
  Q3_REQUIRE(a && y && (OP == kGelu || b), Q3_ERR_NULL);
  Q3_REQUIRE(n >= 0, Q3_ERR_SHAPE);
  if (n == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == Q3_BF16) return launch_ew<bf16, OP>(a, b, y, n, st);
  if (dtype == Q3_F32) return launch_ew<float, OP>(a, b, y, n, st);
  return Q3_ERR_DTYPE;
}

// ===================================================================== row norms
enum NormKind : int { kRMS = 0, kLayer = 1 };

// Rows of `cols` elements, G lanes per row (runtime power of two), VPT
// 16-byte vectors per lane; lane j of a row group holds vectors j, j+G, ...
template <typename T, int VPT, int KIND>
__global__ __launch_bounds__(256) void norm_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                   const T* __restrict__ bias, T* __restrict__ y, int64_t rows,
                                                   int cols, int G, float eps) {
  constexpr int V = Vec16<T>::N;
  typedef typename Vec16<T>::type VT;
  const int lane = threadIdx.x & 63;
  const int rows_per_wave = 64 / G;
  const int64_t wave_id = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  const int64_t row = wave_id * rows_per_wave + lane / G;
  const int j = lane % G;
  const bool valid = row < rows;
  const T* xr = x + (valid ? row : 0) * (int64_t)cols;

  // The weight (and bias) vectors load with the row, so one memory round trip
  // covers every operand (small-row calls are latency-bound).
  float v[VPT][V];
  VT wv[VPT], bv[VPT];
#pragma unroll
  for (int t = 0; t < VPT; ++t) {
    const VT u = valid ? reinterpret_cast<const VT*>(xr)[j + t * G] : VT{};
    wv[t] = reinterpret_cast<const VT*>(w)[j + t * G];
    bv[t] = (KIND == kLayer && bias) ? reinterpret_cast<const VT*>(bias)[j + t * G] : VT{};
#pragma unroll
    for (int e = 0; e < V; ++e) v[t][e] = to_f<T>(u[e]);
  }
  float mean = 0.f;
  if constexpr (KIND == kLayer) {
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < VPT; ++t)
#pragma unroll
      for (int e = 0; e < V; ++e) s += v[t][e];
    for (int o = G / 2; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    mean = s / (float)cols;
  }
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < VPT; ++t)
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float d = v[t][e] - mean;
      ss += d * d;
    }
  for (int o = G / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float rstd = rsqrtf(ss / (float)cols + eps);
  if (!valid) return;
  T* yr = y + row * (int64_t)cols;
#pragma unroll
  for (int t = 0; t < VPT; ++t) {
    const int vi = j + t * G;
    VT out;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      float o = (v[t][e] - mean) * rstd * to_f<T>(wv[t][e]);
      if (KIND == kLayer && bias) o += to_f<T>(bv[t][e]);
      out[e] = from_f<T>(o);
    }
    reinterpret_cast<VT*>(yr)[vi] = out;
  }
}

// Any shape / alignment: one wave per row, two passes over global memory.
template <typename T, int KIND>
__global__ __launch_bounds__(256) void norm_generic_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                           const T* __restrict__ bias, T* __restrict__ y,
                                                           int64_t rows, int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  if (row >= rows) return;
  const T* xr = x + row * (int64_t)cols;
  float mean = 0.f;
  if (KIND == kLayer) {
    float s = 0.f;
    for (int c = lane; c < cols; c += 64) s += to_f<T>(xr[c]);
    mean = wave_sum(s) / (float)cols;
  }
  float ss = 0.f;
  for (int c = lane; c < cols; c += 64) {
    const float d = to_f<T>(xr[c]) - mean;
    ss += d * d;
  }
  const float rstd = rsqrtf(wave_sum(ss) / (float)cols + eps);
  T* yr = y + row * (int64_t)cols;
  for (int c = lane; c < cols; c += 64) {
    float o = (to_f<T>(xr[c]) - mean) * rstd * to_f<T>(w[c]);
    if (KIND == kLayer && bias) o += to_f<T>(bias[c]);
    yr[c] = from_f<T>(o);
  }
}

template <typename T, int KIND, int VPT>
bool try_norm(const void* x, const void* w, const void* b, void* y, int64_t rows, int cols, float eps, int nvec,
              hipStream_t st, int* rc) {
  // Pick the widest G in {64, 32, 16, 8} with nvec == G * VPT.
  for (int G = 64; G >= 8; G >>= 1) {
    if (nvec == G * VPT) {
      const int64_t rows_per_block = 4 * (64 / G);
      const unsigned blocks = (unsigned)q3_cdiv(rows, rows_per_block);
      hipLaunchKernelGGL((norm_kernel<T, VPT, KIND>), dim3(blocks), dim3(256), 0, st, static_cast<const T*>(x),
                         static_cast<const T*>(w), static_cast<const T*>(b), static_cast<T*>(y), rows, cols, G, eps);
      hipError_t e = hipGetLastError();
      *rc = (e == hipSuccess) ? Q3_OK : (int)e;
      return true;
    }
  }
  return false;
}

template <typename T, int KIND>
int launch_norm(const void* x, const void* w, const void* b, void* y, int64_t rows, int cols, float eps,
                hipStream_t st) {
  constexpr int V = Vec16<T>::N;
  const bool vec = (cols % V == 0) && q3_aligned(x, 16) && q3_aligned(w, 16) && q3_aligned(y, 16) &&
                   (b == nullptr || q3_aligned(b, 16));
  int rc = Q3_OK;
  if (vec) {
    const int nvec = cols / V;
    if (try_norm<T, KIND, 1>(x, w, b, y, rows, cols, eps, nvec, st, &rc) ||
        try_norm<T, KIND, 2>(x, w, b, y, rows, cols, eps, nvec, st, &rc) ||
        try_norm<T, KIND, 3>(x, w, b, y, rows, cols, eps, nvec, st, &rc) ||
        try_norm<T, KIND, 4>(x, w, b, y, rows, cols, eps, nvec, st, &rc) ||
        try_norm<T, KIND, 5>(x, w, b, y, rows, cols, eps, nvec, st, &rc) ||
        try_norm<T, KIND, 6>(x, w, b, y, rows, cols, eps, nvec, st, &rc) ||
        try_norm<T, KIND, 8>(x, w, b, y, rows, cols, eps, nvec, st, &rc) ||
        try_norm<T, KIND, 9>(x, w, b, y, rows, cols, eps, nvec, st, &rc) ||
        try_norm<T, KIND, 12>(x, w, b, y, rows, cols, eps, nvec, st, &rc) ||
        try_norm<T, KIND, 16>(x, w, b, y, rows, cols, eps, nvec, st, &rc))
      return rc;
  }
  const unsigned blocks = (unsigned)q3_cdiv(rows, 4);
  hipLaunchKernelGGL((norm_generic_kernel<T, KIND>), dim3(blocks), dim3(256), 0, st, static_cast<const T*>(x),
                     static_cast<const T*>(w), static_cast<const T*>(b), static_cast<T*>(y), rows, cols, eps);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

template <int KIND>
int norm_entry(const void* x, const void* w, const void* b, void* y, int64_t rows, int64_t cols, float eps, int dtype,
               void* stream) {
  Q3_REQUIRE(x && w && y, Q3_ERR_NULL);
  Q3_REQUIRE(rows >= 0 && cols >= 1 && cols < (1 << 24), Q3_ERR_SHAPE);
  if (rows == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == Q3_BF16) return launch_norm<bf16, KIND>(x, w, b, y, rows, (int)cols, eps, st);
  if (dtype == Q3_F32) return launch_norm<float, KIND>(x, w, b, y, rows, (int)cols, eps, st);
  return Q3_ERR_DTYPE;
}

// ===================================================================== softmax
// One wave per row; three passes over the row (max, sum, write) that hit L1/L2
// after the first.
template <typename T>
__global__ __launch_bounds__(256) void softmax_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t rows,
                                                      int cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  if (row >= rows) return;
  const T* xr = x + row * (int64_t)cols;
  float m = -INFINITY;
  for (int c = lane; c < cols; c += 64) m = fmaxf(m, to_f<T>(xr[c]));
  m = wave_max(m);
  float s = 0.f;
  for (int c = lane; c < cols; c += 64) s += expf(to_f<T>(xr[c]) - m);
  s = wave_sum(s);
  const float inv = 1.0f / s;
  T* yr = y + row * (int64_t)cols;
  for (int c = lane; c < cols; c += 64) yr[c] = from_f<T>(expf(to_f<T>(xr[c]) - m) * inv);
}

// ===================================================================== top-k
// One wave per row, the row in registers (up to 64*MAXV values). k rounds of
// a wave arg-max in which the larger value wins and, among equal values, the
// lower index: the reference's tie rule.
struct KV {
  float v;
  int i;
};
__device__ __forceinline__ bool kv_better(float av, int ai, float bv, int bi) {
  return av > bv || (av == bv && ai < bi);
}

template <typename T, int MAXV>
__global__ __launch_bounds__(256) void topk_kernel(const T* __restrict__ x, T* __restrict__ vals,
                                                   int64_t* __restrict__ idx, int64_t rows, int cols, int k) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  if (row >= rows) return;
  const T* xr = x + row * (int64_t)cols;
  float v[MAXV];
  bool live[MAXV];
#pragma unroll
  for (int t = 0; t < MAXV; ++t) {
    const int c = lane + 64 * t;
    live[t] = c < cols;
    v[t] = live[t] ? to_f<T>(xr[c]) : -INFINITY;
  }
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int t = 0; t < MAXV; ++t) {
      const int c = lane + 64 * t;
      if (live[t] && kv_better(v[t], c, bv, bi)) {
        bv = v[t];
        bi = c;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (kv_better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    // bi is now uniform across the wave.
    if (lane == (bi & 63)) {
#pragma unroll
      for (int t = 0; t < MAXV; ++t)
        if (lane + 64 * t == bi) live[t] = false;
    }
    if (lane == 0) {
      vals[row * k + r] = from_f<T>(bv);
      idx[row * k + r] = bi;
    }
  }
}

template <typename T>
int launch_topk(const void* x, void* vals, int64_t* idx, int64_t rows, int cols, int k, hipStream_t st) {
  const unsigned blocks = (unsigned)q3_cdiv(rows, 4);
  const T* xp = static_cast<const T*>(x);
  T* vp = static_cast<T*>(vals);
  if (cols <= 64)
    hipLaunchKernelGGL((topk_kernel<T, 1>), dim3(blocks), dim3(256), 0, st, xp, vp, idx, rows, cols, k);
  else if (cols <= 128)
    hipLaunchKernelGGL((topk_kernel<T, 2>), dim3(blocks), dim3(256), 0, st, xp, vp, idx, rows, cols, k);
  else if (cols <= 256)
    hipLaunchKernelGGL((topk_kernel<T, 4>), dim3(blocks), dim3(256), 0, st, xp, vp, idx, rows, cols, k);
  else if (cols <= 512)
    hipLaunchKernelGGL((topk_kernel<T, 8>), dim3(blocks), dim3(256), 0, st, xp, vp, idx, rows, cols, k);
  else if (cols <= 1024)
    hipLaunchKernelGGL((topk_kernel<T, 16>), dim3(blocks), dim3(256), 0, st, xp, vp, idx, rows, cols, k);
  else
    hipLaunchKernelGGL((topk_kernel<T, 32>), dim3(blocks), dim3(256), 0, st, xp, vp, idx, rows, cols, k);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

}  // namespace

extern "C" {

int q3_residual_add(const void* a, const void* b, void* y, int64_t n, int dtype, void* stream) {
  return ew_entry<kAdd>(a, b, y, n, dtype, stream);
}

int q3_swiglu(const void* gate, const void* up, void* y, int64_t n, int dtype, void* stream) {
  return ew_entry<kSwiGLU>(gate, up, y, n, dtype, stream);
}

int q3_gelu_tanh(const void* x, void* y, int64_t n, int dtype, void* stream) {
  return ew_entry<kGelu>(x, nullptr, y, n, dtype, stream);
}

int q3_rmsnorm(const void* x, const void* weight, void* y, int64_t rows, int64_t cols, float eps, int dtype,
               void* stream) {
  return norm_entry<kRMS>(x, weight, nullptr, y, rows, cols, eps, dtype, stream);
}

int q3_layernorm(const void* x, const void* weight, const void* bias, void* y, int64_t rows, int64_t cols, float eps,
                 int dtype, void* stream) {
  return norm_entry<kLayer>(x, weight, bias, y, rows, cols, eps, dtype, stream);
}

int q3_softmax(const void* x, void* y, int64_t rows, int64_t cols, int dtype, void* stream) {
  Q3_REQUIRE(x && y, Q3_ERR_NULL);
  Q3_REQUIRE(rows >= 0 && cols >= 1 && cols < (1 << 30), Q3_ERR_SHAPE);
  if (rows == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned blocks = (unsigned)q3_cdiv(rows, 4);
  if (dtype == Q3_BF16)
    hipLaunchKernelGGL(softmax_kernel<bf16>, dim3(blocks), dim3(256), 0, st, static_cast<const bf16*>(x),
                       static_cast<bf16*>(y), rows, (int)cols);
  else if (dtype == Q3_F32)
    hipLaunchKernelGGL(softmax_kernel<float>, dim3(blocks), dim3(256), 0, st, static_cast<const float*>(x),
                       static_cast<float*>(y), rows, (int)cols);
  else
    return Q3_ERR_DTYPE;
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

int q3_topk(const void* x, void* vals, int64_t* idx, int64_t rows, int64_t cols, int64_t k, int dtype, void* stream) {
  Q3_REQUIRE(x && vals && idx, Q3_ERR_NULL);
  Q3_REQUIRE(rows >= 0 && cols >= 1 && k >= 1 && k <= cols, Q3_ERR_SHAPE);
  Q3_REQUIRE(cols <= 2048, Q3_ERR_UNSUPPORTED);
  if (rows == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == Q3_BF16) return launch_topk<bf16>(x, vals, idx, rows, (int)cols, (int)k, st);
  if (dtype == Q3_F32) return launch_topk<float>(x, vals, idx, rows, (int)cols, (int)k, st);
  return Q3_ERR_DTYPE;
}

}  // extern "C"
