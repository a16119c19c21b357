// The rest of the reference's op namespace and the backward of every op that
// has an autograd wrapper there:
//
//  * forward: sigmoid_mul (x * sigmoid(gate)) and cross_entropy (per-row
//    log-sum-exp in one pass with an online max, the mean over targets that
//    are not ignore_index computed on the device);
//  * backward: sigmoid_mul, swiglu, gelu_tanh (elementwise); softmax (row);
//    rmsnorm and layernorm (row pass for the input gradient, fixed-order
//    reductions for the weight / bias gradients); cross_entropy; top-k (a
//    scatter of the value gradients); matmul and the batched GEMM (operands
//    transposed into a workspace, then the MFMA GEMM of gemm.hip, and the
//    bias gradient as a fixed-order column sum).
//
// Everything computes in fp32 and rounds once to the tensor dtype. No
// reduction uses atomics: every sum runs in a fixed order, so results are
// bitwise reproducible run to run.
#include "q3_common.h"

namespace {

constexpr int kT = 256;  // threads per block of every kernel here

__device__ __forceinline__ float sigmoid_f(float g) { return 1.0f / (1.0f + expf(-g)); }

// d/dx of 0.5 x (1 + tanh(k0 (x + c x^3))).
__device__ __forceinline__ float gelu_tanh_grad(float x) {
  const float k0 = 0.7978845608028654f, c = 0.044715f;
  const float t = tanhf(k0 * (x + c * x * x * x));
  return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * k0 * (1.0f + 3.0f * c * x * x);
}

// ===================================================================== elementwise
// Up to three inputs (a, b, c) and two outputs (y0, y1) of one shape.
enum EwOp : int { kSigMulFwd = 0, kSigMulBwd = 1, kSwiGLUBwd = 2, kGeluBwd = 3 };

template <int OP>
__device__ __forceinline__ void ew_eval(float a, float b, float c, float& y0, float& y1) {
  if constexpr (OP == kSigMulFwd) {  // a = x, b = gate
    y0 = a * sigmoid_f(b);
  } else if constexpr (OP == kSigMulBwd) {  // a = x, b = gate, c = dy
    const float s = sigmoid_f(b);
    y0 = c * s;
    y1 = c * a * s * (1.0f - s);
  } else if constexpr (OP == kSwiGLUBwd) {  // a = gate, b = up, c = dy
    const float s = sigmoid_f(a);
    y0 = c * b * s * (1.0f + a * (1.0f - s));
    y1 = c * a * s;
  } else {  // kGeluBwd: a = x, c = dy
    y0 = c * gelu_tanh_grad(a);
  }
}

template <int OP>
constexpr bool ew_uses_b() { return OP != kGeluBwd; }
template <int OP>
constexpr bool ew_uses_c() { return OP != kSigMulFwd; }
template <int OP>
constexpr bool ew_two_out() { return OP == kSigMulBwd || OP == kSwiGLUBwd; }

template <typename T, int OP, bool VEC>
__global__ __launch_bounds__(kT) void ew3_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                 const T* __restrict__ c, T* __restrict__ y0, T* __restrict__ y1,
                                                 int64_t n) {
  constexpr int V = VEC ? Vec16<T>::N : 1;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t nv = n / V;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nv; i += stride) {
    T va[V], vb[V], vc[V], o0[V], o1[V];
    if constexpr (VEC) {
      typedef typename Vec16<T>::type VT;
      *reinterpret_cast<VT*>(va) = reinterpret_cast<const VT*>(a)[i];
      if constexpr (ew_uses_b<OP>()) *reinterpret_cast<VT*>(vb) = reinterpret_cast<const VT*>(b)[i];
      if constexpr (ew_uses_c<OP>()) *reinterpret_cast<VT*>(vc) = reinterpret_cast<const VT*>(c)[i];
    } else {
      va[0] = a[i];
      if constexpr (ew_uses_b<OP>()) vb[0] = b[i];
      if constexpr (ew_uses_c<OP>()) vc[0] = c[i];
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
      float r0 = 0.f, r1 = 0.f;
      ew_eval<OP>(to_f<T>(va[j]), ew_uses_b<OP>() ? to_f<T>(vb[j]) : 0.f, ew_uses_c<OP>() ? to_f<T>(vc[j]) : 0.f,
                  r0, r1);
      o0[j] = from_f<T>(r0);
      o1[j] = from_f<T>(r1);
    }
    if constexpr (VEC) {
      typedef typename Vec16<T>::type VT;
      reinterpret_cast<VT*>(y0)[i] = *reinterpret_cast<VT*>(o0);
      if constexpr (ew_two_out<OP>()) reinterpret_cast<VT*>(y1)[i] = *reinterpret_cast<VT*>(o1);
    } else {
      y0[i] = o0[0];
      if constexpr (ew_two_out<OP>()) y1[i] = o1[0];
    }
  }
  if constexpr (VEC) {  // the tail past the last whole vector
    for (int64_t i = nv * V + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += stride) {
      float r0 = 0.f, r1 = 0.f;
      ew_eval<OP>(to_f<T>(a[i]), ew_uses_b<OP>() ? to_f<T>(b[i]) : 0.f, ew_uses_c<OP>() ? to_f<T>(c[i]) : 0.f, r0,
                  r1);
      y0[i] = from_f<T>(r0);
      if constexpr (ew_two_out<OP>()) y1[i] = from_f<T>(r1);
    }
  }
}

template <typename T, int OP>
int launch_ew3(const void* a, const void* b, const void* c, void* y0, void* y1, int64_t n, hipStream_t st) {
  constexpr int V = Vec16<T>::N;
  bool vec = q3_aligned(a, 16) && q3_aligned(y0, 16);
  if (ew_uses_b<OP>()) vec = vec && q3_aligned(b, 16);
  if (ew_uses_c<OP>()) vec = vec && q3_aligned(c, 16);
  if (ew_two_out<OP>()) vec = vec && q3_aligned(y1, 16);
  const int64_t work = vec ? q3_cdiv(n, V) : n;
  const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(q3_cdiv(work, kT), 256 * 16));
  const T* pa = static_cast<const T*>(a);
  const T* pb = static_cast<const T*>(b);
  const T* pc = static_cast<const T*>(c);
  if (vec)
    hipLaunchKernelGGL((ew3_kernel<T, OP, true>), dim3(blocks), dim3(kT), 0, st, pa, pb, pc, static_cast<T*>(y0),
                       static_cast<T*>(y1), n);
  else
    hipLaunchKernelGGL((ew3_kernel<T, OP, false>), dim3(blocks), dim3(kT), 0, st, pa, pb, pc, static_cast<T*>(y0),
                       static_cast<T*>(y1), n);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

template <int OP>
int ew3_entry(const void* a, const void* b, const void* c, void* y0, void* y1, int64_t n, int dtype, void* stream) {
  Q3_REQUIRE(a && y0, Q3_ERR_NULL);
  Q3_REQUIRE(!ew_uses_b<OP>() || b, Q3_ERR_NULL);
  Q3_REQUIRE(!ew_uses_c<OP>() || c, Q3_ERR_NULL);
  Q3_REQUIRE(!ew_two_out<OP>() || y1, Q3_ERR_NULL);
  Q3_REQUIRE(n >= 0, Q3_ERR_SHAPE);
  if (n == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == Q3_BF16) return launch_ew3<bf16, OP>(a, b, c, y0, y1, n, st);
  if (dtype == Q3_F32) return launch_ew3<float, OP>(a, b, c, y0, y1, n, st);
  return Q3_ERR_DTYPE;
}

// ===================================================================== softmax backward
// One wave per row: dot = sum(out * dy), gx = out * (dy - dot).
template <typename T>
__global__ __launch_bounds__(kT) void softmax_bwd_kernel(const T* __restrict__ out, const T* __restrict__ dy,
                                                         T* __restrict__ gx, int64_t rows, int cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  if (row >= rows) return;
  const T* o = out + row * (int64_t)cols;
  const T* g = dy + row * (int64_t)cols;
  float dot = 0.f;
  for (int c = lane; c < cols; c += 64) dot += to_f<T>(o[c]) * to_f<T>(g[c]);
  dot = wave_sum(dot);
  T* r = gx + row * (int64_t)cols;
  for (int c = lane; c < cols; c += 64) r[c] = from_f<T>(to_f<T>(o[c]) * (to_f<T>(g[c]) - dot));
}

// ===================================================================== norm backward
// A block takes kNormRows consecutive rows. Phase 1: one wave per row computes
// the row's statistics into LDS. Phase 2: each thread takes columns c, c + 256,
// ... and, for each of them, walks the block's rows in order: it writes the
// input gradient and sums the weight (and bias) gradient terms, which it
// stores as the block's partial row. colsum_reduce_kernel then sums the
// partial rows in block order.
//   rmsnorm:   r = rsqrt(mean(x^2) + eps), gx = dy w r - x (r^3 / n) sum(dy w x),
//              gw = sum_rows dy x r
//   layernorm: m = mean(x), r = rsqrt(mean((x - m)^2) + eps), xh = (x - m) r, g = dy w,
//              gx = r (g - mean(g) - xh mean(g xh)), gw = sum_rows dy xh, gb = sum_rows dy
constexpr int kNormRows = 32;

template <typename T, bool LAYER>
__global__ __launch_bounds__(kT) void norm_bwd_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                      const T* __restrict__ dy, T* __restrict__ gx,
                                                      float* __restrict__ pw, float* __restrict__ pb, int64_t rows,
                                                      int cols, float eps) {
  __shared__ float s_mean[kNormRows], s_rstd[kNormRows], s_k1[kNormRows], s_k2[kNormRows];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * kNormRows;
  const int nr = (int)std::min<int64_t>(kNormRows, rows - r0);
  const float inv_n = 1.0f / (float)cols;
  for (int rr = wave; rr < nr; rr += kT / 64) {
    const T* xr = x + (r0 + rr) * (int64_t)cols;
    const T* gr = dy + (r0 + rr) * (int64_t)cols;
    if constexpr (LAYER) {
      float s = 0.f;
      for (int c = lane; c < cols; c += 64) s += to_f<T>(xr[c]);
      const float mean = wave_sum(s) * inv_n;
      float v = 0.f, sg = 0.f, sgd = 0.f;
      for (int c = lane; c < cols; c += 64) {
        const float d = to_f<T>(xr[c]) - mean;
        const float g = to_f<T>(gr[c]) * to_f<T>(w[c]);
        v += d * d;
        sg += g;
        sgd += g * d;
      }
      const float rstd = rsqrtf(wave_sum(v) * inv_n + eps);
      sg = wave_sum(sg);
      sgd = wave_sum(sgd);
      if (lane == 0) {
        s_mean[rr] = mean;
        s_rstd[rr] = rstd;
        s_k1[rr] = sg * inv_n;          // mean(g)
        s_k2[rr] = sgd * rstd * inv_n;  // mean(g * xh)
      }
    } else {
      float ss = 0.f, dot = 0.f;
      for (int c = lane; c < cols; c += 64) {
        const float xv = to_f<T>(xr[c]);
        ss += xv * xv;
        dot += to_f<T>(gr[c]) * to_f<T>(w[c]) * xv;
      }
      const float rstd = rsqrtf(wave_sum(ss) * inv_n + eps);
      dot = wave_sum(dot);
      if (lane == 0) {
        s_rstd[rr] = rstd;
        s_k1[rr] = dot * rstd * rstd * rstd * inv_n;
      }
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < cols; c += kT) {
    const float wc = to_f<T>(w[c]);
    float aw = 0.f, ab = 0.f;
    for (int rr = 0; rr < nr; ++rr) {
      const int64_t o = (r0 + rr) * (int64_t)cols + c;
      const float xv = to_f<T>(x[o]), g = to_f<T>(dy[o]);
      const float rstd = s_rstd[rr];
      float gxv;
      if constexpr (LAYER) {
        const float xh = (xv - s_mean[rr]) * rstd;
        gxv = rstd * (g * wc - s_k1[rr] - xh * s_k2[rr]);
        aw += g * xh;
        ab += g;
      } else {
        gxv = g * wc * rstd - xv * s_k1[rr];
        aw += g * xv * rstd;
      }
      gx[o] = from_f<T>(gxv);
    }
    if (pw) pw[(int64_t)blockIdx.x * cols + c] = aw;
    if (LAYER && pb) pb[(int64_t)blockIdx.x * cols + c] = ab;
  }
}

// Partial column sums of a (rows, cols) matrix over kColRows-row chunks:
// part[chunk][c] = sum of the chunk's rows, in row order.
constexpr int kColRows = 256;

template <typename T>
__global__ __launch_bounds__(kT) void colsum_partial_kernel(const T* __restrict__ a, float* __restrict__ part,
                                                            int64_t rows, int64_t cols) {
  const int64_t c = (int64_t)blockIdx.x * kT + threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * kColRows;
  const int64_t r1 = std::min<int64_t>(rows, r0 + kColRows);
  float acc = 0.f;
  for (int64_t r = r0; r < r1; ++r) acc += to_f<T>(a[r * cols + c]);
  part[(int64_t)blockIdx.y * cols + c] = acc;
}

// out[c] = sum over the nparts partial rows, in order, rounded once.
template <typename T>
__global__ __launch_bounds__(kT) void colsum_reduce_kernel(const float* __restrict__ part, T* __restrict__ out,
                                                           int64_t nparts, int64_t cols) {
  const int64_t c = (int64_t)blockIdx.x * kT + threadIdx.x;
  if (c >= cols) return;
  float acc = 0.f;
  for (int64_t p = 0; p < nparts; ++p) acc += part[p * cols + c];
  out[c] = from_f<T>(acc);
}

template <typename T>
int colsum_t(const void* a, void* out, int64_t rows, int64_t cols, float* part, hipStream_t st) {
  const int64_t nparts = q3_cdiv(rows, kColRows);
  hipLaunchKernelGGL(colsum_partial_kernel<T>, dim3((unsigned)q3_cdiv(cols, kT), (unsigned)nparts), dim3(kT), 0, st,
                     static_cast<const T*>(a), part, rows, cols);
  Q3_LAUNCH_CHECK();
  hipLaunchKernelGGL(colsum_reduce_kernel<T>, dim3((unsigned)q3_cdiv(cols, kT)), dim3(kT), 0, st, part,
                     static_cast<T*>(out), nparts, cols);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

template <typename T, bool LAYER>
int norm_bwd_t(const void* x, const void* w, const void* dy, void* gx, void* gw, void* gb, int64_t rows, int cols,
               float eps, float* ws, hipStream_t st) {
  const int64_t nblk = q3_cdiv(rows, kNormRows);
  float* pw = gw ? ws : nullptr;
  float* pb = (LAYER && gb) ? ws + nblk * cols : nullptr;
  hipLaunchKernelGGL((norm_bwd_kernel<T, LAYER>), dim3((unsigned)nblk), dim3(kT), 0, st, static_cast<const T*>(x),
                     static_cast<const T*>(w), static_cast<const T*>(dy), static_cast<T*>(gx), pw, pb, rows, cols,
                     eps);
  Q3_LAUNCH_CHECK();
  if (gw) {
    hipLaunchKernelGGL(colsum_reduce_kernel<T>, dim3((unsigned)q3_cdiv(cols, kT)), dim3(kT), 0, st, pw,
                       static_cast<T*>(gw), nblk, (int64_t)cols);
    Q3_LAUNCH_CHECK();
  }
  if (pb) {
    hipLaunchKernelGGL(colsum_reduce_kernel<T>, dim3((unsigned)q3_cdiv(cols, kT)), dim3(kT), 0, st, pb,
                       static_cast<T*>(gb), nblk, (int64_t)cols);
    Q3_LAUNCH_CHECK();
  }
  return Q3_OK;
}

int64_t norm_bwd_ws(int64_t rows, int64_t cols) { return 2 * q3_cdiv(rows, kNormRows) * cols * 4; }

template <bool LAYER>
int norm_bwd_entry(const void* x, const void* w, const void* dy, void* gx, void* gw, void* gb, int64_t rows,
                   int64_t cols, float eps, int dtype, void* ws, int64_t ws_bytes, void* stream) {
  Q3_REQUIRE(x && w && dy && gx, Q3_ERR_NULL);
  Q3_REQUIRE(rows >= 0 && cols >= 1 && cols < (1 << 24), Q3_ERR_SHAPE);
  Q3_REQUIRE(!(gw || gb) || (ws && ws_bytes >= norm_bwd_ws(rows, cols)), Q3_ERR_WORKSPACE);
  Q3_REQUIRE(!ws || q3_aligned(ws, 16), Q3_ERR_ALIGN);
  if (rows == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* f = static_cast<float*>(ws);
  if (dtype == Q3_BF16) return norm_bwd_t<bf16, LAYER>(x, w, dy, gx, gw, gb, rows, (int)cols, eps, f, st);
  if (dtype == Q3_F32) return norm_bwd_t<float, LAYER>(x, w, dy, gx, gw, gb, rows, (int)cols, eps, f, st);
  return Q3_ERR_DTYPE;
}

// ===================================================================== cross entropy
// Forward: one block per row. Each thread keeps an online (max, sum of
// exp(x - max)) over its strided share of the row (16-byte vectors when the
// row allows), the block merges the 256 pairs in a fixed tree, and thread 0
// writes lse = max + log(sum) and loss = lse - x[target] (both 0 for a target
// equal to ignore_index, as the reference's kernel does; a target outside
// [0, V) is treated the same and sets bit 0 of *status).
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float mm = fmaxf(m, m2);
  s = (m == -INFINITY ? 0.f : s * expf(m - mm)) + (m2 == -INFINITY ? 0.f : s2 * expf(m2 - mm));
  m = mm;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kT) void ce_fwd_kernel(const T* __restrict__ logits, const int64_t* __restrict__ tgt,
                                                    float* __restrict__ loss, float* __restrict__ lse, int64_t V,
                                                    int64_t ignore_index, int* __restrict__ status) {
  __shared__ float s_m[kT / 64], s_s[kT / 64];
  const int64_t row = blockIdx.x;
  const int64_t t = tgt[row];
  const bool valid = t != ignore_index && t >= 0 && t < V;
  if (!valid) {
    if (threadIdx.x == 0) {
      loss[row] = 0.f;
      lse[row] = 0.f;
      if (t != ignore_index && status) atomicOr(status, 1);
    }
    return;
  }
  const T* xr = logits + row * V;
  float m = -INFINITY, s = 0.f;
  auto add = [&](float v) __attribute__((always_inline)) {
    if (v > m) {
      s = s * expf(m - v) + 1.0f;
      m = v;
    } else {
      s += expf(v - m);
    }
  };
  if constexpr (VEC) {
    constexpr int NV = Vec16<T>::N;
    typedef typename Vec16<T>::type VT;
    const int64_t nv = V / NV;
    for (int64_t i = threadIdx.x; i < nv; i += kT) {
      const VT u = reinterpret_cast<const VT*>(xr)[i];
#pragma unroll
      for (int j = 0; j < NV; ++j) add(to_f<T>(u[j]));
    }
    for (int64_t i = nv * NV + threadIdx.x; i < V; i += kT) add(to_f<T>(xr[i]));
  } else {
    for (int64_t i = threadIdx.x; i < V; i += kT) add(to_f<T>(xr[i]));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    lse_merge(m, s, m2, s2);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    s_m[wave] = m;
    s_s[wave] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float mm = s_m[0], ss = s_s[0];
    for (int w = 1; w < kT / 64; ++w) lse_merge(mm, ss, s_m[w], s_s[w]);
    const float l = mm + logf(ss);
    lse[row] = l;
    loss[row] = l - to_f<T>(xr[t]);
  }
}

// The mean over valid targets: one block sums the per-row losses and counts the
// valid targets in a fixed order; out = sum / max(count, 1) (fp32), and the
// count goes to *n_valid for the backward.
__global__ __launch_bounds__(kT) void ce_mean_kernel(const float* __restrict__ loss, const int64_t* __restrict__ tgt,
                                                     int64_t N, int64_t V, int64_t ignore_index,
                                                     float* __restrict__ out, int* __restrict__ n_valid) {
  __shared__ float s_sum[kT];
  __shared__ int s_cnt[kT];
  float acc = 0.f;
  int cnt = 0;
  for (int64_t i = threadIdx.x; i < N; i += kT) {
    acc += loss[i];
    const int64_t t = tgt[i];
    cnt += (t != ignore_index && t >= 0 && t < V) ? 1 : 0;
  }
  s_sum[threadIdx.x] = acc;
  s_cnt[threadIdx.x] = cnt;
  __syncthreads();
  for (int o = kT / 2; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) {
      s_sum[threadIdx.x] += s_sum[threadIdx.x + o];
      s_cnt[threadIdx.x] += s_cnt[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[0] = s_sum[0] / (float)max(s_cnt[0], 1);
    if (n_valid) n_valid[0] = s_cnt[0];
  }
}

// Backward: grad[i, j] = (exp(x_ij - lse_i) - [j == t_i]) * dloss / max(n_valid, 1);
// rows whose target is ignored (or out of range) get zeros. dloss and n_valid
// are read on the device (no host synchronisation).
template <typename T>
__global__ __launch_bounds__(kT) void ce_bwd_kernel(const T* __restrict__ logits, const int64_t* __restrict__ tgt,
                                                    const float* __restrict__ lse, const float* __restrict__ dloss,
                                                    const int* __restrict__ n_valid, T* __restrict__ grad, int64_t V,
                                                    int64_t ignore_index) {
  const int64_t row = blockIdx.y;
  const int64_t t = tgt[row];
  const bool valid = t != ignore_index && t >= 0 && t < V;
  const float scale = dloss[0] / (float)max(n_valid[0], 1);
  const float l = lse[row];
  const T* xr = logits + row * V;
  T* gr = grad + row * V;
  for (int64_t j = (int64_t)blockIdx.x * kT + threadIdx.x; j < V; j += (int64_t)gridDim.x * kT) {
    float g = 0.f;
    if (valid) g = (expf(to_f<T>(xr[j]) - l) - (j == t ? 1.0f : 0.0f)) * scale;
    gr[j] = from_f<T>(g);
  }
}

// ===================================================================== top-k backward
// grad_x[r, c] = grad_vals[r, j] where idx[r, j] == c, else 0 (the indices of a
// row are distinct). One wave per row.
template <typename T>
__global__ __launch_bounds__(kT) void topk_bwd_kernel(const T* __restrict__ gv, const int64_t* __restrict__ idx,
                                                      T* __restrict__ gx, int64_t rows, int cols, int k) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  if (row >= rows) return;
  for (int c = lane; c < cols; c += 64) {
    float v = 0.f;
    for (int j = 0; j < k; ++j)
      if (idx[row * k + j] == c) v = to_f<T>(gv[row * k + j]);
    gx[row * (int64_t)cols + c] = from_f<T>(v);
  }
}

// ===================================================================== transpose
// (E, R, C) -> (E, C, R) through a 64 x 65 LDS tile.
template <typename T>
__global__ __launch_bounds__(kT) void transpose_kernel(const T* __restrict__ a, T* __restrict__ b, int64_t R,
                                                       int64_t C) {
  __shared__ T tile[64][65];
  const int64_t e = blockIdx.z;
  const T* ae = a + e * R * C;
  T* be = b + e * R * C;
  const int64_t c0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += kT / 64) {
    const int64_t r = r0 + i, c = c0 + tx;
    if (r < R && c < C) tile[i][tx] = ae[r * C + c];
  }
  __syncthreads();
  for (int i = ty; i < 64; i += kT / 64) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (r < R && c < C) be[c * R + r] = tile[tx][i];
  }
}

int transpose(const void* a, void* b, int64_t E, int64_t R, int64_t C, int dtype, hipStream_t st) {
  if (E == 0 || R == 0 || C == 0) return Q3_OK;
  const dim3 grid((unsigned)q3_cdiv(C, 64), (unsigned)q3_cdiv(R, 64), (unsigned)E);
  if (dtype == Q3_BF16)
    hipLaunchKernelGGL(transpose_kernel<bf16>, grid, dim3(kT), 0, st, static_cast<const bf16*>(a),
                       static_cast<bf16*>(b), R, C);
  else
    hipLaunchKernelGGL(transpose_kernel<float>, grid, dim3(kT), 0, st, static_cast<const float*>(a),
                       static_cast<float*>(b), R, C);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

// Workspace of the matmul backward: W^T (K, N), dY^T (N, M), X^T (K, M) and
// the bias gradient's partial sums.
struct MmBwdLayout {
  int64_t wt, dyt, xt, part, total;
};
MmBwdLayout mm_bwd_layout(int64_t M, int64_t N, int64_t K, int dtype) {
  const int64_t es = dtype == Q3_BF16 ? 2 : 4;
  MmBwdLayout l{};
  l.wt = 0;
  l.dyt = l.wt + align256(K * N * es);
  l.xt = l.dyt + align256(N * M * es);
  l.part = l.xt + align256(K * M * es);
  l.total = l.part + align256(q3_cdiv(M, kColRows) * N * 4);
  return l;
}

}  // namespace

extern "C" {

int q3_sigmoid_mul(const void* x, const void* gate, void* y, int64_t n, int dtype, void* stream) {
  return ew3_entry<kSigMulFwd>(x, gate, nullptr, y, nullptr, n, dtype, stream);
}

int q3_sigmoid_mul_backward(const void* x, const void* gate, const void* grad_out, void* grad_x, void* grad_gate,
                            int64_t n, int dtype, void* stream) {
  return ew3_entry<kSigMulBwd>(x, gate, grad_out, grad_x, grad_gate, n, dtype, stream);
}

int q3_swiglu_backward(const void* gate, const void* up, const void* grad_out, void* grad_gate, void* grad_up,
                       int64_t n, int dtype, void* stream) {
  return ew3_entry<kSwiGLUBwd>(gate, up, grad_out, grad_gate, grad_up, n, dtype, stream);
}

int q3_gelu_tanh_backward(const void* x, const void* grad_out, void* grad_x, int64_t n, int dtype, void* stream) {
  return ew3_entry<kGeluBwd>(x, nullptr, grad_out, grad_x, nullptr, n, dtype, stream);
}

int q3_softmax_backward(const void* out, const void* grad_out, void* grad_x, int64_t rows, int64_t cols, int dtype,
                        void* stream) {
  Q3_REQUIRE(out && grad_out && grad_x, Q3_ERR_NULL);
  Q3_REQUIRE(rows >= 0 && cols >= 1 && cols < (1 << 30), Q3_ERR_SHAPE);
  if (rows == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned blocks = (unsigned)q3_cdiv(rows, kT / 64);
  if (dtype == Q3_BF16)
    hipLaunchKernelGGL(softmax_bwd_kernel<bf16>, dim3(blocks), dim3(kT), 0, st, static_cast<const bf16*>(out),
                       static_cast<const bf16*>(grad_out), static_cast<bf16*>(grad_x), rows, (int)cols);
  else if (dtype == Q3_F32)
    hipLaunchKernelGGL(softmax_bwd_kernel<float>, dim3(blocks), dim3(kT), 0, st, static_cast<const float*>(out),
                       static_cast<const float*>(grad_out), static_cast<float*>(grad_x), rows, (int)cols);
  else
    return Q3_ERR_DTYPE;
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

int64_t q3_norm_backward_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return norm_bwd_ws(rows, cols);
}

int q3_rmsnorm_backward(const void* x, const void* weight, const void* grad_out, void* grad_x, void* grad_weight,
                        int64_t rows, int64_t cols, float eps, int dtype, void* workspace, int64_t workspace_bytes,
                        void* stream) {
  return norm_bwd_entry<false>(x, weight, grad_out, grad_x, grad_weight, nullptr, rows, cols, eps, dtype, workspace,
                               workspace_bytes, stream);
}

int q3_layernorm_backward(const void* x, const void* weight, const void* grad_out, void* grad_x, void* grad_weight,
                          void* grad_bias, int64_t rows, int64_t cols, float eps, int dtype, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  return norm_bwd_entry<true>(x, weight, grad_out, grad_x, grad_weight, grad_bias, rows, cols, eps, dtype, workspace,
                              workspace_bytes, stream);
}

int q3_cross_entropy(const void* logits, const int64_t* targets, float* loss_per_token, float* lse, float* loss,
                     int* n_valid, int64_t N, int64_t V, int64_t ignore_index, int dtype, int* status, void* stream) {
  Q3_REQUIRE(logits && targets && loss_per_token && lse && loss, Q3_ERR_NULL);
  Q3_REQUIRE(N >= 0 && V >= 1 && N < (1ll << 31), Q3_ERR_SHAPE);
  Q3_REQUIRE(dtype == Q3_BF16 || dtype == Q3_F32, Q3_ERR_DTYPE);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (N > 0) {
    const bool vec = q3_aligned(logits, 16) && V % (dtype == Q3_BF16 ? 8 : 4) == 0;
    const dim3 grid((unsigned)N);
    if (dtype == Q3_BF16) {
      const bf16* l = static_cast<const bf16*>(logits);
      if (vec)
        hipLaunchKernelGGL((ce_fwd_kernel<bf16, true>), grid, dim3(kT), 0, st, l, targets, loss_per_token, lse, V,
                           ignore_index, status);
      else
        hipLaunchKernelGGL((ce_fwd_kernel<bf16, false>), grid, dim3(kT), 0, st, l, targets, loss_per_token, lse, V,
                           ignore_index, status);
    } else {
      const float* l = static_cast<const float*>(logits);
      if (vec)
        hipLaunchKernelGGL((ce_fwd_kernel<float, true>), grid, dim3(kT), 0, st, l, targets, loss_per_token, lse, V,
                           ignore_index, status);
      else
        hipLaunchKernelGGL((ce_fwd_kernel<float, false>), grid, dim3(kT), 0, st, l, targets, loss_per_token, lse,
                           V, ignore_index, status);
    }
    Q3_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL(ce_mean_kernel, dim3(1), dim3(kT), 0, st, loss_per_token, targets, N, V, ignore_index, loss,
                     n_valid);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

int q3_cross_entropy_backward(const void* logits, const int64_t* targets, const float* lse, const float* grad_loss,
                              const int* n_valid, void* grad_logits, int64_t N, int64_t V, int64_t ignore_index,
                              int dtype, void* stream) {
  Q3_REQUIRE(logits && targets && lse && grad_loss && n_valid && grad_logits, Q3_ERR_NULL);
  Q3_REQUIRE(N >= 0 && V >= 1 && N < 65536ll * 1024, Q3_ERR_SHAPE);
  if (N == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned gx = (unsigned)std::min<int64_t>(q3_cdiv(V, kT), 64);
  // grid.y = rows (at most 65535 per launch): launch in row chunks
  for (int64_t r0 = 0; r0 < N; r0 += 65535) {
    const int64_t nr = std::min<int64_t>(65535, N - r0);
    if (dtype == Q3_BF16)
      hipLaunchKernelGGL(ce_bwd_kernel<bf16>, dim3(gx, (unsigned)nr), dim3(kT), 0, st,
                         static_cast<const bf16*>(logits) + r0 * V, targets + r0, lse + r0, grad_loss, n_valid,
                         static_cast<bf16*>(grad_logits) + r0 * V, V, ignore_index);
    else if (dtype == Q3_F32)
      hipLaunchKernelGGL(ce_bwd_kernel<float>, dim3(gx, (unsigned)nr), dim3(kT), 0, st,
                         static_cast<const float*>(logits) + r0 * V, targets + r0, lse + r0, grad_loss, n_valid,
                         static_cast<float*>(grad_logits) + r0 * V, V, ignore_index);
    else
      return Q3_ERR_DTYPE;
    Q3_LAUNCH_CHECK();
  }
  return Q3_OK;
}

int q3_topk_backward(const void* grad_vals, const int64_t* idx, void* grad_x, int64_t rows, int64_t cols, int64_t k,
                     int dtype, void* stream) {
  Q3_REQUIRE(grad_vals && idx && grad_x, Q3_ERR_NULL);
  Q3_REQUIRE(rows >= 0 && cols >= 1 && k >= 1 && k <= cols && cols < (1 << 30), Q3_ERR_SHAPE);
  if (rows == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned blocks = (unsigned)q3_cdiv(rows, kT / 64);
  if (dtype == Q3_BF16)
    hipLaunchKernelGGL(topk_bwd_kernel<bf16>, dim3(blocks), dim3(kT), 0, st, static_cast<const bf16*>(grad_vals),
                       idx, static_cast<bf16*>(grad_x), rows, (int)cols, (int)k);
  else if (dtype == Q3_F32)
    hipLaunchKernelGGL(topk_bwd_kernel<float>, dim3(blocks), dim3(kT), 0, st, static_cast<const float*>(grad_vals),
                       idx, static_cast<float*>(grad_x), rows, (int)cols, (int)k);
  else
    return Q3_ERR_DTYPE;
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

int q3_transpose(const void* a, void* b, int64_t E, int64_t R, int64_t C, int dtype, void* stream) {
  Q3_REQUIRE(a && b, Q3_ERR_NULL);
  Q3_REQUIRE(E >= 0 && R >= 0 && C >= 0 && E < 65536, Q3_ERR_SHAPE);
  Q3_REQUIRE(dtype == Q3_BF16 || dtype == Q3_F32, Q3_ERR_DTYPE);
  return transpose(a, b, E, R, C, dtype, static_cast<hipStream_t>(stream));
}

int64_t q3_matmul_backward_workspace_bytes(int64_t M, int64_t N, int64_t K, int dtype) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return mm_bwd_layout(M, N, K, dtype).total;
}

int q3_matmul_backward(const void* x, const void* w, const void* dy, void* gx, void* gw, void* gb, int64_t M,
                       int64_t N, int64_t K, int dtype, void* workspace, int64_t workspace_bytes, void* gemm_ws,
                       int64_t gemm_ws_bytes, void* stream) {
  Q3_REQUIRE(x && w && dy, Q3_ERR_NULL);
  Q3_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31), Q3_ERR_SHAPE);
  Q3_REQUIRE(dtype == Q3_BF16 || dtype == Q3_F32, Q3_ERR_DTYPE);
  if (M == 0 || N == 0 || K == 0) return Q3_OK;
  const MmBwdLayout l = mm_bwd_layout(M, N, K, dtype);
  Q3_REQUIRE(workspace && workspace_bytes >= l.total, Q3_ERR_WORKSPACE);
  Q3_REQUIRE(q3_aligned(workspace, 256), Q3_ERR_ALIGN);
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc;
  if (gx) {  // gx (M, K) = dY (M, N) . W (N, K) = dY . (W^T)^T with W^T (K, N) as the GEMM's weight
    const int64_t need = q3_matmul_workspace_bytes(M, K, N, dtype, 0);
    Q3_REQUIRE(need <= 0 || (gemm_ws && gemm_ws_bytes >= need), Q3_ERR_WORKSPACE);
    if ((rc = transpose(w, ws + l.wt, 1, N, K, dtype, st)) != Q3_OK) return rc;
    if ((rc = q3_matmul(dy, ws + l.wt, nullptr, nullptr, gx, M, K, N, N, N, 0, K, dtype, gemm_ws, gemm_ws_bytes,
                        stream)) != Q3_OK)
      return rc;
  }
  if (gw) {  // gw (N, K) = dY^T (N, M) . X (M, K) = dY^T . (X^T)^T with X^T (K, M) as the weight
    const int64_t need = q3_matmul_workspace_bytes(N, K, M, dtype, 0);
    Q3_REQUIRE(need <= 0 || (gemm_ws && gemm_ws_bytes >= need), Q3_ERR_WORKSPACE);
    if ((rc = transpose(dy, ws + l.dyt, 1, M, N, dtype, st)) != Q3_OK) return rc;
    if ((rc = transpose(x, ws + l.xt, 1, M, K, dtype, st)) != Q3_OK) return rc;
    if ((rc = q3_matmul(ws + l.dyt, ws + l.xt, nullptr, nullptr, gw, N, K, M, M, M, 0, K, dtype, gemm_ws,
                        gemm_ws_bytes, stream)) != Q3_OK)
      return rc;
  }
  if (gb) {  // gb (N) = sum over the M rows of dY, in row order
    float* part = reinterpret_cast<float*>(ws + l.part);
    if (dtype == Q3_BF16) return colsum_t<bf16>(dy, gb, M, N, part, st);
    return colsum_t<float>(dy, gb, M, N, part, st);
  }
  return Q3_OK;
}

int64_t q3_batched_gemm_backward_workspace_bytes(int64_t E, int64_t M, int64_t N, int64_t K, int dtype) {
  if (E <= 0 || M <= 0 || N <= 0 || K <= 0) return 0;
  const int64_t es = dtype == Q3_BF16 ? 2 : 4;
  return align256(E * K * N * es) + align256(E * N * M * es) + align256(E * K * M * es);
}

int q3_batched_gemm_backward(const void* x, const void* w, const void* dy, void* gx, void* gw, int64_t E, int64_t M,
                             int64_t N, int64_t K, int dtype, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  Q3_REQUIRE(x && w && dy, Q3_ERR_NULL);
  Q3_REQUIRE(E >= 0 && M >= 0 && N >= 0 && K >= 0 && E < 65536, Q3_ERR_SHAPE);
  Q3_REQUIRE(dtype == Q3_BF16 || dtype == Q3_F32, Q3_ERR_DTYPE);
  if (E == 0 || M == 0 || N == 0 || K == 0) return Q3_OK;
  const int64_t es = dtype == Q3_BF16 ? 2 : 4;
  Q3_REQUIRE(workspace && workspace_bytes >= q3_batched_gemm_backward_workspace_bytes(E, M, N, K, dtype),
             Q3_ERR_WORKSPACE);
  Q3_REQUIRE(q3_aligned(workspace, 256), Q3_ERR_ALIGN);
  char* wt = static_cast<char*>(workspace);
  char* dyt = wt + align256(E * K * N * es);
  char* xt = dyt + align256(E * N * M * es);
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc;
  if (gx) {  // gx[e] (M, K) = dY[e] (M, N) . W[e] (N, K)
    if ((rc = transpose(w, wt, E, N, K, dtype, st)) != Q3_OK) return rc;
    if ((rc = q3_batched_gemm(dy, wt, gx, E, M, K, N, dtype, stream)) != Q3_OK) return rc;
  }
  if (gw) {  // gw[e] (N, K) = dY[e]^T (N, M) . X[e] (M, K)
    if ((rc = transpose(dy, dyt, E, M, N, dtype, st)) != Q3_OK) return rc;
    if ((rc = transpose(x, xt, E, M, K, dtype, st)) != Q3_OK) return rc;
    if ((rc = q3_batched_gemm(dyt, xt, gw, E, N, K, M, dtype, stream)) != Q3_OK) return rc;
  }
  return Q3_OK;
}

}  // extern "C"
