// Model-edge and vision-tower glue kernels:
//  * q3_embedding            token-id row gather (CudaEmbedding)
//  * q3_vision_rope_tables   the vision tower's 2D rotary cos/sin tables from
//                            the images' (t, h, w) grids, computed on the GPU
//  * q3_vision_pos_embed     bilinear interpolation of the learned position
//                            grid, in token (merge-block) order, added to the
//                            patch embeddings
// All are HBM-bound row kernels: 16-byte vector accesses, one row (or a few)
// per wave, fp32 arithmetic and one rounding per output element.
#include "q3_common.h"

namespace {

// ------------------------------------------------------------------ embedding
// out[t, :] = weight[ids[t], :]. One wave per token row, 16-byte pieces.
// An id outside [0, rows) writes a zero row and sets bit 0 of *status.
template <typename T>
__global__ __launch_bounds__(256) void embedding_kernel(const int64_t* __restrict__ ids, const T* __restrict__ weight,
                                                        T* __restrict__ out, int64_t n, int64_t rows, int64_t dim,
                                                        int* __restrict__ status) {
  const int64_t t = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (t >= n) return;
  const int64_t id = ids[t];
  const bool ok = id >= 0 && id < rows;
  if (!ok && lane == 0 && status) atomicOr(status, 1);
  constexpr int V = 16 / sizeof(T);
  T* orow = out + t * dim;
  const T* wrow = weight + (ok ? id : 0) * dim;
  if (dim % V == 0) {
    using Vec = u32x4;
    const int64_t nv = dim / V;
    for (int64_t j = lane; j < nv; j += 64) {
      Vec v = ok ? reinterpret_cast<const Vec*>(wrow)[j] : Vec{0, 0, 0, 0};
      reinterpret_cast<Vec*>(orow)[j] = v;
    }
  } else {
    for (int64_t j = lane; j < dim; j += 64) orow[j] = ok ? wrow[j] : from_f<T>(0.f);
  }
}

// ------------------------------------------------------------------ vision rotary tables
// Image table entry: t, h, w (patch grid), first token. Token p of an image
// (frame-major, then merge blocks of m x m patches row-major, then the m x m
// patches of the block row-major) sits at patch row
//   (q / (m m)) / (w / m) * m + (q % (m m)) / m,   q = p % (h w)
// and column
//   (q / (m m)) % (w / m) * m + (q % (m m)) % m.
// Its angles are row * inv_freq[j] for j < D/4 and col * inv_freq[j - D/4]
// for D/4 <= j < D/2 (inv_freq: D/4 fp32 values, theta^(-4 j / D), the
// rotary dimension being D/2); the table repeats them over the two halves of D.
__device__ __forceinline__ int image_of(const int* __restrict__ img, int n_img, int64_t tok) {
  int lo = 0, hi = n_img - 1;  // last image whose first token <= tok
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (img[4 * mid + 3] <= tok) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

__device__ __forceinline__ void patch_rc(const int* __restrict__ img, int i, int64_t tok, int m, int& row, int& col) {
  const int h = img[4 * i + 1], w = img[4 * i + 2];
  const int64_t p = tok - img[4 * i + 3];
  const int q = (int)(p % ((int64_t)h * w));
  const int blk = q / (m * m), in = q % (m * m);
  row = blk / (w / m) * m + in / m;
  col = blk % (w / m) * m + in % m;
}

__global__ __launch_bounds__(256) void vision_rope_kernel(const int* __restrict__ img, int n_img, int64_t total, int m,
                                                          int D, const float* __restrict__ inv_freq,
                                                          float* __restrict__ cos_out, float* __restrict__ sin_out) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total * D) return;
  const int64_t tok = e / D;
  const int j = (int)(e % D);
  int row, col;
  patch_rc(img, image_of(img, n_img, tok), tok, m, row, col);
  const int q = D / 4, jj = j % (D / 2);
  const int pos = jj < q ? row : col;
  const int fi = jj < q ? jj : jj - q;
  float s, c;
  sincosf((float)pos * inv_freq[fi], &s, &c);
  cos_out[e] = c;
  sin_out[e] = s;
}

// ------------------------------------------------------------------ position-embedding interpolation
// For patch row r of an image with h rows, the grid coordinate is
// linspace(0, G - 1, h)[r]; its floor f, the clipped ceiling min(f + 1, G - 1)
// and the fraction give the bilinear weights over the G x G learned table
// (the same for columns). linspace is evaluated the way torch does on the CPU
// (from the start for the first half, from the end for the second), so the
// floors agree at the end points.
__device__ __forceinline__ float linspace_at(int i, int n, float end) {
  if (n == 1) return 0.f;
  const float step = end / (float)(n - 1);
  return i < n / 2 ? step * (float)i : end - step * (float)(n - 1 - i);
}

template <typename T>
__global__ __launch_bounds__(256) void pos_embed_kernel(const int* __restrict__ img, int n_img, int64_t total, int m,
                                                        int G, const T* __restrict__ table, const T* __restrict__ x,
                                                        T* __restrict__ y, int64_t hidden) {
  const int64_t tok = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (tok >= total) return;
  const int i = image_of(img, n_img, tok);
  int row, col;
  patch_rc(img, i, tok, m, row, col);
  const float hc = linspace_at(row, img[4 * i + 1], (float)(G - 1));
  const float wc = linspace_at(col, img[4 * i + 2], (float)(G - 1));
  const int hf = (int)hc, wf = (int)wc;
  const int hcl = min(hf + 1, G - 1), wcl = min(wf + 1, G - 1);
  const float dh = hc - (float)hf, dw = wc - (float)wf;
  const float w00 = (1.f - dh) * (1.f - dw), w01 = (1.f - dh) * dw, w10 = dh * (1.f - dw), w11 = dh * dw;
  const T* r00 = table + (int64_t)(hf * G + wf) * hidden;
  const T* r01 = table + (int64_t)(hf * G + wcl) * hidden;
  const T* r10 = table + (int64_t)(hcl * G + wf) * hidden;
  const T* r11 = table + (int64_t)(hcl * G + wcl) * hidden;
  const T* xr = x + tok * hidden;
  T* yr = y + tok * hidden;
  for (int64_t d = lane; d < hidden; d += 64) {
    const float v = w00 * to_f<T>(r00[d]) + w01 * to_f<T>(r01[d]) + w10 * to_f<T>(r10[d]) + w11 * to_f<T>(r11[d]);
    yr[d] = from_f<T>(to_f<T>(xr[d]) + v);
  }
}

bool check_images(const int* img_host, int64_t n_img, int64_t m, int64_t* total) {
  int64_t t0 = 0;
  for (int64_t i = 0; i < n_img; ++i) {
    const int t = img_host[4 * i], h = img_host[4 * i + 1], w = img_host[4 * i + 2];
    if (t < 1 || h < 1 || w < 1 || h % m || w % m || img_host[4 * i + 3] != t0) return false;
    t0 += (int64_t)t * h * w;
  }
  *total = t0;
  return true;
}

}  // namespace

extern "C" {

int q3_embedding(const int64_t* ids, const void* weight, void* out, int64_t n, int64_t rows, int64_t dim, int dtype,
                 int* status, void* stream) {
  Q3_REQUIRE(ids && weight && out, Q3_ERR_NULL);
  Q3_REQUIRE(n >= 0 && rows >= 1 && dim >= 1, Q3_ERR_SHAPE);
  if (n == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)q3_cdiv(n, 4));
  if (dtype == Q3_BF16) {
    Q3_REQUIRE(dim % 8 != 0 || (q3_aligned(weight, 16) && q3_aligned(out, 16)), Q3_ERR_ALIGN);
    hipLaunchKernelGGL(embedding_kernel<bf16>, grid, dim3(256), 0, st, ids, static_cast<const bf16*>(weight),
                       static_cast<bf16*>(out), n, rows, dim, status);
  } else if (dtype == Q3_F32) {
    Q3_REQUIRE(dim % 4 != 0 || (q3_aligned(weight, 16) && q3_aligned(out, 16)), Q3_ERR_ALIGN);
    hipLaunchKernelGGL(embedding_kernel<float>, grid, dim3(256), 0, st, ids, static_cast<const float*>(weight),
                       static_cast<float*>(out), n, rows, dim, status);
  } else {
    return Q3_ERR_DTYPE;
  }
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

int q3_vision_rope_tables(const int* images, const int* images_host, int64_t n_img, int64_t merge, int64_t head_dim,
                          const float* inv_freq, float* cos_out, float* sin_out, void* stream) {
  Q3_REQUIRE(images && images_host && inv_freq && cos_out && sin_out, Q3_ERR_NULL);
  Q3_REQUIRE(n_img >= 0 && merge >= 1 && head_dim >= 4 && head_dim % 4 == 0, Q3_ERR_SHAPE);
  if (n_img == 0) return Q3_OK;
  int64_t total = 0;
  Q3_REQUIRE(check_images(images_host, n_img, merge, &total), Q3_ERR_SHAPE);
  Q3_REQUIRE(total * head_dim < (1ll << 40), Q3_ERR_UNSUPPORTED);
  hipLaunchKernelGGL(vision_rope_kernel, dim3((unsigned)q3_cdiv(total * head_dim, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), images, (int)n_img, total, (int)merge, (int)head_dim,
                     inv_freq, cos_out, sin_out);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

int q3_vision_pos_embed(const int* images, const int* images_host, int64_t n_img, int64_t merge, int64_t grid_side,
                        const void* table, const void* x, void* y, int64_t hidden, int dtype, void* stream) {
  Q3_REQUIRE(images && images_host && table && x && y, Q3_ERR_NULL);
  Q3_REQUIRE(n_img >= 0 && merge >= 1 && grid_side >= 1 && hidden >= 1, Q3_ERR_SHAPE);
  if (n_img == 0) return Q3_OK;
  int64_t total = 0;
  Q3_REQUIRE(check_images(images_host, n_img, merge, &total), Q3_ERR_SHAPE);
  const dim3 grid((unsigned)q3_cdiv(total, 4));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == Q3_BF16)
    hipLaunchKernelGGL(pos_embed_kernel<bf16>, grid, dim3(256), 0, st, images, (int)n_img, total, (int)merge,
                       (int)grid_side, static_cast<const bf16*>(table), static_cast<const bf16*>(x),
                       static_cast<bf16*>(y), hidden);
  else if (dtype == Q3_F32)
    hipLaunchKernelGGL(pos_embed_kernel<float>, grid, dim3(256), 0, st, images, (int)n_img, total, (int)merge,
                       (int)grid_side, static_cast<const float*>(table), static_cast<const float*>(x),
                       static_cast<float*>(y), hidden);
  else
    return Q3_ERR_DTYPE;
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

}  // extern "C"
