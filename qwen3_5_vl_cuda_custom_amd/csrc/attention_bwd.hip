// Flash-attention backward (replaces flash_attention_backward of
// csrc/flash_attention_op.cpp:15, csrc/flash_attention_op.cu:235-390): the
// gradients of O = softmax(scale * Q K^T [+ causal mask]) V with GQA, from the
// forward's row log-sum-exp, without materialising the attention matrix.
//
//   Dv[i]   = sum_d dO[i, d] O[i, d]
//   P[i, j] = exp(scale * q_i . k_j - lse[i])        (0 where masked)
//   dV[j]  += P[i, j] dO[i]           dP[i, j] = dO[i] . v_j
//   dS[i, j] = P[i, j] (dP[i, j] - Dv[i])
//   dK[j]  += scale * dS[i, j] q_i    dQ[i]  += scale * dS[i, j] k_j
//
// Two passes keep every sum in a fixed order (no atomics, bitwise reproducible
// results): a key-parallel kernel owns 64 keys of one KV head and walks the
// query rows of all the query heads that share the KV head (GQA), summing dK
// and dV in registers; a query-parallel kernel owns 64 query rows and walks
// the keys, summing dQ. Both recompute P from Q, K and the log-sum-exp. Four
// lanes share a row (key or query): lane part p holds dims p, p + 4, p + 8, ...
// (so the four lanes of a row read consecutive LDS words), dot products are
// summed over the four lanes with two shuffles. fp32 math for bf16 and fp32
// tensors; head_dim up to 128. The causal mask is top-left aligned (query i
// sees keys 0..i), as the forward's.
#include "q3_common.h"

namespace {

constexpr int kBT = 256;      // threads per block
constexpr int kRowsPB = 64;   // keys (dK/dV) or queries (dQ) per block: 4 lanes each
constexpr int kTile = 16;     // rows of the other side staged in LDS per step
constexpr int kMaxD = 128;

struct BwdParams {
  const void *q, *k, *v, *o, *dout;
  const float* lse;
  float* dvec;
  void *dq, *dk, *dv;
  int B, Hq, Hkv, Sq, Sk, D, groups;
  float scale;
  int causal;
};

__device__ __forceinline__ float quad_sum(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  return v;
}

// Dv[row] = dO[row] . O[row], one wave per row.
template <typename T>
__global__ __launch_bounds__(kBT) void attn_bwd_dvec_kernel(const BwdParams p, int64_t rows) {
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * kBT + threadIdx.x) >> 6;
  if (row >= rows) return;
  const T* o = static_cast<const T*>(p.o) + row * p.D;
  const T* g = static_cast<const T*>(p.dout) + row * p.D;
  float acc = 0.f;
  for (int d = lane; d < p.D; d += 64) acc += to_f<T>(o[d]) * to_f<T>(g[d]);
  acc = wave_sum(acc);
  if (lane == 0) p.dvec[row] = acc;
}

// dK, dV: block (key tile, b * Hkv + kv head).
template <typename T, int DS>
__global__ __launch_bounds__(kBT) void attn_bwd_dkdv_kernel(const BwdParams p) {
  constexpr int kDP = 4 * DS;  // staged row width: D rounded up to the four lanes' dims
  static_assert(kDP <= kMaxD, "head_dim <= 128");
  __shared__ float s_q[kTile][kMaxD];
  __shared__ float s_do[kTile][kMaxD];
  __shared__ float s_lse[kTile], s_dv[kTile];
  const int tid = threadIdx.x, part = tid & 3;
  const int bh = blockIdx.y, b = bh / p.Hkv, kvh = bh % p.Hkv;
  const int j0 = blockIdx.x * kRowsPB;
  const int j = j0 + (tid >> 2);
  const int D = p.D;
  const bool jv = j < p.Sk;
  const int64_t kv_base = ((int64_t)b * p.Hkv + kvh) * p.Sk;
  const T* kp = static_cast<const T*>(p.k) + (kv_base + (jv ? j : 0)) * D;
  const T* vp = static_cast<const T*>(p.v) + (kv_base + (jv ? j : 0)) * D;
  float kr[DS], vr[DS], dk[DS], dv[DS];
#pragma unroll
  for (int t = 0; t < DS; ++t) {
    const int d = part + 4 * t;
    kr[t] = (jv && d < D) ? to_f<T>(kp[d]) : 0.f;
    vr[t] = (jv && d < D) ? to_f<T>(vp[d]) : 0.f;
    dk[t] = 0.f;
    dv[t] = 0.f;
  }
  const int i_begin = p.causal ? j0 : 0;          // no earlier query sees any of the block's keys
  for (int g = 0; g < p.groups; ++g) {
    const int h = kvh * p.groups + g;
    const int64_t q_base = ((int64_t)b * p.Hq + h) * p.Sq;
    for (int i0 = i_begin; i0 < p.Sq; i0 += kTile) {
      __syncthreads();  // the previous tile's readers are done
      // rows past Sq and dims in [D, 4 * DS) are staged as zeros (every word a lane reads is written)
      for (int e = tid; e < kTile * kDP; e += kBT) {
        const int r = e / kDP, d = e % kDP, i = i0 + r;
        const bool ok = i < p.Sq && d < D;
        s_q[r][d] = ok ? to_f<T>(static_cast<const T*>(p.q)[(q_base + i) * D + d]) : 0.f;
        s_do[r][d] = ok ? to_f<T>(static_cast<const T*>(p.dout)[(q_base + i) * D + d]) : 0.f;
      }
      if (tid < kTile) {
        const int i = i0 + tid;
        s_lse[tid] = i < p.Sq ? p.lse[q_base + i] : 0.f;
        s_dv[tid] = i < p.Sq ? p.dvec[q_base + i] : 0.f;
      }
      __syncthreads();
      const int nr = min(kTile, p.Sq - i0);
      for (int r = 0; r < nr; ++r) {
        const int i = i0 + r;
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int t = 0; t < DS; ++t) {
          s += s_q[r][part + 4 * t] * kr[t];
          dp += s_do[r][part + 4 * t] * vr[t];
        }
        s = quad_sum(s);
        dp = quad_sum(dp);
        const bool live = jv && (!p.causal || j <= i);
        const float pr = live ? expf(p.scale * s - s_lse[r]) : 0.f;
        const float ds = pr * (dp - s_dv[r]);
#pragma unroll
        for (int t = 0; t < DS; ++t) {
          dv[t] += pr * s_do[r][part + 4 * t];
          dk[t] += ds * s_q[r][part + 4 * t];
        }
      }
    }
  }
  if (!jv) return;
  T* dkp = static_cast<T*>(p.dk) + (kv_base + j) * D;
  T* dvp = static_cast<T*>(p.dv) + (kv_base + j) * D;
#pragma unroll
  for (int t = 0; t < DS; ++t) {
    const int d = part + 4 * t;
    if (d < D) {
      dkp[d] = from_f<T>(dk[t] * p.scale);
      dvp[d] = from_f<T>(dv[t]);
    }
  }
}

// dQ: block (query tile, b * Hq + head).
template <typename T, int DS>
__global__ __launch_bounds__(kBT) void attn_bwd_dq_kernel(const BwdParams p) {
  constexpr int kDP = 4 * DS;
  static_assert(kDP <= kMaxD, "head_dim <= 128");
  __shared__ float s_k[kTile][kMaxD];
  __shared__ float s_v[kTile][kMaxD];
  const int tid = threadIdx.x, part = tid & 3;
  const int bh = blockIdx.y, b = bh / p.Hq, h = bh % p.Hq;
  const int kvh = h / p.groups;
  const int i0 = blockIdx.x * kRowsPB;
  const int i = i0 + (tid >> 2);
  const int D = p.D;
  const bool iv = i < p.Sq;
  const int64_t q_row = ((int64_t)b * p.Hq + h) * p.Sq + (iv ? i : 0);
  const T* qp = static_cast<const T*>(p.q) + q_row * D;
  const T* gp = static_cast<const T*>(p.dout) + q_row * D;
  float qr[DS], gr[DS], dq[DS];
#pragma unroll
  for (int t = 0; t < DS; ++t) {
    const int d = part + 4 * t;
    qr[t] = (iv && d < D) ? to_f<T>(qp[d]) : 0.f;
    gr[t] = (iv && d < D) ? to_f<T>(gp[d]) : 0.f;
    dq[t] = 0.f;
  }
  const float lse = iv ? p.lse[q_row] : 0.f;
  const float dvi = iv ? p.dvec[q_row] : 0.f;
  const int64_t kv_base = ((int64_t)b * p.Hkv + kvh) * p.Sk;
  // keys past the block's last query are masked for every row of the block
  const int j_end = p.causal ? min(p.Sk, min(i0 + kRowsPB, p.Sq)) : p.Sk;
  for (int j0 = 0; j0 < j_end; j0 += kTile) {
    __syncthreads();
    for (int e = tid; e < kTile * kDP; e += kBT) {
      const int r = e / kDP, d = e % kDP, j = j0 + r;
      const bool ok = j < p.Sk && d < D;
      s_k[r][d] = ok ? to_f<T>(static_cast<const T*>(p.k)[(kv_base + j) * D + d]) : 0.f;
      s_v[r][d] = ok ? to_f<T>(static_cast<const T*>(p.v)[(kv_base + j) * D + d]) : 0.f;
    }
    __syncthreads();
    const int nr = min(kTile, j_end - j0);
    for (int r = 0; r < nr; ++r) {
      const int j = j0 + r;
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int t = 0; t < DS; ++t) {
        s += qr[t] * s_k[r][part + 4 * t];
        dp += gr[t] * s_v[r][part + 4 * t];
      }
      s = quad_sum(s);
      dp = quad_sum(dp);
      const bool live = iv && (!p.causal || j <= i);
      const float pr = live ? expf(p.scale * s - lse) : 0.f;
      const float ds = pr * (dp - dvi);
#pragma unroll
      for (int t = 0; t < DS; ++t) dq[t] += ds * s_k[r][part + 4 * t];
    }
  }
  if (!iv) return;
  T* dqp = static_cast<T*>(p.dq) + q_row * D;
#pragma unroll
  for (int t = 0; t < DS; ++t) {
    const int d = part + 4 * t;
    if (d < D) dqp[d] = from_f<T>(dq[t] * p.scale);
  }
}

template <typename T, int DS>
int attn_bwd_t(const BwdParams& p, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
  hipLaunchKernelGGL(attn_bwd_dvec_kernel<T>, dim3((unsigned)q3_cdiv(rows, kBT / 64)), dim3(kBT), 0, st, p, rows);
  Q3_LAUNCH_CHECK();
  if (p.Sk > 0) {
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, DS>), dim3((unsigned)q3_cdiv(p.Sk, kRowsPB), (unsigned)(p.B * p.Hkv)),
                       dim3(kBT), 0, st, p);
    Q3_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL((attn_bwd_dq_kernel<T, DS>), dim3((unsigned)q3_cdiv(p.Sq, kRowsPB), (unsigned)(p.B * p.Hq)),
                     dim3(kBT), 0, st, p);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

template <typename T>
int attn_bwd_d(const BwdParams& p, hipStream_t st) {
  if (p.D <= 32) return attn_bwd_t<T, 8>(p, st);
  if (p.D <= 64) return attn_bwd_t<T, 16>(p, st);
  if (p.D <= 96) return attn_bwd_t<T, 24>(p, st);
  return attn_bwd_t<T, 32>(p, st);
}

}  // namespace

extern "C" {

int64_t q3_flash_attention_backward_workspace_bytes(int64_t B, int64_t Hq, int64_t Sq) {
  if (B <= 0 || Hq <= 0 || Sq <= 0) return 0;
  return B * Hq * Sq * 4;
}

int q3_flash_attention_backward(const void* q, const void* k, const void* v, const void* o, const float* lse,
                                const void* grad_out, void* grad_q, void* grad_k, void* grad_v, int64_t B, int64_t Hq,
                                int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, float scale, int is_causal,
                                int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  Q3_REQUIRE(q && k && v && o && lse && grad_out && grad_q && grad_k && grad_v, Q3_ERR_NULL);
  Q3_REQUIRE(B >= 0 && Hq >= 1 && Hkv >= 1 && Sq >= 0 && Sk >= 0 && D >= 1, Q3_ERR_SHAPE);
  Q3_REQUIRE(Hq % Hkv == 0 && B * Hq < 65536 && Sq < (1ll << 30) && Sk < (1ll << 30), Q3_ERR_SHAPE);
  Q3_REQUIRE(D <= kMaxD, Q3_ERR_UNSUPPORTED);
  Q3_REQUIRE(dtype == Q3_BF16 || dtype == Q3_F32, Q3_ERR_DTYPE);
  if (B == 0 || Sq == 0) return Q3_OK;
  Q3_REQUIRE(workspace && workspace_bytes >= q3_flash_attention_backward_workspace_bytes(B, Hq, Sq),
             Q3_ERR_WORKSPACE);
  Q3_REQUIRE(q3_aligned(workspace, 4), Q3_ERR_ALIGN);
  BwdParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.dout = grad_out;
  p.lse = lse;
  p.dvec = static_cast<float*>(workspace);
  p.dq = grad_q;
  p.dk = grad_k;
  p.dv = grad_v;
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.Sq = (int)Sq;
  p.Sk = (int)Sk;
  p.D = (int)D;
  p.groups = (int)(Hq / Hkv);
  p.scale = scale;
  p.causal = is_causal ? 1 : 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == Q3_BF16) return attn_bwd_d<bf16>(p, st);
  return attn_bwd_d<float>(p, st);
}

}  // extern "C"
