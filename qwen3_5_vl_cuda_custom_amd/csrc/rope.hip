// Rotary position embedding kernels.
//
//  q3_rope          rotate-half RoPE with a cos/sin table (S, Dr) or (B, S, Dr)
//  q3_mrope         rotate-half mRoPE with cos/sin (3, B, S, Dr) and the
//                   chunked section layout: for i < Dr/2, element i uses axis
//                   0 if i < s0, axis 1 if i < s0 + s1, else axis 2
//  q3_qk_norm_rope  fused attention prologue: per-head RMSNorm of q and k, mRoPE
//                   from integer positions (angles pos * inv_freq in fp32, as
//                   the reference builds them), copy of v, all read from the
//                   projection outputs in (B, S, H, D) layout and written to any
//                   strided destination (e.g. straight into a KV cache)
//
// Rotate-half on pairs (i, i + Dr/2) with c = cos[i], s = sin[i], i < Dr/2:
//   y[i] = x[i] c - x[i + Dr/2] s,   y[i + Dr/2] = x[i + Dr/2] c + x[i] s
// and dims >= Dr pass through.
#include <type_traits>

#include "q3_common.h"

namespace {

struct RopeGeom {
  int B, H, S, D, Dr;
  int64_t xb, xh, xs;  // x strides
  int64_t yb, yh, ys;  // y strides
  int64_t ca, cb, cs;  // cos/sin strides: axis, batch, seq (element i contiguous)
  int s0, s1;          // section boundaries (plain rope: s0 = Dr/2)
};

template <typename T, typename TC>
__global__ __launch_bounds__(256) void rope_kernel(const T* __restrict__ x, const TC* __restrict__ cosp,
                                                   const TC* __restrict__ sinp, T* __restrict__ y, RopeGeom g) {
  const int half = g.Dr / 2;
  const int per_row = half + (g.D - g.Dr);
  const int64_t total = (int64_t)g.B * g.H * g.S * per_row;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int j = (int)(t % per_row);
    int64_t row = t / per_row;
    const int s = (int)(row % g.S);
    row /= g.S;
    const int h = (int)(row % g.H);
    const int b = (int)(row / g.H);
    const T* xr = x + b * g.xb + h * g.xh + s * g.xs;
    T* yr = y + b * g.yb + h * g.yh + s * g.ys;
    if (j < half) {
      const int axis = (j < g.s0) ? 0 : (j < g.s0 + g.s1 ? 1 : 2);
      const int64_t co = axis * g.ca + b * g.cb + s * g.cs + j;
      const float c = to_f<TC>(cosp[co]);
      const float sn = to_f<TC>(sinp[co]);
      const float x1 = to_f<T>(xr[j]);
      const float x2 = to_f<T>(xr[j + half]);
      yr[j] = from_f<T>(x1 * c - x2 * sn);
      yr[j + half] = from_f<T>(x2 * c + x1 * sn);
    } else {
      const int d = g.Dr + (j - half);
      yr[d] = xr[d];
    }
  }
}

// The same rotation with V consecutive pairs per thread (vector loads of x,
// y, cos and sin) and 32-bit index arithmetic: thread t handles slot t % P of
// row t / P, rows ordered (b, h, s), P = (Dr/2 + D - Dr) / V slots per row.
// Slots below Dr/2 V rotate pairs [j, j + V) with [j + Dr/2, ...); the others
// copy V pass-through elements (skipped when y aliases x in place).
template <typename T, int V>
using vec_t = T __attribute__((ext_vector_type(V)));

template <typename T, typename TC, int V>
__global__ __launch_bounds__(256) void rope_vec_kernel(const T* x, const TC* __restrict__ cosp,
                                                       const TC* __restrict__ sinp, T* y, RopeGeom g,
                                                       int P, int total, int copy_tail) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  const int half = g.Dr / 2;
  int row = t / P;
  const int j = (t - row * P) * V;
  const int s = row % g.S;
  row /= g.S;
  const int h = row % g.H;
  const int b = row / g.H;
  const T* xr = x + b * g.xb + h * g.xh + s * g.xs;
  T* yr = y + b * g.yb + h * g.yh + s * g.ys;
  if (j < half) {
    const vec_t<T, V> x1 = *reinterpret_cast<const vec_t<T, V>*>(xr + j);
    const vec_t<T, V> x2 = *reinterpret_cast<const vec_t<T, V>*>(xr + j + half);
    float c[V], sn[V];
    if (g.s0 >= half) {  // one axis: the table row is contiguous
      const int64_t co = b * g.cb + s * g.cs + j;
      const vec_t<TC, V> cv = *reinterpret_cast<const vec_t<TC, V>*>(cosp + co);
      const vec_t<TC, V> sv = *reinterpret_cast<const vec_t<TC, V>*>(sinp + co);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        c[e] = to_f<TC>(cv[e]);
        sn[e] = to_f<TC>(sv[e]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const int i = j + e;
        const int axis = (i < g.s0) ? 0 : (i < g.s0 + g.s1 ? 1 : 2);
        const int64_t co = axis * g.ca + b * g.cb + s * g.cs + i;
        c[e] = to_f<TC>(cosp[co]);
        sn[e] = to_f<TC>(sinp[co]);
      }
    }
    vec_t<T, V> y1, y2;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float a = to_f<T>(x1[e]), bb = to_f<T>(x2[e]);
      y1[e] = from_f<T>(a * c[e] - bb * sn[e]);
      y2[e] = from_f<T>(bb * c[e] + a * sn[e]);
    }
    *reinterpret_cast<vec_t<T, V>*>(yr + j) = y1;
    *reinterpret_cast<vec_t<T, V>*>(yr + j + half) = y2;
  } else if (copy_tail) {
    const int d = g.Dr + (j - half);
    *reinterpret_cast<vec_t<T, V>*>(yr + d) = *reinterpret_cast<const vec_t<T, V>*>(xr + d);
  }
}

template <typename T, typename TC, int V>
bool try_rope_vec(const void* x, const void* cosp, const void* sinp, void* y, const RopeGeom& g, hipStream_t st) {
  const int half = g.Dr / 2, tail = g.D - g.Dr;
  if (half % V || tail % V) return false;
  const int64_t ve = V * (int64_t)sizeof(T), vc = V * (int64_t)sizeof(TC);
  auto al = [](const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)a) == 0; };
  const int64_t ts = sizeof(T), cs = sizeof(TC);
  bool ok = al(x, ve) && al(y, ve) && al(cosp, vc) && al(sinp, vc);
  for (int64_t st_ : {g.xb, g.xh, g.xs, g.yb, g.yh, g.ys}) ok = ok && (st_ * ts) % ve == 0;
  for (int64_t st_ : {g.ca, g.cb, g.cs}) ok = ok && (st_ * cs) % vc == 0;
  const int64_t P = (half + tail) / V;
  const int64_t rows = (int64_t)g.B * g.H * g.S;
  if (!ok || rows * P >= (1ll << 31) - 256) return false;
  const int total = (int)(rows * P);
  const int copy_tail = tail > 0 && (x != y);
  hipLaunchKernelGGL((rope_vec_kernel<T, TC, V>), dim3((unsigned)q3_cdiv(total, 256)), dim3(256), 0, st,
                     static_cast<const T*>(x), static_cast<const TC*>(cosp), static_cast<const TC*>(sinp),
                     static_cast<T*>(y), g, (int)P, total, copy_tail);
  return true;
}

template <typename T, typename TC>
bool try_rope_fast(const void* x, const void* cosp, const void* sinp, void* y, const RopeGeom& g, hipStream_t st) {
  return try_rope_vec<T, TC, 4>(x, cosp, sinp, y, g, st) || try_rope_vec<T, TC, 2>(x, cosp, sinp, y, g, st) ||
         try_rope_vec<T, TC, 1>(x, cosp, sinp, y, g, st);
}

template <typename T>
int launch_rope_t(const void* x, const void* cosp, const void* sinp, void* y, const RopeGeom& g, int cos_dtype,
                  hipStream_t st) {
  const int64_t total = (int64_t)g.B * g.H * g.S * (g.Dr / 2 + g.D - g.Dr);
  if (total == 0) return Q3_OK;
  if (cos_dtype == Q3_F32 ? try_rope_fast<T, float>(x, cosp, sinp, y, g, st)
                          : cos_dtype == Q3_BF16 && try_rope_fast<T, bf16>(x, cosp, sinp, y, g, st)) {
    Q3_LAUNCH_CHECK();
    return Q3_OK;
  }
  const unsigned blocks = (unsigned)std::min<int64_t>(q3_cdiv(total, 256), 65536);
  if (cos_dtype == Q3_F32)
    hipLaunchKernelGGL((rope_kernel<T, float>), dim3(blocks), dim3(256), 0, st, static_cast<const T*>(x),
                       static_cast<const float*>(cosp), static_cast<const float*>(sinp), static_cast<T*>(y), g);
  else if (cos_dtype == Q3_BF16)
    hipLaunchKernelGGL((rope_kernel<T, bf16>), dim3(blocks), dim3(256), 0, st, static_cast<const T*>(x),
                       static_cast<const bf16*>(cosp), static_cast<const bf16*>(sinp), static_cast<T*>(y), g);
  else
    return Q3_ERR_DTYPE;
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

int launch_rope(const void* x, const void* cosp, const void* sinp, void* y, const RopeGeom& g, int dtype,
                int cos_dtype, hipStream_t st) {
  Q3_REQUIRE(x && cosp && sinp && y, Q3_ERR_NULL);
  Q3_REQUIRE(g.B >= 0 && g.H >= 0 && g.S >= 0 && g.D >= 1, Q3_ERR_SHAPE);
  Q3_REQUIRE(g.Dr >= 2 && g.Dr % 2 == 0 && g.Dr <= g.D, Q3_ERR_SHAPE);
  Q3_REQUIRE(g.s0 >= 0 && g.s1 >= 0 && g.s0 + g.s1 <= g.Dr / 2, Q3_ERR_SHAPE);
  if (dtype == Q3_BF16) return launch_rope_t<bf16>(x, cosp, sinp, y, g, cos_dtype, st);
  if (dtype == Q3_F32) return launch_rope_t<float>(x, cosp, sinp, y, g, cos_dtype, st);
  return Q3_ERR_DTYPE;
}

// ------------------------------------------------------------------ fused prologue
struct QKNormRopeArgs {
  const void* q_in;
  const void* k_in;
  const void* v_in;
  void* q_out;
  void* k_out;
  void* v_out;
  const void* q_w;
  const void* k_w;
  const int* pos;          // (3, B, S) int32
  const float* inv_freq;   // (D/2) fp32
  const int* dst_seq_off;  // (B) int32 offset added to s for k_out / v_out, or null
  int64_t dst_seq_cap;     // k_out / v_out rows at sequence index >= cap are not written
  int B, S, Hq, Hkv, D;
  int s0, s1;
  float eps;
  int64_t st[18];  // (b, s, h) strides of q_in, k_in, v_in, q_out, k_out, v_out
  // Paged k_out / v_out (null: strided as above): cache row r (= s + offset) of
  // sequence b is row r % page_rows of page block_table[b * max_pages +
  // r / page_rows], and the b strides of k_out / v_out are the page strides. A
  // page id outside [0, num_pages) drops the row and sets bit 1 of *status.
  const int* block_table;
  int max_pages, page_rows, num_pages;
  int* status;
  // If set, token t = b * S + s writes its rotary table row: D fp32 values,
  // cos of the D/2 angles then their sin (for a consumer that rotates q
  // itself). q_in == null: the q rows are not processed (k and v only).
  float* rope_tab;
};

// One block per (b, s) token. The D/2 rotary angles of the token (pos[axis]
// * inv_freq[i], fp32, sincosf) are computed once into LDS and shared by all
// of its q, k (and v) head rows. A group of G = D/8 lanes handles one head
// row, lane j holding elements [8j, 8j+8); the rotate-half partner of lane j
// is lane j ^ (G/2). A lane group loads BATCH of its rows at a time (rows
// past the end repeat the last one). BATCH = 1 with at most 80 VGPRs (six
// waves per SIMD) measured fastest at D = 128, 48 rows per token: S=4096
// 27.8 -> 23.5 us, a 32-token decode step 5.4 -> 5.1 us; a batch that does
// not divide the 16-row passes into the token's rows (2, 4) loads rows it
// never uses, and 8 waves per SIMD spill. The fp32 and unaligned forms keep
// the default bound (at 80 VGPRs they spill).
constexpr int kQKBatch = 1;
constexpr int kQKMinBlocks = 6;

// One of three kernel arguments by a per-lane index, as selects (indexing the
// argument array with a lane-varying index would load it from memory).
__device__ __forceinline__ int64_t pick3(int k, int64_t x0, int64_t x1, int64_t x2) {
  return k == 0 ? x0 : (k == 1 ? x1 : x2);
}

// Eight consecutive elements at p (16-byte vectors when VEC: p 16-byte aligned).
template <typename T, bool VEC>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  if constexpr (VEC) {
    typedef typename Vec16<T>::type VT;
    constexpr int N = Vec16<T>::N;
#pragma unroll
    for (int c = 0; c < 8 / N; ++c) {
      const VT u = reinterpret_cast<const VT*>(p)[c];
#pragma unroll
      for (int e = 0; e < N; ++e) v[c * N + e] = to_f<T>(u[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = to_f<T>(p[e]);
  }
}
template <typename T, bool VEC>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  if constexpr (VEC) {
    typedef typename Vec16<T>::type VT;
    constexpr int N = Vec16<T>::N;
#pragma unroll
    for (int c = 0; c < 8 / N; ++c) {
      VT u;
#pragma unroll
      for (int e = 0; e < N; ++e) u[e] = from_f<T>(v[c * N + e]);
      reinterpret_cast<VT*>(p)[c] = u;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = from_f<T>(v[e]);
  }
}

// Row `row` of a token's q | k | v rows: kind 0 = q, 1 = k, 2 = v, and its head.
__device__ __forceinline__ void qk_row_kind(const QKNormRopeArgs& a, int row, int& kind, int& h) {
  kind = row < a.Hq ? 0 : (row < a.Hq + a.Hkv ? 1 : 2);
  h = kind == 0 ? row : (kind == 1 ? row - a.Hq : row - a.Hq - a.Hkv);
}

// Input row `row` of token (b, s).
template <typename T>
__device__ __forceinline__ const T* qk_in_row(const QKNormRopeArgs& a, int64_t b, int64_t s, int row) {
  int kind, h;
  qk_row_kind(a, row, kind, h);
  return static_cast<const T*>(kind == 0 ? a.q_in : (kind == 1 ? a.k_in : a.v_in)) +
         b * pick3(kind, a.st[0], a.st[3], a.st[6]) + s * pick3(kind, a.st[1], a.st[4], a.st[7]) +
         h * pick3(kind, a.st[2], a.st[5], a.st[8]);
}

// One head row of token (b, s), held by a group of G lanes (lane j: elements
// [8j, 8j+8) in x): RMSNorm (with weights) and mRoPE for q and k rows, then the
// store (k / v rows at sequence offset so_b, through the block table when
// paged; rows past dst_seq_cap or on a rejected page are not written).
template <typename T, int G, bool VEC>
__device__ __forceinline__ void qk_row(const QKNormRopeArgs& a, int64_t b, int64_t s, int row, int j, int so_b,
                                       float (&x)[8], const float (&cs)[8], const float (&sn)[8],
                                       const float (&wq)[8], const float (&wk)[8]) {
  constexpr int D = G * 8;
  const bool lo = j < G / 2;
  int kind, h;
  qk_row_kind(a, row, kind, h);
  const int so = kind > 0 ? so_b : 0;
  bool skip_store = kind > 0 && (s + (int64_t)so >= a.dst_seq_cap || s + so < 0);
  int64_t ob = b, orow = s + so;  // k / v: page and row within it when paged
  if (kind > 0 && a.block_table && !skip_store) {
    const int pg = a.block_table[b * a.max_pages + orow / a.page_rows];
    if ((unsigned)pg >= (unsigned)a.num_pages) {
      if (a.status && j == 0) atomicOr(a.status, 2);
      skip_store = true;
    }
    ob = pg;
    orow %= a.page_rows;
  }
  T* out = static_cast<T*>(kind == 0 ? a.q_out : (kind == 1 ? a.k_out : a.v_out)) +
           ob * pick3(kind, a.st[9], a.st[12], a.st[15]) + orow * pick3(kind, a.st[10], a.st[13], a.st[16]) +
           h * pick3(kind, a.st[11], a.st[14], a.st[17]);
  if (kind < 2) {
    // RMSNorm over the head (skipped when no weights are given).
    if (a.q_w != nullptr) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
      ss = group_sum<G>(ss);
      const float rstd = rsqrtf(ss / (float)D + a.eps);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = x[e] * rstd * (kind == 0 ? wq[e] : wk[e]);
    }
    // mRoPE.
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = __shfl_xor(x[e], G / 2, 64);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      // lo half: x1*c - x2*s  (partner holds x2); hi half: x2*c + x1*s (partner holds x1).
      x[e] = lo ? (x[e] * cs[e] - p[e] * sn[e]) : (x[e] * cs[e] + p[e] * sn[e]);
  }
  if (skip_store) return;
  store8<T, VEC>(out + 8 * j, x);
}

template <typename T, int G, bool VEC, int BATCH = kQKBatch, int MINB = 1>
__global__ __launch_bounds__(256, MINB) void qk_norm_rope_kernel(const QKNormRopeArgs a) {
  constexpr int D = G * 8;
  constexpr int HALF = D / 2;
  constexpr int RPP = 256 / G;  // rows per pass of the block
  __shared__ float s_cos[HALF], s_sin[HALF];
  const int tid = threadIdx.x;
  const int b = blockIdx.x / a.S, s = blockIdx.x % a.S;
  const int j = tid % G;
  const int nrows = a.Hq + a.Hkv + (a.v_out ? a.Hkv : 0);

  // The token's angles: thread i < HALF loads its position and frequency.
  int posv = 0;
  float fr = 0.f;
  if (tid < HALF) {
    const int axis = (tid < a.s0) ? 0 : (tid < a.s0 + a.s1 ? 1 : 2);
    posv = a.pos[((int64_t)axis * a.B + b) * a.S + s];
    fr = a.inv_freq[tid];
  }
  // Norm weights of lane j (read from q_in when there are none: never used).
  const bool has_w = a.q_w != nullptr;
  float wq[8], wk[8];
  load8<T, VEC>(static_cast<const T*>(has_w ? a.q_w : a.q_in) + 8 * j, wq);
  load8<T, VEC>(static_cast<const T*>(has_w ? a.k_w : a.q_in) + 8 * j, wk);
  // Rows past the end load row nrows - 1 again (no branch around the loads).
  float v[BATCH][8];
  auto load_batch = [&](int r0) {
#pragma unroll
    for (int u = 0; u < BATCH; ++u) load8<T, VEC>(qk_in_row<T>(a, b, s, min(r0 + u * RPP, nrows - 1)) + 8 * j, v[u]);
  };
  // gridDim.y blocks share a token's rows: block y takes passes y, y + gridDim.y, ...
  const int first = (a.q_in ? 0 : a.Hq) + (int)blockIdx.y * BATCH * RPP + tid / G;
  load_batch(first);
  const int so_b = a.dst_seq_off ? a.dst_seq_off[b] : 0;
  if (tid < HALF) {
    float sn, c;
    sincosf((float)posv * fr, &sn, &c);
    s_cos[tid] = c;
    s_sin[tid] = sn;
    if (a.rope_tab) {
      float* tr = a.rope_tab + (int64_t)blockIdx.x * D;
      tr[tid] = c;
      tr[HALF + tid] = sn;
    }
  }
  __syncthreads();
  float cs[8], sn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int i = (8 * j + e) % HALF;
    cs[e] = s_cos[i];
    sn[e] = s_sin[i];
  }
  for (int r0 = first; r0 < nrows; r0 += BATCH * RPP * (int)gridDim.y) {  // uniform per lane group
    if (r0 != first) load_batch(r0);
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int row = r0 + u * RPP;
      if (row >= nrows) break;
      qk_row<T, G, VEC>(a, b, s, row, j, so_b, v[u], cs, sn, wq, wk);
    }
  }
}

// k rows only, with the rotary table written (the fused prefill prologue: q
// is rotated by the attention kernel). TPB tokens per block, so that the
// per-token latency chain (position load, sincosf, LDS exchange) of several
// tokens overlaps: thread i < TPB * D/2 computes angle i % (D/2) of token
// i / (D/2); lane groups of G take the block's TPB * Hkv k rows, RPP at a
// time. bf16 with 16-byte aligned rows; same per-row arithmetic as
// qk_norm_rope_kernel (qk_row).
template <int G, int TPB>
__global__ __launch_bounds__(256) void k_norm_rope_table_kernel(const QKNormRopeArgs a) {
  constexpr int D = G * 8;
  constexpr int HALF = D / 2;
  constexpr int RPP = 256 / G;
  static_assert(TPB * HALF <= 256, "one angle per thread");
  __shared__ float s_cos[TPB][HALF], s_sin[TPB][HALF];
  const int tid = threadIdx.x;
  const int j = tid % G;
  const int64_t ntok = (int64_t)a.B * a.S;
  const int64_t tok0 = (int64_t)blockIdx.x * TPB;
  const int nrows = TPB * a.Hkv;
  auto token_of = [&](int r, int64_t& b, int64_t& s) {
    const int64_t tok = min(tok0 + r / a.Hkv, ntok - 1);
    b = tok / a.S;
    s = tok % a.S;
  };
  float wq[8], wk[8];
  load8<bf16, true>(static_cast<const bf16*>(a.q_w) + 8 * j, wq);
  load8<bf16, true>(static_cast<const bf16*>(a.k_w) + 8 * j, wk);
  const int first = tid / G;
  float x[8];
  {
    int64_t b, s;
    token_of(min(first, nrows - 1), b, s);
    load8<bf16, true>(qk_in_row<bf16>(a, b, s, a.Hq + min(first, nrows - 1) % a.Hkv) + 8 * j, x);
  }
  if (tid < TPB * HALF) {
    const int tt = tid / HALF, i = tid % HALF;
    const int64_t tok = min(tok0 + tt, ntok - 1);
    const int64_t b = tok / a.S, s = tok % a.S;
    const int axis = (i < a.s0) ? 0 : (i < a.s0 + a.s1 ? 1 : 2);
    const int posv = a.pos[((int64_t)axis * a.B + b) * a.S + s];
    float sn, c;
    sincosf((float)posv * a.inv_freq[i], &sn, &c);
    s_cos[tt][i] = c;
    s_sin[tt][i] = sn;
    if (tok0 + tt < ntok) {
      float* tr = a.rope_tab + tok * D;
      tr[i] = c;
      tr[HALF + i] = sn;
    }
  }
  __syncthreads();
  for (int r = first; r < nrows; r += RPP) {  // uniform per lane group
    if (tok0 + r / a.Hkv >= ntok) break;
    int64_t b, s;
    token_of(r, b, s);
    const int row = a.Hq + r % a.Hkv;
    if (r != first) load8<bf16, true>(qk_in_row<bf16>(a, b, s, row) + 8 * j, x);
    const int tt = r / a.Hkv;
    float cs[8], sn[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = (8 * j + e) % HALF;
      cs[e] = s_cos[tt][i];
      sn[e] = s_sin[tt][i];
    }
    qk_row<bf16, G, true>(a, b, s, row, j, 0, x, cs, sn, wq, wk);
  }
}

template <typename T>
int launch_qk(const QKNormRopeArgs& a, hipStream_t st) {
  const int64_t tokens = (int64_t)a.B * a.S;
  if (tokens == 0) return Q3_OK;
  Q3_REQUIRE(tokens < (1ll << 31), Q3_ERR_SHAPE);
  const int G = a.D / 8;
  // 16-byte vector access when every row start is 16-byte aligned.
  bool vec = q3_aligned(a.q_in, 16) && q3_aligned(a.k_in, 16) && q3_aligned(a.q_out, 16) &&
             q3_aligned(a.k_out, 16) && (!a.v_in || (q3_aligned(a.v_in, 16) && q3_aligned(a.v_out, 16))) &&
             (!a.q_w || (q3_aligned(a.q_w, 16) && q3_aligned(a.k_w, 16)));
  for (int i = 0; i < 18; ++i) vec = vec && (a.st[i] * (int64_t)sizeof(T)) % 16 == 0;
  // Few tokens (decode): the passes over a token's rows run in parallel blocks
  // instead of one after another (each block recomputes the token's angles).
  const int rows = (a.q_in ? a.Hq : 0) + a.Hkv + (a.v_out ? a.Hkv : 0);
  const int passes = (int)q3_cdiv(rows, kQKBatch * (256 / G));
  const unsigned ysplit = tokens <= 256 ? (unsigned)std::max(passes, 1) : 1u;
  auto go = [&](auto g, auto v) {
    constexpr int minb = std::is_same<T, bf16>::value && decltype(v)::value ? kQKMinBlocks : 1;
    hipLaunchKernelGGL((qk_norm_rope_kernel<T, decltype(g)::value, decltype(v)::value, kQKBatch, minb>),
                       dim3((unsigned)tokens, ysplit), dim3(256), 0, st, a);
  };
  using VT = std::true_type;
  using VF = std::false_type;
  switch (G) {
    case 8:
      vec ? go(std::integral_constant<int, 8>{}, VT{}) : go(std::integral_constant<int, 8>{}, VF{});
      break;
    case 16:
      vec ? go(std::integral_constant<int, 16>{}, VT{}) : go(std::integral_constant<int, 16>{}, VF{});
      break;
    case 32:
      vec ? go(std::integral_constant<int, 32>{}, VT{}) : go(std::integral_constant<int, 32>{}, VF{});
      break;
    default:
      return Q3_ERR_UNSUPPORTED;
  }
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

}  // namespace

namespace {

int qk_impl(const void* q_in, const void* k_in, const void* v_in, void* q_out, void* k_out, void* v_out,
            const void* q_weight, const void* k_weight, const int* positions, const float* inv_freq,
            const int* dst_seq_offset, int64_t dst_seq_cap, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
            int64_t D, const int64_t* section, float eps, const int64_t* strides, int dtype, const int* block_table,
            int64_t max_pages, int64_t page_rows, int64_t num_pages, int* status, void* stream) {
  Q3_REQUIRE(q_in && k_in && q_out && k_out && positions && inv_freq && section && strides, Q3_ERR_NULL);
  Q3_REQUIRE((q_weight == nullptr) == (k_weight == nullptr), Q3_ERR_NULL);
  Q3_REQUIRE((v_in == nullptr) == (v_out == nullptr), Q3_ERR_NULL);
  Q3_REQUIRE(B >= 0 && S >= 0 && Hq >= 1 && Hkv >= 1 && D >= 16, Q3_ERR_SHAPE);
  Q3_REQUIRE(D % 16 == 0 && D <= 256, Q3_ERR_UNSUPPORTED);
  Q3_REQUIRE(section[0] >= 0 && section[1] >= 0 && section[2] >= 0 && section[0] + section[1] + section[2] == D / 2,
             Q3_ERR_SHAPE);
  QKNormRopeArgs a{};
  a.q_in = q_in;
  a.k_in = k_in;
  a.v_in = v_in;
  a.q_out = q_out;
  a.k_out = k_out;
  a.v_out = v_out;
  a.q_w = q_weight;
  a.k_w = k_weight;
  a.pos = positions;
  a.inv_freq = inv_freq;
  a.dst_seq_off = dst_seq_offset;
  a.dst_seq_cap = dst_seq_cap > 0 ? dst_seq_cap : INT64_MAX;
  a.B = (int)B;
  a.S = (int)S;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.D = (int)D;
  a.s0 = (int)section[0];
  a.s1 = (int)section[1];
  a.eps = eps;
  for (int i = 0; i < 18; ++i) a.st[i] = strides[i];
  a.block_table = block_table;
  a.max_pages = (int)max_pages;
  a.page_rows = (int)page_rows;
  a.num_pages = (int)num_pages;
  a.status = status;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == Q3_BF16) return launch_qk<bf16>(a, st);
  if (dtype == Q3_F32) return launch_qk<float>(a, st);
  return Q3_ERR_DTYPE;
}

}  // namespace

namespace q3 {

// k rows only: per-head RMSNorm + mRoPE of k in place ((b, s, h) element
// strides kst), and each token's rotary table row into tab (B * S rows of D
// fp32). bf16; the caller has validated shapes and pointers.
int k_norm_rope_table(void* k, const void* q_weight, const void* k_weight, const int* positions,
                      const float* inv_freq, float* tab, int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                      const int64_t* section, float eps, const int64_t* kst, hipStream_t st) {
  QKNormRopeArgs a{};
  a.k_in = k;
  a.k_out = k;
  a.q_w = q_weight;
  a.k_w = k_weight;
  a.pos = positions;
  a.inv_freq = inv_freq;
  a.dst_seq_cap = INT64_MAX;
  a.B = (int)B;
  a.S = (int)S;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.D = (int)D;
  a.s0 = (int)section[0];
  a.s1 = (int)section[1];
  a.eps = eps;
  for (int i = 0; i < 3; ++i) a.st[3 + i] = a.st[12 + i] = kst[i];
  a.rope_tab = tab;
  bool vec = q3_aligned(k, 16) && q3_aligned(q_weight, 16) && q3_aligned(k_weight, 16);
  for (int i = 0; i < 3; ++i) vec = vec && (kst[i] * 2) % 16 == 0;
  if (!vec || (D != 64 && D != 128)) return launch_qk<bf16>(a, st);  // one token per block
  const int64_t tokens = B * S;
  if (tokens == 0) return Q3_OK;
  constexpr int kTPB = 4;
  const dim3 grid((unsigned)q3_cdiv(tokens, kTPB));
  if (D == 128)
    hipLaunchKernelGGL((k_norm_rope_table_kernel<16, kTPB>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((k_norm_rope_table_kernel<8, kTPB>), grid, dim3(256), 0, st, a);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

}  // namespace q3

extern "C" {

int q3_rope(const void* x, const void* cos, const void* sin, void* y, int64_t B, int64_t H, int64_t S, int64_t D,
            int64_t D_rope, const int64_t* x_strides, const int64_t* y_strides, int64_t cos_batch_stride,
            int64_t cos_seq_stride, int dtype, int cos_dtype, void* stream) {
  Q3_REQUIRE(x_strides && y_strides, Q3_ERR_NULL);
  RopeGeom g{(int)B, (int)H, (int)S, (int)D, (int)D_rope, x_strides[0], x_strides[1], x_strides[2],
             y_strides[0], y_strides[1], y_strides[2], 0, cos_batch_stride, cos_seq_stride, (int)(D_rope / 2), 0};
  return launch_rope(x, cos, sin, y, g, dtype, cos_dtype, static_cast<hipStream_t>(stream));
}

int q3_mrope(const void* x, const void* cos3d, const void* sin3d, void* y, int64_t B, int64_t H, int64_t S, int64_t D,
             int64_t D_rope, const int64_t* section, const int64_t* x_strides, const int64_t* y_strides,
             const int64_t* cos_strides, int dtype, int cos_dtype, void* stream) {
  Q3_REQUIRE(section && x_strides && y_strides && cos_strides, Q3_ERR_NULL);
  RopeGeom g{(int)B, (int)H, (int)S, (int)D, (int)D_rope, x_strides[0], x_strides[1], x_strides[2],
             y_strides[0], y_strides[1], y_strides[2], cos_strides[0], cos_strides[1], cos_strides[2],
             (int)section[0], (int)section[1]};
  Q3_REQUIRE(section[0] + section[1] + section[2] == D_rope / 2, Q3_ERR_SHAPE);
  return launch_rope(x, cos3d, sin3d, y, g, dtype, cos_dtype, static_cast<hipStream_t>(stream));
}

int q3_qk_norm_rope(const void* q_in, const void* k_in, const void* v_in, void* q_out, void* k_out, void* v_out,
                    const void* q_weight, const void* k_weight, const int* positions, const float* inv_freq,
                    const int* dst_seq_offset, int64_t dst_seq_cap, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                    int64_t D, const int64_t* section, float eps, const int64_t* strides, int dtype, void* stream) {
  return qk_impl(q_in, k_in, v_in, q_out, k_out, v_out, q_weight, k_weight, positions, inv_freq, dst_seq_offset,
                 dst_seq_cap, B, S, Hq, Hkv, D, section, eps, strides, dtype, nullptr, 0, 0, 0, nullptr, stream);
}

int q3_qk_norm_rope_paged(const void* q_in, const void* k_in, const void* v_in, void* q_out, void* k_pages,
                          void* v_pages, const void* q_weight, const void* k_weight, const int* positions,
                          const float* inv_freq, const int* block_table, int64_t max_pages, int64_t page_rows,
                          int64_t num_pages, const int* kv_lens, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                          int64_t D, const int64_t* section, float eps, const int64_t* strides, int dtype,
                          int* status, void* stream) {
  Q3_REQUIRE(block_table && kv_lens, Q3_ERR_NULL);
  Q3_REQUIRE(max_pages >= 1 && num_pages >= 1 && page_rows >= 32 && page_rows % 32 == 0, Q3_ERR_SHAPE);
  Q3_REQUIRE(max_pages * page_rows < (1ll << 31) && num_pages < (1ll << 31), Q3_ERR_SHAPE);
  return qk_impl(q_in, k_in, v_in, q_out, k_pages, v_pages, q_weight, k_weight, positions, inv_freq, kv_lens,
                 max_pages * page_rows, B, S, Hq, Hkv, D, section, eps, strides, dtype, block_table, max_pages,
                 page_rows, num_pages, status, stream);
}

}  // extern "C"
