// Sparse-MoE kernels.
//
//  q3_moe_route     router probabilities -> top-k -> renormalise, one wave per
//                   token: fp32 softmax over the (bf16) logits, k rounds of a
//                   wave arg-max (larger probability wins, lower expert index
//                   among equals), weights = p / sum(p_selected) cast to bf16.
//  q3_moe_experts   dispatch + expert MLPs + combine for routed tokens:
//                     1. count      block per expert: #(token, slot) pairs
//                     2. scan       one block: expert offsets and the m-tile table
//                     3. scatter    block per expert: its pairs in ascending
//                                   token order (a block-wide ballot prefix sum)
//                     4. GEMM 1     grouped MFMA GEMM, gathered token rows x
//                                   gate/up of the pair's expert, SwiGLU epilogue
//                     5. GEMM 2     grouped MFMA GEMM x down, epilogue
//                                   bf16(bf16(y) * routing weight)
//                     6. combine    one wave per token: its k expert rows added
//                                   in ascending expert order with a bf16
//                                   rounding after each add (the order and
//                                   rounding of a per-expert bf16 index_add),
//                                   optionally plus a residual
//  q3_index_add     deterministic target[idx[i]] += src[i]: bucket the sources
//                   by target, then each target adds its sources in ascending
//                   source order in fp32 and rounds once.
#include <algorithm>

#include <climits>

#include "gemm_kernels.h"

using namespace q3;

namespace {

// Expert GEMM tiles: 256 rows x 256 weight rows (SwiGLU: 128 gate/up output
// columns), 8 waves, 64-wide K stages in 2 X and 3 W slots (the whole 160 KB of
// LDS). Every expert's weights stream from HBM exactly once per layer, so W is
// issued two stages ahead. Measured at T=4096, H=2048, I=768, E=128, top-8
// (random routing, 193 m-tiles): gate/up 274 us, down 184 us, against 312 and
// 182 us for 320-row tiles with 2 W slots (one m-tile per expert but 1.42x the
// time per tile wave); with 256 rows per expert, 232 and 156 against 328 and 183.
constexpr int kMoeBM = 256;
constexpr int kMoeBN = 256;
constexpr int kMoeNSTW = 3;

// ------------------------------------------------------------------ routing
// partials (split-K router, q3_moe_router): the logits are first summed from
// nsplit fp32 planes of (T, E), in plane order, rounded once to bf16 and
// written to `logits_out`; the routing then uses those bf16 values.
template <int MAXV>
__global__ __launch_bounds__(256) void moe_route_kernel(const bf16* __restrict__ logits, int* __restrict__ top_idx,
                                                        bf16* __restrict__ top_w, float* __restrict__ top_p,
                                                        int T, int E, int k, int norm,
                                                        const float* __restrict__ partials, int nsplit,
                                                        bf16* __restrict__ logits_out) {
  const int lane = threadIdx.x & 63;
  const int t = (int)(((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6);
  if (t >= T) return;
  const bf16* lr = logits + (int64_t)t * E;
  float v[MAXV];
  bool live[MAXV];
  float mx = -INFINITY;
  if (partials) {
    const int64_t plane = (int64_t)T * E;
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      const int e = lane + 64 * i;
      live[i] = e < E;
      float acc = 0.f;
      for (int z = 0; z < nsplit; ++z) acc += live[i] ? partials[z * plane + (int64_t)t * E + e] : 0.f;
      const bf16 b = f2bf(acc);
      if (live[i]) logits_out[(int64_t)t * E + e] = b;
      v[i] = live[i] ? bf2f(b) : -INFINITY;
    }
  } else {
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      const int e = lane + 64 * i;
      live[i] = e < E;
      v[i] = live[i] ? bf2f(lr[e]) : -INFINITY;
    }
  }
#pragma unroll
  for (int i = 0; i < MAXV; ++i) mx = fmaxf(mx, v[i]);
  mx = wave_max(mx);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    v[i] = live[i] ? expf(v[i] - mx) : 0.f;
    s += v[i];
  }
  s = wave_sum(s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) v[i] *= inv;
  // Top-k by threshold (the same k entries in the same order as k rounds of a
  // wave arg-max, without their shuffle chains). Probabilities are >= +0, so
  // they order as their bit patterns: thr = the k-th largest key, found by a
  // binary search over the bits with ballot counts. The entries above thr and
  // the lowest-index entries equal to it make the k; each then takes its place
  // (larger first, lower expert index among equals) by comparing itself with
  // the selected entries one at a time.
  uint32_t key[MAXV];
#pragma unroll
  for (int i = 0; i < MAXV; ++i) key[i] = __float_as_uint(v[i]);
  uint32_t thr = 0;
  for (int bit = 30; bit >= 0; --bit) {
    const uint32_t cand = thr | (1u << bit);
    int c = 0;
#pragma unroll
    for (int i = 0; i < MAXV; ++i) c += __builtin_popcountll(__ballot(live[i] && key[i] >= cand));
    if (c >= k) thr = cand;
  }
  int need = k;  // entries equal to thr that are taken, lowest index first
#pragma unroll
  for (int i = 0; i < MAXV; ++i) need -= __builtin_popcountll(__ballot(live[i] && key[i] > thr));
  bool sel[MAXV];
  int eq_before = 0;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const uint64_t eq = __ballot(live[i] && key[i] == thr);
    const int below = eq_before + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(eq >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)eq, 0u));
    sel[i] = live[i] && (key[i] > thr || (key[i] == thr && below < need));
    eq_before += __builtin_popcountll(eq);
  }
  int pos[MAXV];
#pragma unroll
  for (int i = 0; i < MAXV; ++i) pos[i] = 0;
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    uint64_t m = __ballot(sel[j]);
    while (m) {
      const int l = __builtin_ctzll(m);
      m &= m - 1;
      const uint32_t ky = (uint32_t)__builtin_amdgcn_readlane((int)key[j], l);
      const int ey = l + 64 * j;
#pragma unroll
      for (int i = 0; i < MAXV; ++i) pos[i] += (ky > key[i] || (ky == key[i] && ey < lane + 64 * i)) ? 1 : 0;
    }
  }
  // Renormalise: the sum runs over the selected values in selection order.
  float sel_sum = 0.f;
  for (int r = 0; r < k; ++r) {
    uint32_t vr = 0;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      const uint64_t m = __ballot(sel[j] && pos[j] == r);
      if (m) vr = (uint32_t)__builtin_amdgcn_readlane((int)key[j], __builtin_ctzll(m));
    }
    sel_sum += __uint_as_float(vr);
  }
#pragma unroll
  for (int i = 0; i < MAXV; ++i)
    if (sel[i]) {
      const int64_t o = (int64_t)t * k + pos[i];
      top_idx[o] = lane + 64 * i;
      top_w[o] = f2bf(norm ? v[i] / sel_sum : v[i]);
      if (top_p) top_p[o] = v[i];
    }
}

// ------------------------------------------------------------------ permute
// Workspace carve-out (all int32 unless noted):
//   hist[chunks][E], cstart[chunks][E], counts[E], offsets[E + 1],
//   tile_table[max_tiles], n_tiles[1],
//   sorted_token[P], sorted_w (bf16)[P], pos_of[P]   (P = T * k)
struct MoeWs {
  int* hist;    // (chunks, E) entries per chunk and expert
  int* cstart;  // (chunks, E) first row of the chunk's entries in each expert's block
  int* counts;
  int* offsets;
  int* tile_table;
  int* n_tiles;
  int* sorted_token;
  bf16* sorted_w;
  int* pos_of;
  bf16* act;     // (P, I)
  bf16* y_perm;  // (P, H)
};

constexpr int kMoeChunk = 64;  // tokens per dispatch chunk (one wave)

// Wave per 64-token chunk: number of (token, slot) entries of the chunk per
// expert (ids outside [0, E) are never dispatched).
__global__ __launch_bounds__(64) void moe_hist_kernel(const int* __restrict__ top_idx, int T, int k, int E,
                                                      int* __restrict__ hist) {
  extern __shared__ int s_cnt[];  // E counters
  const int c = blockIdx.x, lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) s_cnt[e] = 0;
  __syncthreads();
  const int t = c * kMoeChunk + lane;
  if (t < T)
    for (int s = 0; s < k; ++s) {
      const int e = top_idx[(int64_t)t * k + s];
      if (e >= 0 && e < E) atomicAdd(&s_cnt[e], 1);
    }
  __syncthreads();
  for (int e = lane; e < E; e += 64) hist[(int64_t)c * E + e] = s_cnt[e];
}

// Exclusive scan of a[0, n) in LDS by one wave (lane l takes a contiguous
// run of ceil(n / 64) entries); returns the total to every lane.
__device__ int wave_excl_scan(int* a, int n) {
  const int lane = threadIdx.x & 63;
  const int per = (n + 63) / 64, b0 = lane * per;
  int loc = 0;
  for (int i = 0; i < per; ++i)
    if (b0 + i < n) loc += a[b0 + i];
  int incl = loc;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  int run = incl - loc;
  for (int i = 0; i < per; ++i)
    if (b0 + i < n) {
      const int x = a[b0 + i];
      a[b0 + i] = run;
      run += x;
    }
  return __shfl(incl, 63, 64);
}

// One block of 1024 threads: per-expert counts and offsets (exclusive scan),
// each chunk's first position per expert, and the m-tile table of the grouped
// GEMMs (tiles of kMoeBM rows, expert-major). Thread (g, e) sums the chunk
// range g of expert e (G = 1024 / E ranges; independent loads), so the chunk
// prefix per expert is a short scan over the ranges; the two scans over the
// experts run on one wave each (with a block-wide scan over 1024 threads,
// ~40 barriers, the dispatch took 21.7 us at C4 against 18.7).
__global__ __launch_bounds__(1024) void moe_plan_kernel(const int* __restrict__ hist, int NC, int E,
                                                        int* __restrict__ counts, int* __restrict__ offsets,
                                                        int* __restrict__ cstart, int* __restrict__ tile_table,
                                                        int* __restrict__ n_tiles) {
  __shared__ int s_off[2048], s_til[2048], s_part[1024], s_tot[2];
  const int tid = threadIdx.x;
  const int G = E <= 1024 ? 1024 / E : 1;  // chunk ranges per expert
  // Partial sums (for E > 1024 one range per expert, thread strides over experts).
  for (int e0 = 0; e0 < E; e0 += 1024 / G) {
    const int e = e0 + tid % (1024 / G), g = tid / (1024 / G);
    const bool act = e < E && g < G;
    int sum = 0;
    if (act) {
      const int c0 = (int)((int64_t)g * NC / G), c1 = (int)((int64_t)(g + 1) * NC / G);
#pragma unroll 8
      for (int ci = c0; ci < c1; ++ci) sum += hist[(int64_t)ci * E + e];
    }
    if (G > 1) {
      if (act) s_part[g * E + e] = sum;
    } else if (act) {
      s_off[e] = sum;
    }
  }
  __syncthreads();
  if (G > 1) {
    for (int e = tid; e < E; e += 1024) {
      int run = 0;
      for (int g = 0; g < G; ++g) {
        const int v = s_part[g * E + e];
        s_part[g * E + e] = run;  // exclusive prefix over ranges
        run += v;
      }
      s_off[e] = run;
    }
    __syncthreads();
  }
  for (int e = tid; e < E; e += 1024) {
    counts[e] = s_off[e];
    s_til[e] = (s_off[e] + kMoeBM - 1) / kMoeBM;
  }
  __syncthreads();
  // The two scans over the experts, one wave each.
  if (tid < 64) {
    const int tot = wave_excl_scan(s_off, E);
    if (tid == 0) s_tot[0] = tot;
  } else if (tid < 128) {
    const int tot = wave_excl_scan(s_til, E);
    if (tid == 64) s_tot[1] = tot;
  }
  __syncthreads();
  const int rows = s_tot[0], tiles = s_tot[1];
  for (int e = tid; e < E; e += 1024) {
    const int off = s_off[e];
    offsets[e] = off;
    const int end = e + 1 < E ? s_off[e + 1] : rows;
    int tt = s_til[e];
    for (int m = off; m < end; m += kMoeBM) tile_table[tt++] = (e << 20) | m;
  }
  // Chunk starts: range g of expert e begins at off_e + (rows of ranges < g).
  for (int e0 = 0; e0 < E; e0 += 1024 / G) {
    const int e = e0 + tid % (1024 / G), g = tid / (1024 / G);
    if (e >= E || g >= G) continue;
    int run = s_off[e] + (G > 1 ? s_part[g * E + e] : 0);
    const int c0 = (int)((int64_t)g * NC / G), c1 = (int)((int64_t)(g + 1) * NC / G);
    for (int ci = c0; ci < c1; ++ci) {
      cstart[(int64_t)ci * E + e] = run;
      run += hist[(int64_t)ci * E + e];
    }
  }
  if (tid == 0) {
    offsets[E] = rows;
    *n_tiles = tiles;
  }
}

// Wave per chunk: every (token, slot) entry of an expert gets the next row of
// that expert's block, in (token, slot) order: the order of nonzero() on the
// (T, k) routing matrix. Lane l of every wave holds token l's k expert ids in
// registers and the chunk's histogram and start rows sit in LDS; the block's
// waves split the experts, and per expert present in the chunk one ballot per
// slot counts the entries of the lanes below.
constexpr int kPlaceWaves = 8;  // waves per chunk; wave w places experts e = w (mod 8)

template <int KMAX>
__global__ __launch_bounds__(kPlaceWaves * 64) void moe_place_kernel(const int* __restrict__ top_idx,
                                                       const bf16* __restrict__ top_w, int T, int k, int E,
                                                       const int* __restrict__ hist, const int* __restrict__ cstart,
                                                       int* __restrict__ sorted_token, bf16* __restrict__ sorted_w,
                                                       int* __restrict__ pos_of) {
  extern __shared__ int s_row[];  // [0, E): the chunk's counts, [E, 2E): its start rows
  const int c = blockIdx.x, lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int e = threadIdx.x; e < E; e += kPlaceWaves * 64) {
    s_row[e] = hist[(int64_t)c * E + e];
    s_row[E + e] = cstart[(int64_t)c * E + e];
  }
  const int t = c * kMoeChunk + lane;
  int ex[KMAX];
  bf16 wv[KMAX];
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    const bool ok = t < T && s < k;
    ex[s] = ok ? top_idx[(int64_t)t * k + s] : -1;
    wv[s] = ok ? top_w[(int64_t)t * k + s] : bf16{};
  }
  __syncthreads();
  int dst[KMAX];  // row of each slot's entry (-1: not dispatched)
#pragma unroll
  for (int s = 0; s < KMAX; ++s) dst[s] = -1;
  for (int e = wave; e < E; e += kPlaceWaves) {
    if (s_row[e] == 0) continue;  // uniform
    // Entries of lower lanes (earlier tokens) with expert e: per slot, the
    // ballot's set bits below this lane.
    int below = 0;
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
      const uint64_t m = __ballot(ex[s] == e);
      below += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    }
    int pos = s_row[E + e] + below;
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
      if (ex[s] == e) dst[s] = pos++;
  }
  // One store per slot and array, all lanes together (a slot's row was set
  // by the wave that owns its expert).
#pragma unroll
  for (int s = 0; s < KMAX; ++s)
    if (dst[s] >= 0) {
      sorted_token[dst[s]] = t;
      sorted_w[dst[s]] = wv[s];
      pos_of[(int64_t)t * k + s] = dst[s];
    }
}

// One wave per token: add its k expert rows in ascending expert order.
template <int VPL>
__global__ __launch_bounds__(256) void moe_combine_kernel(const int* __restrict__ top_idx,
                                                          const int* __restrict__ pos_of,
                                                          const bf16* __restrict__ y_perm,
                                                          const bf16* __restrict__ residual, bf16* __restrict__ out,
                                                          int T, int k, int H, int E) {
  const int lane = threadIdx.x & 63;
  const int t = (int)(((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6);
  if (t >= T) return;
  int ex[32], ps[32];
  int kk = 0;  // slots with a valid expert id (others were never dispatched)
  for (int s = 0; s < k; ++s) {
    const int e = top_idx[(int64_t)t * k + s];
    const int pp = pos_of[(int64_t)t * k + s];
    if (e < 0 || e >= E || pp < 0 || pp >= T * k) continue;
    ex[kk] = e;
    ps[kk] = pp;
    ++kk;
  }
  k = kk;
  // insertion sort by expert id
  for (int i = 1; i < k; ++i) {
    const int e = ex[i], p = ps[i];
    int j = i - 1;
    while (j >= 0 && ex[j] > e) {
      ex[j + 1] = ex[j];
      ps[j + 1] = ps[j];
      --j;
    }
    ex[j + 1] = e;
    ps[j + 1] = p;
  }
  // lane owns vectors lane + 64 * i of 8 bf16
  const int nvec = H / 8;
  for (int i = 0; i < VPL; ++i) {
    const int vi = lane + 64 * i;
    if (vi >= nvec) break;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < k; ++s) {
      const bf16x8 yv = reinterpret_cast<const bf16x8*>(y_perm + (int64_t)ps[s] * H)[vi];
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] = bf2f(f2bf(acc[q] + bf2f(yv[q])));
    }
    bf16x8 o;
    if (residual) {
      const bf16x8 rv = reinterpret_cast<const bf16x8*>(residual + (int64_t)t * H)[vi];
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] = f2bf(acc[q] + bf2f(rv[q]));
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] = f2bf(acc[q]);
    }
    reinterpret_cast<bf16x8*>(out + (int64_t)t * H)[vi] = o;
  }
}

// Combine, wide form (k <= 8, H = 8 * blockDim.x): one block per token,
// thread j owns columns [8j, 8j + 8). The token's valid slots are ranked by
// expert id in registers (ties by slot), every thread issues its k row loads
// at once, then adds them in rank order with the same per-add bf16 rounding.
template <int KMAX>
__global__ __launch_bounds__(1024) void moe_combine_wide_kernel(const int* __restrict__ top_idx,
                                                                const int* __restrict__ pos_of,
                                                                const bf16* __restrict__ y_perm,
                                                                const bf16* __restrict__ residual,
                                                                bf16* __restrict__ out, int T, int k, int H, int E) {
  const int t = blockIdx.x;
  const int j = threadIdx.x;
  int e[KMAX], p[KMAX];
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    int ee = INT_MAX, pp = -1;
    if (s < k) {
      ee = top_idx[(int64_t)t * k + s];
      pp = pos_of[(int64_t)t * k + s];
      if (ee < 0 || ee >= E || pp < 0 || pp >= T * k) {  // never dispatched
        ee = INT_MAX;
        pp = -1;
      }
    }
    e[s] = ee;
    p[s] = pp;
  }
  // rank[s]: slots before s in (expert, slot) order; invalid slots rank last
  int ps[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) ps[r] = -1;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    int rank = 0;
#pragma unroll
    for (int q = 0; q < KMAX; ++q) rank += (e[q] < e[s]) || (e[q] == e[s] && q < s);
#pragma unroll
    for (int r = 0; r < KMAX; ++r)
      if (rank == r) ps[r] = p[s];
  }
  bf16x8 yv[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r)
    yv[r] = ps[r] >= 0 ? reinterpret_cast<const bf16x8*>(y_perm + (int64_t)ps[r] * H)[j] : bf16x8{};
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < KMAX; ++r)
    if (ps[r] >= 0)
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] = bf2f(f2bf(acc[q] + bf2f(yv[r][q])));
  bf16x8 o;
  if (residual) {
    const bf16x8 rv = reinterpret_cast<const bf16x8*>(residual + (int64_t)t * H)[j];
#pragma unroll
    for (int q = 0; q < 8; ++q) o[q] = f2bf(acc[q] + bf2f(rv[q]));
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) o[q] = f2bf(acc[q]);
  }
  reinterpret_cast<bf16x8*>(out + (int64_t)t * H)[j] = o;
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

int64_t moe_ws_layout(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, MoeWs* ws, char* base) {
  const int64_t P = T * k;
  const int64_t max_tiles = q3_cdiv(P, kMoeBM) + E;
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  MoeWs w{};
  const int64_t NC = q3_cdiv(T, kMoeChunk);
  w.hist = reinterpret_cast<int*>(take(NC * E * 4));
  w.cstart = reinterpret_cast<int*>(take(NC * E * 4));
  w.counts = reinterpret_cast<int*>(take(E * 4));
  w.offsets = reinterpret_cast<int*>(take((E + 1) * 4));
  w.tile_table = reinterpret_cast<int*>(take(max_tiles * 4));
  w.n_tiles = reinterpret_cast<int*>(take(4));
  w.sorted_token = reinterpret_cast<int*>(take(P * 4));
  w.sorted_w = reinterpret_cast<bf16*>(take(P * 2));
  w.pos_of = reinterpret_cast<int*>(take(P * 4));
  w.act = reinterpret_cast<bf16*>(take(P * I * 2));
  w.y_perm = reinterpret_cast<bf16*>(take(P * H * 2));
  if (ws) *ws = w;
  return off;
}

// Workspace of the dispatch alone (q3_moe_permute): the per-chunk tables,
// counts and the m-tile table; the sorted list, weights and positions go to
// the caller's buffers.
int64_t moe_permute_ws_layout(int64_t T, int64_t E, int64_t k, MoeWs* ws, char* base) {
  const int64_t P = T * k;
  const int64_t max_tiles = q3_cdiv(P, kMoeBM) + E;
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  MoeWs w{};
  const int64_t NC = q3_cdiv(T, kMoeChunk);
  w.hist = reinterpret_cast<int*>(take(NC * E * 4));
  w.cstart = reinterpret_cast<int*>(take(NC * E * 4));
  w.counts = reinterpret_cast<int*>(take(E * 4));
  w.tile_table = reinterpret_cast<int*>(take(max_tiles * 4));
  w.n_tiles = reinterpret_cast<int*>(take(4));
  if (ws) *ws = w;
  return off;
}

// Dispatch: per-expert counts and offsets, the m-tile table, and every
// (token, slot) entry's row in expert-major, (token, slot)-ascending order
// (the order of the reference's per-expert nonzero(), modules/moe.py:75).
int moe_dispatch(const int* top_idx, const bf16* top_w, int64_t T, int64_t k, int64_t E, const MoeWs& w,
                 hipStream_t st) {
  const int NC = (int)q3_cdiv(T, kMoeChunk);
  hipLaunchKernelGGL(moe_hist_kernel, dim3((unsigned)NC), dim3(64), E * sizeof(int), st, top_idx, (int)T, (int)k,
                     (int)E, w.hist);
  hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(1024), 0, st, w.hist, NC, (int)E, w.counts, w.offsets, w.cstart,
                     w.tile_table, w.n_tiles);
  const dim3 place_blk(kPlaceWaves * 64);
  const size_t place_lds = 2 * E * sizeof(int);
  if (k <= 8)
    hipLaunchKernelGGL(moe_place_kernel<8>, dim3((unsigned)NC), place_blk, place_lds, st, top_idx, top_w, (int)T,
                       (int)k, (int)E, w.hist, w.cstart, w.sorted_token, w.sorted_w, w.pos_of);
  else
    hipLaunchKernelGGL(moe_place_kernel<32>, dim3((unsigned)NC), place_blk, place_lds, st, top_idx, top_w, (int)T,
                       (int)k, (int)E, w.hist, w.cstart, w.sorted_token, w.sorted_w, w.pos_of);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

// ------------------------------------------------------------------ index_add
__global__ void fill_int_kernel(int* p, int64_t n, int v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

__global__ void ia_count_kernel(const int64_t* __restrict__ idx, int64_t ns, int64_t nt, int* __restrict__ counts,
                                int* __restrict__ bad) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < ns; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = idx[i];
    if (t < 0 || t >= nt) {
      atomicOr(bad, 1);
      continue;
    }
    atomicAdd(&counts[t], 1);
  }
}

__global__ void ia_scan_kernel(const int* __restrict__ counts, int64_t nt, int* __restrict__ starts) {
  // Single block, 256 threads: chunked scan.
  __shared__ int s[256];
  __shared__ int carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int64_t c0 = 0; c0 < nt; c0 += 256) {
    const int64_t i = c0 + threadIdx.x;
    const int v = i < nt ? counts[i] : 0;
    s[threadIdx.x] = v;
    __syncthreads();
    for (int o = 1; o < 256; o <<= 1) {
      const int a = (threadIdx.x >= (unsigned)o) ? s[threadIdx.x - o] : 0;
      __syncthreads();
      s[threadIdx.x] += a;
      __syncthreads();
    }
    if (i < nt) starts[i] = carry + s[threadIdx.x] - v;
    __syncthreads();
    if (threadIdx.x == 255) carry += s[255];
    __syncthreads();
  }
  if (threadIdx.x == 0) starts[nt] = carry;
}

__global__ void ia_scatter_kernel(const int64_t* __restrict__ idx, int64_t ns, int64_t nt,
                                  const int* __restrict__ starts, int* __restrict__ fill, int* __restrict__ bucket) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < ns; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = idx[i];
    if (t < 0 || t >= nt) continue;
    const int slot = atomicAdd(&fill[t], 1);
    bucket[starts[t] + slot] = (int)i;
  }
}

// One wave per target row. Its sources are added in ascending source index,
// in fp32 starting from the target value, with one rounding at the end (the
// order and precision of torch's CPU index_add_). The bucket (unordered after
// the atomic scatter) is rank-sorted in LDS when it holds <= kIaLds entries;
// longer buckets take the next-smallest index by repeated wave minima.
constexpr int kIaLds = 1024;

template <typename T>
__global__ __launch_bounds__(256) void ia_accumulate_kernel(T* __restrict__ target, const T* __restrict__ src,
                                                            const int* __restrict__ starts,
                                                            const int* __restrict__ bucket, int64_t nt, int64_t D) {
  __shared__ int s_raw[4][kIaLds];
  __shared__ int s_sorted[4][kIaLds];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t t = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (t >= nt) return;
  const int b0 = starts[t], c = starts[t + 1] - b0;
  if (c == 0) return;
  T* tr = target + t * D;
  if (c <= kIaLds) {
    for (int j = lane; j < c; j += 64) s_raw[wave][j] = bucket[b0 + j];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    for (int j = lane; j < c; j += 64) {
      const int v = s_raw[wave][j];
      int rank = 0;
      for (int q = 0; q < c; ++q) rank += s_raw[wave][q] < v;  // source indices are distinct
      s_sorted[wave][rank] = v;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    for (int64_t d = lane; d < D; d += 64) {
      float acc = to_f<T>(tr[d]);
      for (int n = 0; n < c; ++n) acc += to_f<T>(src[(int64_t)s_sorted[wave][n] * D + d]);
      tr[d] = from_f<T>(acc);
    }
    return;
  }
  for (int64_t d0 = 0; d0 < D; d0 += 64) {
    const int64_t d = d0 + lane;
    float acc = d < D ? to_f<T>(tr[d]) : 0.f;
    int prev = -1;
    for (int n = 0; n < c; ++n) {
      int best = 0x7fffffff;
      for (int j = lane; j < c; j += 64) {
        const int v = bucket[b0 + j];
        if (v > prev && v < best) best = v;
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) best = min(best, __shfl_xor(best, o, 64));
      prev = best;
      if (d < D) acc += to_f<T>(src[(int64_t)best * D + d]);
    }
    if (d < D) tr[d] = from_f<T>(acc);
  }
}

template <typename T>
int index_add_t(void* target, const void* src, const int64_t* idx, int64_t ns, int64_t nt, int64_t D, char* ws,
                int* status, hipStream_t st) {
  int* counts = reinterpret_cast<int*>(ws);
  int* fill = counts + nt;
  int* starts = fill + nt;
  int* bucket = starts + nt + 1;
  int* bad = status ? status : bucket + ns;  // the caller's status word is sticky: never cleared here
  const unsigned fb = (unsigned)std::min<int64_t>(q3_cdiv(2 * nt + 1, 256), 1024);
  hipLaunchKernelGGL(fill_int_kernel, dim3(fb), dim3(256), 0, st, counts, 2 * nt, 0);
  if (!status) hipLaunchKernelGGL(fill_int_kernel, dim3(1), dim3(64), 0, st, bad, (int64_t)1, 0);
  const unsigned sb = (unsigned)std::max<int64_t>(1, std::min<int64_t>(q3_cdiv(ns, 256), 1024));
  hipLaunchKernelGGL(ia_count_kernel, dim3(sb), dim3(256), 0, st, idx, ns, nt, counts, bad);
  hipLaunchKernelGGL(ia_scan_kernel, dim3(1), dim3(256), 0, st, counts, nt, starts);
  hipLaunchKernelGGL(ia_scatter_kernel, dim3(sb), dim3(256), 0, st, idx, ns, nt, starts, fill, bucket);
  hipLaunchKernelGGL(ia_accumulate_kernel<T>, dim3((unsigned)q3_cdiv(nt, 4)), dim3(256), 0, st,
                     static_cast<T*>(target), static_cast<const T*>(src), starts, bucket, nt, D);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

}  // namespace

namespace {

// Splits over K of the router GEMM (q3_moe_router): enough (T/128 x E/128)
// tiles x splits to give every CU one (at most 256), each split a multiple of
// 64 columns dividing H (a 2048-wide router at 4096 tokens: 32 tiles x 8
// splits of 256).
int router_splits(int64_t T, int64_t H, int64_t E) {
  const int64_t tiles = q3_cdiv(T, 128) * q3_cdiv(E, 128);
  int best = 1;
  for (int s = 2; s <= 64; ++s)
    if (tiles * s <= 256 && H % s == 0 && (H / s) % 64 == 0) best = s;
  return best;
}

int launch_route(const bf16* lg, int* top_idx, bf16* tw, float* top_p, int64_t T, int64_t E, int64_t k, int norm,
                 const float* partials, int ns, bf16* lg_out, hipStream_t st) {
  const unsigned blocks = (unsigned)q3_cdiv(T, 4);
  if (E <= 64)
    hipLaunchKernelGGL(moe_route_kernel<1>, dim3(blocks), dim3(256), 0, st, lg, top_idx, tw, top_p, (int)T, (int)E,
                       (int)k, norm, partials, ns, lg_out);
  else if (E <= 128)
    hipLaunchKernelGGL(moe_route_kernel<2>, dim3(blocks), dim3(256), 0, st, lg, top_idx, tw, top_p, (int)T, (int)E,
                       (int)k, norm, partials, ns, lg_out);
  else if (E <= 256)
    hipLaunchKernelGGL(moe_route_kernel<4>, dim3(blocks), dim3(256), 0, st, lg, top_idx, tw, top_p, (int)T, (int)E,
                       (int)k, norm, partials, ns, lg_out);
  else
    hipLaunchKernelGGL(moe_route_kernel<8>, dim3(blocks), dim3(256), 0, st, lg, top_idx, tw, top_p, (int)T, (int)E,
                       (int)k, norm, partials, ns, lg_out);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

}  // namespace

extern "C" {

// logits (T, E) bf16 -> top_idx (T, k) int32, top_w (T, k) bf16 (renormalised
// when norm != 0), top_p (T, k) fp32 selected probabilities (optional).
int q3_moe_route(const void* logits, int* top_idx, void* top_w, float* top_p, int64_t T, int64_t E, int64_t k,
                 int norm, void* stream) {
  Q3_REQUIRE(logits && top_idx && top_w, Q3_ERR_NULL);
  Q3_REQUIRE(T >= 0 && E >= 1 && k >= 1 && k <= E, Q3_ERR_SHAPE);
  Q3_REQUIRE(E <= 512 && k <= 32, Q3_ERR_UNSUPPORTED);
  if (T == 0) return Q3_OK;
  return launch_route(static_cast<const bf16*>(logits), top_idx, static_cast<bf16*>(top_w), top_p, T, E, k, norm,
                      nullptr, 0, nullptr, static_cast<hipStream_t>(stream));
}

int64_t q3_moe_router_workspace_bytes(int64_t T, int64_t H, int64_t E) {
  if (T <= 0 || H <= 0 || E <= 0) return 0;
  return (int64_t)router_splits(T, H, E) * T * E * 4;
}

int q3_moe_router(const void* x, const void* gate_w, void* logits, int* top_idx, void* top_w, float* top_p,
                  int64_t T, int64_t H, int64_t E, int64_t k, int norm, void* workspace, int64_t workspace_bytes,
                  void* stream) {
  Q3_REQUIRE(x && gate_w && logits && top_idx && top_w, Q3_ERR_NULL);
  Q3_REQUIRE(T >= 0 && H >= 1 && E >= 1 && k >= 1 && k <= E, Q3_ERR_SHAPE);
  Q3_REQUIRE(E <= 512 && k <= 32, Q3_ERR_UNSUPPORTED);
  Q3_REQUIRE(H % 8 == 0 && q3_aligned(x, 16) && q3_aligned(gate_w, 16), Q3_ERR_ALIGN);
  Q3_REQUIRE(T * H * 2 < 0x7fffffffLL && E * H * 2 < 0x7fffffffLL, Q3_ERR_UNSUPPORTED);
  if (T == 0) return Q3_OK;
  const int ns = router_splits(T, H, E);
  const int64_t ks = H / ns;
  Q3_REQUIRE(workspace != nullptr && workspace_bytes >= (int64_t)ns * T * E * 4, Q3_ERR_WORKSPACE);
  Q3_REQUIRE(q3_aligned(workspace, 16), Q3_ERR_ALIGN);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Split z: X and W columns [z ks, (z + 1) ks) -> fp32 plane z of (T, E).
  GemmParams p{};
  p.X = static_cast<const bf16*>(x);
  p.W = static_cast<const bf16*>(gate_w);
  p.C = static_cast<bf16*>(workspace);
  p.M = (int)T;
  p.N = (int)E;
  p.K = (int)ks;
  p.ldx = H;
  p.ldw = H;
  p.ldc = E;
  p.bsX = ks;
  p.bsW = ks;
  p.bsC = T * E;
  p.group_m = 8;
  p.seg.n = 1;
  p.seg.w[0] = p.W;
  const int64_t tiles = q3_cdiv(T, 128) * q3_cdiv(E, 128);
  hipLaunchKernelGGL((gemm_bf16_dma_kernel<128, 128, 2, 2, kEpiStoreF32, false, 4, 64, 5>),
                     dim3((unsigned)tiles, 1, (unsigned)ns), dim3(256), 0, st, p);
  Q3_LAUNCH_CHECK();
  return launch_route(static_cast<const bf16*>(logits), top_idx, static_cast<bf16*>(top_w), top_p, T, E, k, norm,
                      static_cast<const float*>(workspace), ns, static_cast<bf16*>(logits), st);
}

int64_t q3_moe_experts_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k) {
  if (T <= 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  return moe_ws_layout(T, H, I, E, k, nullptr, nullptr);
}

// x (T, H) bf16; gate_up (E, 2I, H); down (E, H, I); top_idx (T, k) int32;
// top_w (T, k) bf16; out (T, H) bf16 = sum over the token's experts of
// w * down(swiglu(gate_up x)) (+ residual (T, H) when given).
int q3_moe_experts(const void* x, const void* gate_up, const void* down, const int* top_idx, const void* top_w,
                   const void* residual, void* out, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                   void* workspace, int64_t workspace_bytes, void* stream) {
  Q3_REQUIRE(x && gate_up && down && top_idx && top_w && out, Q3_ERR_NULL);
  Q3_REQUIRE(T >= 0 && H >= 8 && I >= 8 && E >= 1 && k >= 1 && k <= E, Q3_ERR_SHAPE);
  Q3_REQUIRE(H % 8 == 0 && I % 8 == 0 && k <= 32 && E < 2048 && T * k < (1 << 20), Q3_ERR_UNSUPPORTED);
  Q3_REQUIRE(q3_aligned(x, 16) && q3_aligned(gate_up, 16) && q3_aligned(down, 16) && q3_aligned(out, 16) &&
                 (!residual || q3_aligned(residual, 16)),
             Q3_ERR_ALIGN);
  if (T == 0) return Q3_OK;
  Q3_REQUIRE(workspace && workspace_bytes >= q3_moe_experts_workspace_bytes(T, H, I, E, k), Q3_ERR_WORKSPACE);
  hipStream_t st = static_cast<hipStream_t>(stream);
  MoeWs w{};
  moe_ws_layout(T, H, I, E, k, &w, static_cast<char*>(workspace));
  const int64_t P = T * k;
  const int64_t max_tiles = q3_cdiv(P, kMoeBM) + E;
  {
    const int rc = moe_dispatch(top_idx, static_cast<const bf16*>(top_w), T, k, E, w, st);
    if (rc != Q3_OK) return rc;
  }

  // GEMM 1: act[pos] = swiglu(x[token(pos)] . gate_up[e]^T)
  {
    GemmParams p{};
    p.X = static_cast<const bf16*>(x);
    p.W = static_cast<const bf16*>(gate_up);           // gate rows [0, I)
    p.W2 = static_cast<const bf16*>(gate_up) + I * H;  // up rows [I, 2I)
    p.C = w.act;
    p.M = (int)P;
    p.N = (int)I;
    p.K = (int)H;
    p.ldx = H;
    p.ldw = H;
    p.ldc = I;
    p.gather = w.sorted_token;
    p.M_src = (int)T;
    p.tile_table = w.tile_table;
    p.group_end = w.offsets + 1;
    p.n_tiles_total = w.n_tiles;
    p.expert_stride_w = 2 * I * H;
    const int64_t ntn = q3_cdiv(I, kMoeBN / 2);
    // Grid: a multiple of 8 (the kernel deals the valid tiles out per XCD).
    hipLaunchKernelGGL((gemm_bf16_dma_kernel<kMoeBM, kMoeBN, 2, 4, kEpiSwiGLU, true, 2, 64, kMoeNSTW>),
                       dim3((unsigned)(q3_cdiv(max_tiles * ntn, 8) * 8)),
                       dim3(512), 0, st, p);
    Q3_LAUNCH_CHECK();
  }
  // GEMM 2: y_perm[pos] = bf16(bf16(act[pos] . down[e]^T) * w[pos])
  {
    GemmParams p{};
    p.X = w.act;
    p.W = static_cast<const bf16*>(down);
    p.C = w.y_perm;
    p.rowscale = w.sorted_w;
    p.M = (int)P;
    p.N = (int)H;
    p.K = (int)I;
    p.ldx = I;
    p.ldw = I;
    p.ldc = H;
    p.gather = nullptr;
    p.tile_table = w.tile_table;
    p.group_end = w.offsets + 1;
    p.n_tiles_total = w.n_tiles;
    p.expert_stride_w = H * I;
    const int64_t ntn = q3_cdiv(H, kMoeBN);
    hipLaunchKernelGGL((gemm_bf16_dma_kernel<kMoeBM, kMoeBN, 2, 4, kEpiRowScale, true, 2, 64, kMoeNSTW>),
                       dim3((unsigned)(q3_cdiv(max_tiles * ntn, 8) * 8)), dim3(512), 0, st, p);
    Q3_LAUNCH_CHECK();
  }
  const int vpl = (int)q3_cdiv(H / 8, 64);
  const unsigned cb = (unsigned)q3_cdiv(T, 4);
  const bf16* res = static_cast<const bf16*>(residual);
  bf16* o = static_cast<bf16*>(out);
  if (k <= 8 && H % 8 == 0 && H / 8 <= 1024) {
    hipLaunchKernelGGL(moe_combine_wide_kernel<8>, dim3((unsigned)T), dim3((unsigned)(H / 8)), 0, st, top_idx,
                       w.pos_of, w.y_perm, res, o, (int)T, (int)k, (int)H, (int)E);
  } else if (vpl <= 4)
    hipLaunchKernelGGL(moe_combine_kernel<4>, dim3(cb), dim3(256), 0, st, top_idx, w.pos_of, w.y_perm, res, o, (int)T,
                       (int)k, (int)H, (int)E);
  else if (vpl <= 8)
    hipLaunchKernelGGL(moe_combine_kernel<8>, dim3(cb), dim3(256), 0, st, top_idx, w.pos_of, w.y_perm, res, o, (int)T,
                       (int)k, (int)H, (int)E);
  else
    hipLaunchKernelGGL(moe_combine_kernel<64>, dim3(cb), dim3(256), 0, st, top_idx, w.pos_of, w.y_perm, res, o,
                       (int)T, (int)k, (int)H, (int)E);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

int64_t q3_moe_permute_workspace_bytes(int64_t T, int64_t E, int64_t k) {
  if (T <= 0 || E <= 0 || k <= 0) return 0;
  return moe_permute_ws_layout(T, E, k, nullptr, nullptr);
}

// The dispatch of q3_moe_experts on its own: offsets (E + 1) int32,
// sorted_token / sorted_w (T * k) (int32 / bf16) and pos_of (T, k) int32.
int q3_moe_permute(const int* top_idx, const void* top_w, int* offsets, int* sorted_token, void* sorted_w,
                   int* pos_of, int64_t T, int64_t E, int64_t k, void* workspace, int64_t workspace_bytes,
                   void* stream) {
  Q3_REQUIRE(top_idx && top_w && offsets && sorted_token && sorted_w && pos_of, Q3_ERR_NULL);
  Q3_REQUIRE(T >= 0 && E >= 1 && k >= 1 && k <= E, Q3_ERR_SHAPE);
  Q3_REQUIRE(k <= 32 && E < 2048 && T * k < (1 << 20), Q3_ERR_UNSUPPORTED);
  if (T == 0) return Q3_OK;
  Q3_REQUIRE(workspace && workspace_bytes >= q3_moe_permute_workspace_bytes(T, E, k), Q3_ERR_WORKSPACE);
  MoeWs w{};
  moe_permute_ws_layout(T, E, k, &w, static_cast<char*>(workspace));
  w.offsets = offsets;
  w.sorted_token = sorted_token;
  w.sorted_w = static_cast<bf16*>(sorted_w);
  w.pos_of = pos_of;
  return moe_dispatch(top_idx, static_cast<const bf16*>(top_w), T, k, E, w, static_cast<hipStream_t>(stream));
}

int64_t q3_index_add_workspace_bytes(int64_t n_src, int64_t n_target) {
  if (n_src < 0 || n_target < 0) return 0;
  return (3 * n_target + 1 + n_src + 1) * (int64_t)sizeof(int);
}

// target (n_target, D) += rows of src (n_src, D) at idx (n_src) int64, in place.
// Source rows whose index is outside [0, n_target) are skipped, and bit 0 of
// *status (a device int, when given) is set: the check costs the host nothing.
int q3_index_add(void* target, const void* src, const int64_t* idx, int64_t n_src, int64_t n_target, int64_t D,
                 int dtype, void* workspace, int64_t workspace_bytes, int* status, void* stream) {
  Q3_REQUIRE(target && (src || n_src == 0) && (idx || n_src == 0), Q3_ERR_NULL);
  Q3_REQUIRE(n_src >= 0 && n_target >= 0 && D >= 0, Q3_ERR_SHAPE);
  Q3_REQUIRE(n_src < (1ll << 31) && n_target < (1ll << 31), Q3_ERR_UNSUPPORTED);
  if (n_src == 0 || n_target == 0 || D == 0) return Q3_OK;
  Q3_REQUIRE(workspace && workspace_bytes >= q3_index_add_workspace_bytes(n_src, n_target), Q3_ERR_WORKSPACE);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (dtype == Q3_BF16) return index_add_t<bf16>(target, src, idx, n_src, n_target, D, ws, status, st);
  if (dtype == Q3_F32) return index_add_t<float>(target, src, idx, n_src, n_target, D, ws, status, st);
  return Q3_ERR_DTYPE;
}

}  // extern "C"
