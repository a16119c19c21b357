// Flash attention on gfx950 MFMA, bf16 in / fp32 softmax and accumulation.
//
// Prefill (q3_flash_attention): one block = 4 waves; each wave owns 32 query
// rows of one head. With GQA the 4 waves of a block are (up to) 4 query heads
// of the same KV head over the same 32 queries, so one K/V tile in LDS feeds all
// of them and all waves share one causal extent.
//
// Per 64-key tile and wave:
//   S^T (64 keys x 32 q) = K (64 x D) * Q^T (D x 32)   A = K from LDS, B = Q in registers
//   online softmax per query: a query is a lane column, so its statistics are
//   lane-local apart from one exchange between lanes l and l ^ 32
//   O^T (D x 32 q) += V^T (D x 64) * P^T (64 x 32)       A = V^T from LDS, B = P^T
// P^T is used straight from the S^T accumulators: register r of lane l holds key
// 8*(r/4) + 4*(l/32) + r%4, which, read as the B operand's k index 8*(l/32) + t
// (t = r), is a fixed key permutation; the V^T fragment reads use the same one.
// The O^T accumulators are per-lane queries, so the softmax rescale is local.
//
// Decode (q3_decode_attention): stream-K over 32-key units of all (sequence,
// KV head) pairs, one wave-private DMA ring per wave; the MFMA query columns
// are the GQA group's heads (see the decode section below).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "gemm_tile.h"

#include "q3_common.h"

namespace {

constexpr int kKT = 64;      // keys per tile
constexpr int kRowK = 128;   // LDS K-tile row length (elements)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

struct AttnParams {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  bf16* o;
  float* lse;
  int B, Hq, Hkv, Sq, Sk;
  int64_t qb, qh, qs, kb, kh, ks, vb, vh, vs, ob, oh, os;
  float scale_log2;
  int causal;
  int groups;
  // decode
  const int* kv_lens;
  int len_add;      // decode: sequence b attends to kv_lens[b] + len_add cache rows
  // prefill into a KV cache: sequence b's query i is token q_off[b] + i; it
  // sees keys [0, q_off[b] + i] (causal) and the sequence has q_off[b] + Sq
  // keys (clamped to Sk). Null: offset 0, Sk keys.
  const int* q_off;
  // packed variable-length sequences (vision tower): sequence b is rows
  // [cu_seqlens[b], cu_seqlens[b + 1]) of one packed (H, total, D) tensor for
  // q, k, v and o alike (the batch strides are unused); Sq = Sk = max length.
  const int* cu_seqlens;
  int* lens_inc;    // decode: if set, lens_inc[b] += 1 once the step has read the lengths
  int* dec_hdr;     // decode workspace header: unit prefix over sequences (B + 1 ints)
  int dec_waves;    // decode: waves in the main kernel's grid
  float* partial;  // decode workspace
  // Paged KV cache (decode): cache row r of sequence b is row r % page_rows of
  // page block_table[b * max_pages + r / page_rows] (page_rows a multiple of the
  // 32-key unit); kb / vb are then the page strides. Null: one contiguous cache
  // per sequence. A page id outside [0, num_pages) reads as zero rows and sets
  // bit 1 of *status (when given).
  const int* block_table;
  int max_pages, page_rows, num_pages;
  int* status;
  // Prefill with the q prologue fused (pipelined kernel, D a multiple of 32):
  // q holds the projection output; each query row is RMS-normalised (weight
  // qn_w, eps qn_eps) and rotated by the row of rope_tab for token b * Sq + i
  // (D fp32: cos of the D/2 angles, then their sin) before use. Null: q is used
  // as given.
  const bf16* qn_w;
  const float* rope_tab;
  float qn_eps;
};

// ----------------------------------------------------------------- prefill
// Prefill kernel, sized for two blocks (8 waves) per CU:
//  * K tiles go global -> LDS with buffer_load ... lds (no staging
//    registers); rows are 128 elements (256 B) apart whatever D is, and row
//    r's 16-byte chunk c sits at slot c ^ (r & 15). Chunks at or past D load
//    as zeros (out-of-range buffer offsets), which pads D to the MFMA K step.
//  * V tiles are staged through registers and written transposed: V^T row d
//    holds the tile's 64 keys as 8 chunks of 16 bytes, chunk 2j + h holding
//    the 4-key units 4j + h and 4j + 2 + h (the two units one lane feeds to a
//    PV MFMA), at slot chunk ^ ((d >> 1) & 7). One ds_read_b128 per fragment,
//    conflict-free for 16 consecutive rows.
//  * The running max is raised only when a tile's max exceeds it by more than
//    kRescale (log2 units), so the O rescale almost never runs; P stays below
//    2^kRescale and O / l is unchanged.
//  * The row max is exchanged between the two lane halves that share a query
//    with v_permlane32_swap; the row sums stay per half until the end.
namespace fwd {
constexpr float kRescale = 8.0f;

__device__ __forceinline__ int k_off(int r, int c) { return r * kRowK + ((c ^ (r & 15)) << 3); }
__device__ __forceinline__ int vt_off(int d, int chunk) { return d * kKT + ((chunk ^ ((d >> 1) & 7)) << 3); }

__device__ __forceinline__ float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
}  // namespace fwd

template <int D, int WH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void flash_fwd_kernel(
    const AttnParams p) {
  using namespace fwd;
  static_assert(D % 8 == 0 && D <= kRowK, "head_dim");
  constexpr int KSTEPS = (D + 15) / 16;  // MFMA K steps over the (zero-padded) head dim
  constexpr int OT = (D + 31) / 32;      // 32-row output tiles of O^T
  constexpr int VCH = D / 8;             // 16-byte chunks per V row
  constexpr int WQ = 4 / WH;
  constexpr int QB = WQ * 32;
  __shared__ __attribute__((aligned(1024))) bf16 sK[2][kKT * kRowK];
  __shared__ __attribute__((aligned(1024))) bf16 sV[2][OT * 32 * kKT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wh = wave % WH;
  const int wq = wave / WH;
  const int l32 = lane & 31;
  const int h = lane >> 5;

  // Blocks are dispatched x-fastest: heads vary fastest and query tiles go
  // heaviest-first (causal) in the slow dimension.
  const int n_qt = (p.Sq + QB - 1) / QB;
  const int qt = p.causal ? (n_qt - 1 - (int)blockIdx.y) : (int)blockIdx.y;
  const int hgroups = p.groups / WH;
  int yb = blockIdx.x;
  const int hg = yb % hgroups;
  yb /= hgroups;
  const int kvh = yb % p.Hkv;
  const int b = yb / p.Hkv;
  const int hq = kvh * p.groups + hg * WH + wh;

  // Packed sequences: this block's sequence starts at row `row0` of every
  // tensor and has Sq = Sk = its own length; tiles past it have nothing to do.
  int64_t qb_off = (int64_t)b * p.qb, kb_off = (int64_t)b * p.kb, vb_off = (int64_t)b * p.vb,
          ob_off = (int64_t)b * p.ob;
  int Sq = p.Sq, Sk = p.Sk;
  if (p.cu_seqlens) {
    const int row0 = __builtin_amdgcn_readfirstlane(p.cu_seqlens[b]);
    Sq = Sk = __builtin_amdgcn_readfirstlane(p.cu_seqlens[b + 1]) - row0;
    qb_off = (int64_t)row0 * p.qs;
    kb_off = (int64_t)row0 * p.ks;
    vb_off = (int64_t)row0 * p.vs;
    ob_off = (int64_t)row0 * p.os;
    if (qt * QB >= Sq) return;  // uniform over the block
  }

  const int q0 = qt * QB + wq * 32;
  const int qidx = q0 + l32;
  const int qend_block = min(Sq, qt * QB + QB);
  const int off = p.q_off ? __builtin_amdgcn_readfirstlane(max(p.q_off[b], 0)) : 0;
  const int Skb = p.q_off ? min(Sk, off + Sq) : Sk;  // keys of this sequence
  const int klimit = p.causal ? min(Skb, qend_block + off) : Skb;
  const int nkt = (klimit + kKT - 1) / kKT;

  const bf16* kbase = p.k + kb_off + (int64_t)kvh * p.kh;
  const bf16* vbase = p.v + vb_off + (int64_t)kvh * p.vh;
  const int ks2 = (int)p.ks * 2;  // host guarantees Sk * ks * 2 < 2^31
  const __amdgpu_buffer_rsrc_t krs = q3::make_rsrc(kbase, (int64_t)(Sk - 1) * ks2 + D * 2);
  (void)VCH;

  // Q fragments (B operand): lane supplies Q[qidx][16 ks + 8 h .. +7].
  bf16x8 qf[KSTEPS];
  {
    const bf16* qrow = p.q + qb_off + (int64_t)hq * p.qh + (int64_t)qidx * p.qs;
    const bool ok = qidx < Sq;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      qf[ks] = (ok && ks * 16 + 8 * h < D) ? *reinterpret_cast<const bf16x8*>(qrow + ks * 16 + 8 * h) : bf16x8{};
  }
  floatx16 o[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t) o[t] = floatx16{};
  float m = -INFINITY, lpart = 0.f;

  // K: this wave's 16 rows of the tile, 4 rows per DMA instruction.
  auto issue_k = [&](int kt, int stage) {
    const uint32_t lds0 = q3::lds_addr(&sK[stage][0]) + wave * (16 * kRowK * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * wave + 4 * i + (lane >> 4);
      const int c = (lane & 15) ^ (r & 15);
      const uint32_t off = c * 8 < D ? (uint32_t)((kt * kKT + r) * ks2 + c * 16) : q3::kOOB;
      q3::dma16(krs, off, lds0 + i * 1024);
    }
  };
  // V: thread = (d chunk cd = tid & 15, key quad u = tid >> 4).
  const int vcd = tid & 15, vu = tid >> 4;
  const bool vlive = vcd < VCH;
  bf16x8 vreg[4];
  auto load_v = [&](int kt) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int key = kt * kKT + 4 * vu + kk;
      vreg[kk] = (vlive && key < Skb) ? *reinterpret_cast<const bf16x8*>(vbase + (int64_t)key * p.vs + vcd * 8)
                                       : bf16x8{};
    }
  };
  // Rows D .. 32*OT of V^T are never written; they only feed O^T rows that
  // are never stored.
  auto store_v = [&](int stage) {
    if (!vlive) return;
    bf16* dst = sV[stage];
    const int chunk = 2 * (vu >> 2) + (vu & 1);
    const int half = (vu >> 1) & 1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = vcd * 8 + e;
      u32x2 w = {pack_bf16x2(vreg[0][e], vreg[1][e]), pack_bf16x2(vreg[2][e], vreg[3][e])};
      *reinterpret_cast<u32x2*>(dst + vt_off(d, chunk) + 4 * half) = w;
    }
  };

  if (nkt > 0) {
    issue_k(0, 0);
    load_v(0);
    store_v(0);
  }
  q3::vm_wait<0>();
  __syncthreads();

  const int wave_last_q = min(q0 + 31, Sq - 1);
  const float c = p.scale_log2;
  for (int kt = 0; kt < nkt; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nkt;
    if (more) {
      issue_k(kt + 1, cur ^ 1);
      load_v(kt + 1);
    }
    const int k0 = kt * kKT;
    if (q0 < Sq && (!p.causal || k0 <= wave_last_q + off)) {
      const bf16* sKc = sK[cur];
      const bf16* sVc = sV[cur];
      floatx16 s0 = floatx16{}, s1 = floatx16{};
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(sKc + k_off(l32, 2 * ks + h));
        const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(sKc + k_off(32 + l32, 2 * ks + h));
        s0 = mfma32x32x16(a0, qf[ks], s0);
        s1 = mfma32x32x16(a1, qf[ks], s1);
      }
      // Wave-uniform: does any key of this tile need masking for this wave?
      const bool need_mask = (p.causal && k0 + kKT - 1 > q0 + off) || (k0 + kKT > Skb);
      if (need_mask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (key >= Skb || (p.causal && key > qidx + off)) s0[r] = -INFINITY;
          if (key + 32 >= Skb || (p.causal && key + 32 > qidx + off)) s1[r] = -INFINITY;
        }
      }
      float mloc = fmaxf(s0[0], s1[0]);
#pragma unroll
      for (int r = 1; r < 16; ++r) mloc = fmaxf(mloc, fmaxf(s0[r], s1[r]));
      mloc = half_max(mloc) * c;
      const bool raise = mloc > m + kRescale;
      if (__builtin_amdgcn_ballot_w64(raise) != 0) {
        const float mnew = raise ? mloc : m;
        const float alpha = fast_exp2(m - mnew);
        lpart *= alpha;
#pragma unroll
        for (int t = 0; t < OT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
        m = mnew;
      }
      const float nm = (m == -INFINITY) ? 0.f : -m;
      bf16x8 pb[4];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p0 = fast_exp2(fmaf(s0[r], c, nm));
        const float p1 = fast_exp2(fmaf(s1[r], c, nm));
        lpart += p0 + p1;
        pb[r >> 3][r & 7] = f2bf(p0);
        pb[2 + (r >> 3)][r & 7] = f2bf(p1);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < OT; ++t) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(sVc + vt_off(t * 32 + l32, 2 * j + h));
          o[t] = mfma32x32x16(a, pb[j], o[t]);
        }
    }
    if (more) store_v(cur ^ 1);
    q3::vm_wait<0>();
    __syncthreads();
  }

  if (qidx >= Sq) return;
  const float l = lpart + __shfl_xor(lpart, 32, 64);
  const float inv_l = l > 0.f ? 1.0f / l : 0.f;
  bf16* orow = p.o + ob_off + (int64_t)hq * p.oh + (int64_t)qidx * p.os;
#pragma unroll
  for (int t = 0; t < OT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = t * 32 + 8 * g + 4 * h;
      if (d < D) {
        bf16x4 v4;
#pragma unroll
        for (int e = 0; e < 4; ++e) v4[e] = f2bf(o[t][4 * g + e] * inv_l);
        *reinterpret_cast<bf16x4*>(orow + d) = v4;
      }
    }
  if (p.lse && h == 0) {  // (never with packed sequences)
    p.lse[((int64_t)b * p.Hq + hq) * p.Sq + qidx] = (m + log2f(l)) * 0.6931471805599453f;
  }
}

// ----------------------------------------------------------------- decode
// One query token per (sequence, query head) over a ragged cache, split so
// that every wave streams the same number of K/V bytes whatever the lengths:
//
//  * Work units are 32-key tiles of a (sequence b, KV head) pair, listed
//    pair-major (pair p = b * Hkv + kvh has n_b = ceil(L_b / 32) units). The
//    grid has one block of BW waves per CU (4 for groups <= 8, one per SIMD,
//    so the MFMA/softmax work of one wave runs beside the others' streams);
//    of its NW = 256 * BW waves the first W = min(U, NW) take units
//    [w * U / W, (w + 1) * U / W) of the U in all (at least one each).
//  * Each wave owns a ring of kDecSlots LDS slots. A unit's slot holds its K
//    tile, its V tile and the group's query rows, all filled by direct-to-LDS
//    loads (buffer_load ... lds, non-temporal for K and V, which are read
//    once), issued NSLOT - 1 units ahead, so the wave's stream never stops
//    between units or pairs.
//      K tile: 32 rows x 128, chunk c of row r at slot c ^ (r & 15).
//      V tile: 32 rows x 128, chunk c of row r at slot c ^ ((r & 3) << 2).
//    The PV A operand (V^T fragments) is read with ds_read_b64_tr_b16, which
//    transposes within 16-lane groups: lane i of a group receives element
//    i % 4 of the 8-byte piece that lane 4r + i / 4 addressed, r = 0..3. With
//    lane 4r + q addressing V[key_r][d0 + 4q], lane i gets V[key_0..3][d0 + i].
//  * MFMA query columns are the G heads of the group: S^T = K Q^T, online
//    softmax per column (exp2 on log2e-scaled scores, max raised only when a
//    tile exceeds it by kRescale), O^T += V^T P^T with P^T straight from the
//    S^T accumulators.
//  * A pair finished inside one wave is normalised and stored at once; a pair
//    split between waves leaves one (m, l, O) record per wave in the
//    workspace (record w + p, unique and increasing in (w, p)), merged by
//    flash_decode_combine.
constexpr int kDecUnit = 32;                                   // keys per unit
constexpr int kDecBlocks = 256;                                // one block per CU
constexpr int kDecWavesMax = kDecBlocks * 4;                   // waves of the widest variant
constexpr int kDecMaxBatch = 1024;                             // sequences the fast path takes
constexpr int kDecTile = kDecUnit * kRowK;                     // elements of a K or V tile

// Partial layout per record: m[G], l[G], O[G][D] (fp32), G = groups.
__host__ __device__ inline int dec_partial_floats(int groups, int D) { return groups * (D + 2); }

typedef short short4v __attribute__((ext_vector_type(4)));
typedef short short8v __attribute__((ext_vector_type(8)));

__device__ __forceinline__ short4v lds_read_tr16(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (short4v __attribute__((address_space(3)))*)(reinterpret_cast<uintptr_t>(p)));
}

__device__ __forceinline__ int dec_v_off(int r, int c) { return r * kRowK + ((c ^ ((r & 3) << 2)) << 3); }

// Waves that get work: min(U, NW) of the grid's NW, so every one of them has
// at least one unit; wave w takes units [w * U / nw, (w + 1) * U / nw).
__device__ __forceinline__ int dec_active_waves(int64_t U, int NW) { return (int)min<int64_t>(U, NW); }
// Active wave whose unit range contains unit u.
__device__ __forceinline__ int dec_wave_of(int64_t u, int64_t U, int NW) {
  return (int)(((u + 1) * dec_active_waves(U, NW) - 1) / U);
}

// Exclusive prefix over sequences of their unit counts, into s_pre[0..B]
// (and the clamped lengths into s_len). Block-wide; ends with a barrier.
__device__ void dec_prefix(const AttnParams& p, int* s_pre, int* s_len) {
  const int B = p.B, tid = threadIdx.x, nt = blockDim.x;
  const int per = (B + nt - 1) / nt;
  int local = 0;
  for (int i = 0; i < per; ++i) {
    const int b = tid * per + i;
    if (b < B) {
      const int L = min(max(p.kv_lens[b] + p.len_add, 0), p.Sk);
      s_len[b] = L;
      local += (L + kDecUnit - 1) / kDecUnit;
    }
  }
  // exclusive scan of `local` over the block: wave scan, then wave totals
  __shared__ int s_wsum[16];
  const int lane = tid & 63, wv = tid >> 6;
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  if (lane == 63) s_wsum[wv] = incl;
  __syncthreads();
  int base = 0;
  for (int j = 0; j < wv; ++j) base += s_wsum[j];
  int run = base + incl - local;
  for (int i = 0; i < per; ++i) {
    const int b = tid * per + i;
    if (b < B) {
      s_pre[b] = run;
      run += (s_len[b] + kDecUnit - 1) / kDecUnit;
    }
  }
  if (tid == nt - 1) s_pre[B] = run;
  __syncthreads();
}

// Position of a unit: sequence, KV head, tile, units of the sequence.
struct DecCursor {
  int b, kvh, tile, nb;
};

template <int QI, int NSLOT, int BW>
__global__ __launch_bounds__(64 * BW) void flash_decode_kernel(const AttnParams p) {
  constexpr int D = 128;
  constexpr int KSTEPS = D / 16;
  constexpr int OT = D / 32;
  constexpr int SLOT = 2 * kDecTile + QI * 4 * kRowK;  // elements per ring slot: K, V, 4 QI query rows
  constexpr int PER_UNIT = 2 * (kDecUnit / 4) + QI;     // DMA instructions per unit
  __shared__ int s_pre[kDecMaxBatch + 1];
  __shared__ int s_len[kDecMaxBatch];
  __shared__ __attribute__((aligned(1024))) bf16 ring[BW * NSLOT * SLOT];

  dec_prefix(p, s_pre, s_len);  // block-wide, before the waves part ways
  if (blockIdx.x == 0)           // for the combine kernel, which must not read the lengths
    for (int i = threadIdx.x; i <= p.B; i += blockDim.x) p.dec_hdr[i] = s_pre[i];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  const int B = p.B, Hkv = p.Hkv, G = p.groups;
  const int64_t U = (int64_t)Hkv * s_pre[B];
  const int w = blockIdx.x * BW + wave;
  const int nw = dec_active_waves(U, kDecBlocks * BW);
  if (w >= nw) return;
  const int64_t u0 = (int64_t)w * U / nw, u1 = (int64_t)(w + 1) * U / nw;

  auto locate = [&](int64_t u) {
    int lo = 0, hi = B - 1;  // largest b with Hkv * s_pre[b] <= u
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((int64_t)Hkv * s_pre[mid] <= u) lo = mid;
      else hi = mid - 1;
    }
    DecCursor c;
    c.b = lo;
    c.nb = s_pre[lo + 1] - s_pre[lo];
    const int r = (int)(u - (int64_t)Hkv * s_pre[lo]);
    c.kvh = r / c.nb;
    c.tile = r - c.kvh * c.nb;
    return c;
  };
  auto advance = [&](DecCursor& c) {
    if (++c.tile < c.nb) return;
    c.tile = 0;
    if (++c.kvh < Hkv) return;
    c.kvh = 0;
    do {
      ++c.b;
    } while (c.b < B && s_pre[c.b + 1] == s_pre[c.b]);
    c.nb = c.b < B ? s_pre[c.b + 1] - s_pre[c.b] : 0;
  };

  bf16* myring = ring + wave * NSLOT * SLOT;
  const uint32_t lring = q3::lds_addr(myring);
  const int ks2 = (int)p.ks * 2, vs2 = (int)p.vs * 2;  // host guarantees Sk * stride * 2 < 2^31

  // DMA of one unit into ring slot `slot` (zeros when `live` is false).
  auto issue = [&](const DecCursor& c, bool live, bool need_q, int slot) {
    const int L = live ? s_len[c.b] : 1;
    const int k0 = c.tile * kDecUnit;
    // Unit rows: cache rows [k0, k0 + 32) at rows [kr0, kr0 + 32) of kbase /
    // vbase; rows at or past L load zeros (past the buffer resource's end).
    const bf16* kbase;
    const bf16* vbase;
    int kr0, nrow;
    bool lv = live;
    if (p.block_table) {
      // The page id is wave-uniform (one unit per wave); pinned to a scalar so
      // the buffer resources built from it stay scalar.
      int pg = lv ? __builtin_amdgcn_readfirstlane(p.block_table[(int64_t)c.b * p.max_pages + k0 / p.page_rows]) : 0;
      if ((unsigned)pg >= (unsigned)p.num_pages) {
        if (lv && p.status && lane == 0) atomicOr(p.status, 2);
        lv = false;
        pg = 0;
      }
      kr0 = k0 % p.page_rows;
      // A unit that loads nothing (a prefetch past the wave's range, whose tile
      // may lie beyond L = 1, or a rejected page) keeps a one-row resource, so
      // its kOOB offsets stay out of range.
      nrow = lv ? kr0 + min(kDecUnit, L - k0) : 1;
      kbase = p.k + (int64_t)pg * p.kb + (int64_t)c.kvh * p.kh;
      vbase = p.v + (int64_t)pg * p.vb + (int64_t)c.kvh * p.vh;
    } else {
      kr0 = k0;
      nrow = L;
      kbase = p.k + (int64_t)c.b * p.kb + (int64_t)c.kvh * p.kh;
      vbase = p.v + (int64_t)c.b * p.vb + (int64_t)c.kvh * p.vh;
    }
    // Wave-uniform by construction; pinned to scalars so the buffer resources
    // built from them stay scalar after the two branches merge.
    auto pin = [](const bf16* x) {
      const uint64_t v = reinterpret_cast<uint64_t>(x);
      const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
      const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
      return reinterpret_cast<const bf16*>(((uint64_t)hi << 32) | lo);
    };
    kbase = pin(kbase);
    vbase = pin(vbase);
    kr0 = __builtin_amdgcn_readfirstlane(kr0);
    nrow = __builtin_amdgcn_readfirstlane(nrow);
    const bf16* qbase = p.q + (int64_t)c.b * p.qb + (int64_t)c.kvh * G * p.qh;
    const __amdgpu_buffer_rsrc_t krs = q3::make_rsrc(kbase, (int64_t)(nrow - 1) * ks2 + D * 2);
    const __amdgpu_buffer_rsrc_t vrs = q3::make_rsrc(vbase, (int64_t)(nrow - 1) * vs2 + D * 2);
    const __amdgpu_buffer_rsrc_t qrs = q3::make_rsrc(qbase, (int64_t)(G - 1) * p.qh * 2 + D * 2);
    const uint32_t lk = lring + (uint32_t)(slot * SLOT * 2);
    const uint32_t lv_ = lk + kDecTile * 2, lq = lv_ + kDecTile * 2;
    const int cs = lane & 15;
#pragma unroll
    for (int i = 0; i < kDecUnit / 4; ++i) {
      const int r = 4 * i + (lane >> 4);
      const uint32_t ko = lv ? (uint32_t)((kr0 + r) * ks2 + ((cs ^ (r & 15)) << 4)) : q3::kOOB;
      const uint32_t vo = lv ? (uint32_t)((kr0 + r) * vs2 + ((cs ^ ((r & 3) << 2)) << 4)) : q3::kOOB;
      q3::dma16_nt(krs, ko, lk + i * 1024);
      q3::dma16_nt(vrs, vo, lv_ + i * 1024);
    }
#pragma unroll
    for (int i = 0; i < QI; ++i) {
      const int j = 4 * i + (lane >> 4);  // query head of the group
      const uint32_t qo = (live && need_q && j < G) ? (uint32_t)(j * (int)p.qh * 2 + cs * 16) : q3::kOOB;
      q3::dma16(qrs, qo, lq + i * 1024);
    }
  };

  const float c2 = p.scale_log2;
  const bool qvalid = l32 < G;
  bf16x8 qf[KSTEPS];
  floatx16 o[OT];
  float m = -INFINITY, lsum = 0.f;
  auto reset = [&]() {
#pragma unroll
    for (int t = 0; t < OT; ++t) o[t] = floatx16{};
    m = -INFINITY;
    lsum = 0.f;
  };
  reset();

  // Stores the finished (or this wave's part of the) pair of cursor c.
  auto flush = [&](const DecCursor& c, int64_t pair_u0) {
    const int pair = c.b * Hkv + c.kvh;
    const int64_t pair_u1 = pair_u0 + c.nb;
    const float l = lsum + __shfl_xor(lsum, 32, 64);
    const bool whole = pair_u0 >= u0 && pair_u1 <= u1;
    if (whole) {
      if (!qvalid) return;
      const float inv = l > 0.f ? 1.0f / l : 0.f;
      bf16* orow = p.o + (int64_t)c.b * p.ob + (int64_t)(c.kvh * G + l32) * p.oh;
#pragma unroll
      for (int t = 0; t < OT; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * t + 8 * g + 4 * h;
          bf16x4 v4;
#pragma unroll
          for (int e = 0; e < 4; ++e) v4[e] = f2bf(o[t][4 * g + e] * inv);
          *reinterpret_cast<bf16x4*>(orow + d) = v4;
        }
    } else {
      const int PF = dec_partial_floats(G, D);
      float* rec = p.partial + (int64_t)(w + pair) * PF;
      if (!qvalid) return;
      if (h == 0) {
        rec[l32] = m;
        rec[G + l32] = l;
      }
#pragma unroll
      for (int t = 0; t < OT; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * t + 8 * g + 4 * h;
#pragma unroll
          for (int e = 0; e < 4; ++e) rec[2 * G + l32 * D + d + e] = o[t][4 * g + e];
        }
    }
  };

  DecCursor cc = locate(u0);  // compute cursor
  DecCursor ic = cc;          // issue cursor, NSLOT - 1 units ahead
  int64_t pair_u0 = u0 - cc.tile;  // first unit of the current pair
#pragma unroll
  for (int s = 0; s < NSLOT - 1; ++s) {
    const int64_t u = u0 + s;
    issue(ic, u < u1, ic.tile == 0 || u == u0, s);
    if (u < u1) advance(ic);
  }

  for (int64_t u = u0; u < u1; ++u) {
    const int slot = (int)((u - u0) % NSLOT);
    {
      const int64_t un = u + NSLOT - 1;
      issue(ic, un < u1, ic.tile == 0, (int)((un - u0) % NSLOT));
      if (un < u1) advance(ic);
    }
    q3::vm_wait<(NSLOT - 1) * PER_UNIT>();  // unit u's K, V (and Q) are in LDS

    const bf16* sK = myring + slot * SLOT;
    const bf16* sV = sK + kDecTile;
    const bf16* sQ = sV + kDecTile;
    if (cc.tile == 0 || u == u0) {
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks)
        qf[ks] = qvalid ? *reinterpret_cast<const bf16x8*>(sQ + l32 * kRowK + ks * 16 + 8 * h) : bf16x8{};
    }
    floatx16 s = floatx16{};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(sK + fwd::k_off(l32, 2 * ks + h));
      s = mfma32x32x16(a, qf[ks], s);
    }
    const int L = s_len[cc.b];
    const int k0 = cc.tile * kDecUnit;
    if (k0 + kDecUnit > L) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (k0 + 8 * (r >> 2) + 4 * h + (r & 3) >= L) s[r] = -INFINITY;
    }
    float mloc = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mloc = fmaxf(mloc, s[r]);
    mloc = fwd::half_max(mloc) * c2;  // finite: key k0 < L is live
    const bool raise = mloc > m + fwd::kRescale;
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {
      const float mnew = raise ? mloc : m;
      const float alpha = fast_exp2(m - mnew);
      lsum *= alpha;
#pragma unroll
      for (int t = 0; t < OT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
      m = mnew;
    }
    bf16x8 pb[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = fast_exp2(fmaf(s[r], c2, -m));
      lsum += pr;
      pb[r >> 3][r & 7] = f2bf(pr);
    }
    // V^T fragments by transposed reads: lane (g16, rr, qq) addresses
    // V[16 j + 4 h + rr (+ 8)][32 t + 16 g16 + 4 qq].
    const int g16 = (lane >> 4) & 1, rr = (lane & 15) >> 2, qq = lane & 3;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int key = 16 * j + 4 * h + rr;
#pragma unroll
      for (int t = 0; t < OT; ++t) {
        const int d = 32 * t + 16 * g16 + 4 * qq;
        const short4v lo = lds_read_tr16(sV + dec_v_off(key, d >> 3) + (d & 7));
        const short4v hi = lds_read_tr16(sV + dec_v_off(key + 8, d >> 3) + (d & 7));
        const short8v a8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[t] = mfma32x32x16(__builtin_bit_cast(bf16x8, a8), pb[j], o[t]);
      }
    }

    const bool pair_end = cc.tile == cc.nb - 1;
    if (pair_end || u == u1 - 1) {
      flush(cc, pair_u0);
      reset();
    }
    if (pair_end) pair_u0 += cc.nb;
    advance(cc);
  }
  q3::vm_wait<0>();  // no DMA may still target this block's LDS when the wave retires
}

// Merges the per-wave records of the pairs split between waves: one block
// per pair, one thread per (head, d) output.
template <int D>
__global__ __launch_bounds__(256) void flash_decode_combine(const AttnParams p) {
  const int* s_pre = p.dec_hdr;  // written by the main kernel
  const int pair = blockIdx.x;
  const int Hkv = p.Hkv, G = p.groups;
  const int b = pair / Hkv, kvh = pair % Hkv;
  // Advance the sequence's cache length (one block per sequence; nothing in
  // this launch reads the lengths).
  if (p.lens_inc && kvh == 0 && threadIdx.x == 0) p.lens_inc[b] += 1;
  const int nb = s_pre[b + 1] - s_pre[b];
  bf16* obase = p.o + (int64_t)b * p.ob + (int64_t)kvh * G * p.oh;
  if (nb == 0) {  // empty sequence: zeros
    for (int e = threadIdx.x; e < G * D; e += blockDim.x) obase[(int64_t)(e / D) * p.oh + e % D] = f2bf(0.f);
    return;
  }
  const int64_t U = (int64_t)Hkv * s_pre[p.B];
  const int64_t pu0 = (int64_t)Hkv * s_pre[b] + (int64_t)kvh * nb;
  const int wf = dec_wave_of(pu0, U, p.dec_waves), wl = dec_wave_of(pu0 + nb - 1, U, p.dec_waves);
  if (wf == wl) return;  // finished by its wave
  // Records in batches of kB with all their loads (m, l and the output
  // element) in flight together, merged into a running (max, sum, acc).
  constexpr int kB = 8;
  const int PF = dec_partial_floats(G, D);
  for (int e = threadIdx.x; e < G * D; e += blockDim.x) {
    const int qc = e / D, d = e % D;
    float mm = -INFINITY, l = 0.f, acc = 0.f;
    for (int w0 = wf; w0 <= wl; w0 += kB) {
      float mv[kB], lv[kB], ov[kB];
#pragma unroll
      for (int u = 0; u < kB; ++u) {
        const float* rec = p.partial + (int64_t)(min(w0 + u, wl) + pair) * PF;
        mv[u] = w0 + u <= wl ? rec[qc] : -INFINITY;
        lv[u] = rec[G + qc];
        ov[u] = rec[2 * G + qc * D + d];
      }
      float mb = mm;
#pragma unroll
      for (int u = 0; u < kB; ++u) mb = fmaxf(mb, mv[u]);
      const float sc = fast_exp2(mm - mb);  // 0 on the first batch (mm = -inf)
      l *= sc;
      acc *= sc;
#pragma unroll
      for (int u = 0; u < kB; ++u) {
        const float wt = fast_exp2(mv[u] - mb);  // 0 for the padding records
        l += lv[u] * wt;
        acc += ov[u] * wt;
      }
      mm = mb;
    }
    obase[(int64_t)qc * p.oh + d] = f2bf(l > 0.f ? acc / l : 0.f);
  }
}

// ----------------------------------------------------------------- prefill, pipelined (D = 128)
// Prefill kernel for head_dim 128 and GQA groups that are a multiple of 4
// (the text layers): one block = 8 waves = 4 query heads of one KV head x 2
// halves of the same 64 queries; each wave owns 32 queries of its head. All
// 8 waves share one K/V tile ring, and a wave's state (O, two S tiles, Q)
// fits 256 registers, so two waves run per SIMD: the MFMAs of one overlap
// the softmax of the other (with 64 queries per wave, one wave per SIMD, the
// same block ran ~12% slower at S=4096).
//  * 32-key K and V tiles go global -> LDS by direct-to-LDS loads into a ring
//    of kPipeStages tiles, kAhead tiles ahead. K rows: chunk c of row r at
//    slot c ^ (r & 15); V rows: chunk c at slot c ^ ((r & 3) << 2), read
//    transposed by ds_read_b64_tr_b16 (the decode kernel's V^T scheme).
//  * Per tile: S^T = K Q^T (16 MFMAs), online softmax (exp2 on log2e-scaled
//    scores; the running max rises only by more than kRescale), O^T += V^T P^T
//    (16 MFMAs) with P^T straight from the S^T accumulators.
//  * Software pipeline: step t runs O += V(t-1) P(t-1) and S(t+1) = K(t+1) Q^T
//    (32 MFMAs, neither depends on step t's softmax) and the softmax of S(t),
//    so the VALU work of the softmax runs under MFMAs already issued.
//  * O and the S tiles live in arch VGPRs (see scale_acc), so the softmax reads
//    S straight from the MFMA results and the rare rescale scales O in place.
namespace fwdp {
constexpr int kQ = 64;           // queries per block (32 per wave)
constexpr int kKeys = 32;        // keys per tile
constexpr int kPagedPrefillRegs = 8;  // paged prefill: page ids held per lane (64 * 8 = 512 pages a sequence)
constexpr int kPipeStages = 8;   // K/V tile ring depth
constexpr int kAhead = 6;        // step t issues tile t + kAhead (its slot held tile t - 2)
constexpr int kTile = kKeys * kRowK;

// acc *= alpha (the rare rescale of O). This source is built with MFMA results
// in arch VGPRs (build flag -amdgpu-mfma-vgpr-form): at 2 waves per SIMD a wave
// has 256 registers, which the compiler otherwise splits 128 VGPRs + 128 AGPRs,
// with the S tiles in AGPRs and 16 v_accvgpr_read copies per tile in the
// softmax; in VGPRs the whole state fits (202 registers at D = 128).
__device__ __forceinline__ void scale_acc(floatx16& acc, float alpha) {
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] *= alpha;
}

// The q prologue of the fused prefill on one query's fragments: the lane holds
// elements 16 ks + 8 h + e (ks < D / 16, e < 8), the other lane half (lane ^
// 32) the rest of the row. RMSNorm over the row (fp32 sum of squares, the
// halves exchanged once), times the weight, then rotate-half with the rotary
// table row (cos of the D/2 angles, then their sin): element i < D/2 pairs
// with i + D/2, which is k-step ks + D/32 of the same lane. One rounding to
// bf16 at the end, as the separate fused norm + rotation kernel. The table
// row sits in LDS as D/4 16-byte chunks, chunk c of row r at slot
// (c + r) mod D/4 (conflict-free reads across the 32 rows of a wave).
template <int D>
__device__ __forceinline__ void q_norm_rope_frag(bf16x8 (&qf)[D / 16], const bf16* __restrict__ w,
                                                 const char* tab_lds, int row, float eps, int h) {
  constexpr int KS = D / 16, HK = KS / 2, CPR = D / 4;
  auto chunk = [&](int c) {
    return *reinterpret_cast<const float4*>(tab_lds + (row * CPR + ((c + row) & (CPR - 1))) * 16);
  };
  bf16x8 wv[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) wv[ks] = *reinterpret_cast<const bf16x8*>(w + ks * 16 + 8 * h);
  float ss = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = (float)qf[ks][e];
      ss = fmaf(v, v, ss);
    }
  ss += __shfl_xor(ss, 32, 64);
  const float rstd = rsqrtf(ss / (float)D + eps);
#pragma unroll
  for (int ks = 0; ks < HK; ++ks) {
    const int c0 = ks * 4 + 2 * h;  // cos chunks c0, c0 + 1; sin chunks D/8 further
    const float4 ca = chunk(c0), cb = chunk(c0 + 1), sa = chunk(D / 8 + c0), sb = chunk(D / 8 + c0 + 1);
    const float c[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
    const float sn[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float lo = (float)qf[ks][e] * rstd * (float)wv[ks][e];
      const float hi = (float)qf[ks + HK][e] * rstd * (float)wv[ks + HK][e];
      // contraction spelled out, so the rounding does not depend on the compiler's choice
      qf[ks][e] = (bf16)fmaf(lo, c[e], -(hi * sn[e]));
      qf[ks + HK][e] = (bf16)fmaf(hi, c[e], lo * sn[e]);
    }
  }
}
}  // namespace fwdp

// PAGED (GQA prefill over a paged KV cache, p.block_table set): cache row r of
// sequence b is row r % page_rows of page block_table[b * max_pages + r /
// page_rows], p.kb / p.vb are the page strides and Sk = max_pages * page_rows.
// A 32-key tile lies inside one page (page_rows is a multiple of 32). Lane j
// holds the id of the sequence's page j + 64 i in pg_ids[i] (loaded once, before
// the first tile), so a tile's page base is a readlane away and the pipelined
// loop never waits on memory for it. A page id outside [0, num_pages) reads as
// zero rows and sets bit 1 of *status.
template <int D, bool MHA, bool PAGED = false>
__global__ __launch_bounds__(512) void flash_fwd_pipe_kernel(const AttnParams p) {
  using namespace fwdp;
  static_assert(D % 8 == 0 && D <= kRowK, "head_dim");
  constexpr int KSTEPS = (D + 15) / 16;  // MFMA k-steps over the (zero-padded) head dim
  constexpr int OT = (D + 31) / 32;      // 32-row tiles of O^T
  constexpr int QBLK = MHA ? 4 * kQ : kQ;  // queries per block
  constexpr int PERW = 2;  // DMA instructions per wave per tile (1 K + 1 V)
  static_assert(kAhead + 2 == kPipeStages, "step t reuses the slot of tile t - 2");
  __shared__ __attribute__((aligned(1024))) bf16 ring[kPipeStages * 2 * kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int h = lane >> 5;
  // GQA: the group's 4 heads x 2 query halves; MHA: one head, 4 query
  // quarters x 2 halves (every wave of the block shares the K/V tiles).
  const int hw = wave & 3, qh = wave >> 2;

  int Sq = p.Sq, Sk = p.Sk;
  const bool causal = p.causal != 0;
  const int n_qt = (Sq + QBLK - 1) / QBLK;
  const int qt = causal ? (n_qt - 1 - (int)blockIdx.y) : (int)blockIdx.y;  // heaviest first
  int yb = blockIdx.x;
  int kvh, b, hq;
  if constexpr (MHA) {  // one query head per block (any groups; the vision tower's MHA is groups 1)
    hq = yb % p.Hq;
    b = yb / p.Hq;
    kvh = hq / p.groups;
  } else {
    const int hg = yb % (p.groups / 4);
    yb /= p.groups / 4;
    kvh = yb % p.Hkv;
    b = yb / p.Hkv;
    hq = kvh * p.groups + hg * 4 + hw;
  }
  // Packed sequences: this block's sequence starts at row `row0` of every
  // tensor and has Sq = Sk = its own length; tiles past it have nothing to do.
  int64_t qb_off = (int64_t)b * p.qb, kb_off = (int64_t)b * p.kb, vb_off = (int64_t)b * p.vb,
          ob_off = (int64_t)b * p.ob;
  if (p.cu_seqlens) {
    const int row0 = __builtin_amdgcn_readfirstlane(p.cu_seqlens[b]);
    Sq = Sk = __builtin_amdgcn_readfirstlane(p.cu_seqlens[b + 1]) - row0;
    qb_off = (int64_t)row0 * p.qs;
    kb_off = (int64_t)row0 * p.ks;
    vb_off = (int64_t)row0 * p.vs;
    ob_off = (int64_t)row0 * p.os;
    if (qt * QBLK >= Sq) return;  // uniform over the block
  }
  const int q0 = qt * QBLK;
  const int qw0 = MHA ? q0 + 64 * hw + 32 * qh : q0 + 32 * qh;  // this wave's first query
  const int off = p.q_off ? __builtin_amdgcn_readfirstlane(max(p.q_off[b], 0)) : 0;
  const int Skb = p.q_off ? min(Sk, off + Sq) : Sk;  // keys of this sequence
  const int klimit = causal ? min(Skb, q0 + QBLK + off) : Skb;
  const int nkt = (klimit + kKeys - 1) / kKeys;

  const int ks2 = (int)p.ks * 2, vs2 = (int)p.vs * 2;
  // Paged: the resources span the whole page pool from this KV head's rows.
  const bf16* kbase = p.k + (PAGED ? 0 : kb_off) + (int64_t)kvh * p.kh;
  const bf16* vbase = p.v + (PAGED ? 0 : vb_off) + (int64_t)kvh * p.vh;
  const __amdgpu_buffer_rsrc_t krs =
      q3::make_rsrc(kbase, PAGED ? (int64_t)p.num_pages * p.kb * 2 - (int64_t)kvh * p.kh * 2
                                 : (int64_t)(Sk - 1) * ks2 + D * 2);
  const __amdgpu_buffer_rsrc_t vrs =
      q3::make_rsrc(vbase, PAGED ? (int64_t)p.num_pages * p.vb * 2 - (int64_t)kvh * p.vh * 2
                                 : (int64_t)(Sk - 1) * vs2 + D * 2);
  const uint32_t lbase = q3::lds_addr(ring);
  // Paged: register i of lane j holds the 16-bit ids of pages j + 128 i (low
  // half) and j + 128 i + 64 (high half); 0xffff marks a page that reads as
  // zeros. A vector type, so the ids stay in registers (a private array may be
  // moved to LDS).
  constexpr int kPgRegs = kPagedPrefillRegs / 2;
  typedef uint32_t pg_vec_t __attribute__((ext_vector_type(kPagedPrefillRegs / 2)));
  pg_vec_t pg_ids = {};
  if constexpr (PAGED) {
    const int npg = (klimit + p.page_rows - 1) / p.page_rows;  // pages this block reads
#pragma unroll
    for (int i = 0; i < 2 * kPgRegs; ++i) {
      const int j = lane + 64 * i;
      uint32_t id = 0xffffu;
      if (j < npg) {
        const int pg = p.block_table[(int64_t)b * p.max_pages + j];
        if ((unsigned)pg < (unsigned)p.num_pages) {
          id = (uint32_t)pg;
        } else if (p.status && wave == 0) {
          atomicOr(p.status, 2);
        }
      }
      pg_ids[i >> 1] |= id << (16 * (i & 1));
    }
  }

  // Wave w loads rows 4w .. 4w + 3 of tile t's K and V (one instruction each);
  // chunks at or past D load as zeros (which pads D to the MFMA k-step).
  const int cs = lane & 15;
  const int r0 = 4 * wave + (lane >> 4);
  const int kch = cs ^ (r0 & 15), vch = cs ^ ((r0 & 3) << 2);  // global chunk each lane fetches
  const uint32_t kc0 = (uint32_t)(kch << 4) | (kch * 8 < D ? 0u : q3::kOOB);
  const uint32_t vc0 = (uint32_t)(vch << 4) | (vch * 8 < D ? 0u : q3::kOOB);
  auto issue = [&](int t) {
    const uint32_t lk = lbase + (uint32_t)((t % kPipeStages) * 2 * kTile * 2) + (uint32_t)(4 * wave * kRowK * 2);
    const uint32_t lv = lk + kTile * 2;
    bool live = t < nkt;
    const int row = t * kKeys;
    if constexpr (PAGED) {
      const int pi = row / p.page_rows;  // the tile's page (uniform)
      uint32_t sel = pg_ids[0];
#pragma unroll
      for (int i = 1; i < kPgRegs; ++i) sel = (pi >> 7) == i ? pg_ids[i] : sel;
      const int pg = (int)((__builtin_amdgcn_readlane(sel, pi & 63) >> (16 * ((pi >> 6) & 1))) & 0xffffu);
      live = live && pg != 0xffff;
      const int prow = row - pi * p.page_rows + r0;  // row within the page
      q3::dma16(krs, live ? (uint32_t)(pg * (int)p.kb * 2 + prow * ks2) + kc0 : q3::kOOB, lk);
      q3::dma16(vrs, live ? (uint32_t)(pg * (int)p.vb * 2 + prow * vs2) + vc0 : q3::kOOB, lv);
    } else {
      q3::dma16(krs, live ? (uint32_t)((row + r0) * ks2) + kc0 : q3::kOOB, lk);
      q3::dma16(vrs, live ? (uint32_t)((row + r0) * vs2) + vc0 : q3::kOOB, lv);
    }
  };

  // Fused q prologue (GQA, D = 64 or 128): the first kAhead K/V tiles are
  // requested first; ring slots kAhead and kAhead + 1 (free until tile kAhead
  // is issued, after the prologue) take the rotary-table rows of the block's
  // kQ queries by direct-to-LDS loads, read once per block instead of once
  // per head wave.
  constexpr bool kQpro = !MHA && (D == 64 || D == 128);
  static_assert(!kQpro || kQ * D * 4 <= 2 * 2 * kTile * 2, "table rows fit two ring slots");
  const bool qpro = kQpro && p.rope_tab != nullptr;
  if constexpr (kQpro) {
    if (qpro) {
      if (nkt > 0) {
#pragma unroll
        for (int s = 0; s < kAhead; ++s) issue(s);
      }
      constexpr int CPR = D / 4;          // 16-byte chunks per table row
      constexpr int NI = kQ * CPR / 512;  // direct-to-LDS loads per thread
      const int ntab = min(kQ, Sq - q0);  // rows past the sequence load as zeros
      const __amdgpu_buffer_rsrc_t trs =
          q3::make_rsrc(p.rope_tab + ((int64_t)b * Sq + q0) * D, (int64_t)ntab * D * 4);
      const uint32_t ltab = lbase + (uint32_t)(kAhead * 2 * kTile * 2);
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int pos = (i * 8 + wave) * 64 + lane;  // LDS slot of 16 bytes
        const int row = pos / CPR, chunk = ((pos % CPR) - row) & (CPR - 1);
        q3::dma16(trs, (uint32_t)((row * D + chunk * 4) * 4), ltab + (uint32_t)((i * 8 + wave) * 64 * 16));
      }
    }
  }

  // Q fragments (B operand): lane supplies Q[qw0 + l32][16 ks + 8 h .. + 7].
  bf16x8 qf[KSTEPS];
  {
    const int qi = qw0 + l32;
    const bf16* qrow = p.q + qb_off + (int64_t)hq * p.qh + (int64_t)qi * p.qs;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      qf[ks] = (qi < Sq && ks * 16 + 8 * h < D) ? *reinterpret_cast<const bf16x8*>(qrow + ks * 16 + 8 * h)
                                                : bf16x8{};
    if constexpr (kQpro) {
      if (qpro) {
        q3::vm_wait<0>();
        __syncthreads();
        if (qi < Sq)
          q_norm_rope_frag<D>(qf, p.qn_w, reinterpret_cast<const char*>(ring) + kAhead * 2 * kTile * 2,
                              qw0 - q0 + l32, p.qn_eps, h);
        __syncthreads();  // the table's slots are free again
        if (nkt > 0) issue(kAhead);
      }
    }
  }

  floatx16 o[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t) o[t] = floatx16{};
  float m = -INFINITY, lsum = 0.f;
  const float c = p.scale_log2;

  int koff[KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) koff[ks] = fwd::k_off(l32, 2 * ks + h);
  const int g16 = (lane >> 4) & 1, rr = (lane & 15) >> 2, qq = lane & 3;
  int voff[OT];
#pragma unroll
  for (int dt = 0; dt < OT; ++dt) {
    const int d = 32 * dt + 16 * g16 + 4 * qq;
    voff[dt] = dec_v_off(4 * h + rr, d >> 3) + (d & 7);
  }

  auto qk = [&](floatx16& s, int t) {
    const bf16* sK = ring + (t % kPipeStages) * 2 * kTile;
    s = floatx16{};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(sK + koff[ks]);
      s = mfma32x32x16(a, qf[ks], s);
    }
  };
  auto tile_mask = [&](auto mask, int t) -> uint32_t {
    uint32_t bits = 0;
    const int k0 = t * kKeys;
    if (decltype(mask)::value && ((causal && k0 + kKeys - 1 > qw0 + off) || k0 + kKeys > Skb)) {  // uniform
      const int qi = qw0 + l32 + off;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (key >= Skb || (causal && key > qi)) bits |= 1u << r;
      }
    }
    return bits;
  };
  auto softmax_max = [&](const floatx16& s, uint32_t drop, bf16x8 (&pp)[2]) {
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, (drop >> r) & 1 ? -INFINITY : s[r]);
    const float mloc = fwd::half_max(mx) * c;  // -inf only for a tile wholly above this wave's queries
    const bool raise = mloc > m + fwd::kRescale;
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {
      const float mnew = raise ? mloc : m;
      const float alpha = fast_exp2(m - mnew);
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < OT; ++dt) scale_acc(o[dt], alpha);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) pp[j][e] = f2bf(bf2f(pp[j][e]) * alpha);
      m = mnew;
    }
  };
  auto softmax_exp = [&](const floatx16& s, uint32_t drop, bf16x8 (&pb)[2]) {
    const float nm = -m;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = (drop >> r) & 1 ? 0.f : fast_exp2(fmaf(s[r], c, nm));
      lsum += pr;
      pb[r >> 3][r & 7] = f2bf(pr);
    }
  };
  auto pv = [&](int t, const bf16x8 (&pb)[2]) {
    const bf16* sV = ring + (t % kPipeStages) * 2 * kTile + kTile;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int dt = 0; dt < OT; ++dt) {
        const short4v lo = lds_read_tr16(sV + voff[dt] + 16 * j * kRowK);
        const short4v hi = lds_read_tr16(sV + voff[dt] + (16 * j + 8) * kRowK);
        const short8v a8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[dt] = mfma32x32x16(__builtin_bit_cast(bf16x8, a8), pb[j], o[dt]);
      }
    }
  };
  auto step = [&](auto mask, int t, const floatx16& cur, floatx16& nxt, bf16x8 (&pp)[2], bf16x8 (&pc)[2]) {
    q3::vm_wait<(kAhead - 2) * PERW>();  // this wave's part of tile t + 1 has landed
    __syncthreads();                      // every wave's; step t - 1 is done with tile t - 2
    issue(t + kAhead);
    const uint32_t drop = tile_mask(mask, t);
    softmax_max(cur, drop, pp);
    // The step as 16 fenced chunks, each one MFMA (slots 0-7: O += V(t-1) P(t-1)
    // for the (j, dt) pairs; slots 8-15: S(t+1) = K(t+1) Q^T k-steps), the LDS
    // fragment reads of the slot three ahead, and one exponential of S(t), so
    // every MFMA has its operands in registers and an independent slice of the
    // softmax to hide behind.
    const bf16* sV = ring + ((t - 1) % kPipeStages) * 2 * kTile + kTile;
    const bf16* sK = ring + ((t + 1) % kPipeStages) * 2 * kTile;
    constexpr int NPV = 2 * OT, NU = NPV + KSTEPS;  // MFMA slots: PV (j, dt), then QK (ks)
    short4v vlo[NPV], vhi[NPV];
    bf16x8 kf[KSTEPS];
    auto read_u = [&](int u) {
      if (u < NPV) {
        const int j = u / OT, dt = u % OT;
        vlo[u] = lds_read_tr16(sV + voff[dt] + 16 * j * kRowK);
        vhi[u] = lds_read_tr16(sV + voff[dt] + (16 * j + 8) * kRowK);
      } else {
        kf[u - NPV] = *reinterpret_cast<const bf16x8*>(sK + koff[u - NPV]);
      }
    };
    auto mma_u = [&](int u) {
      if (u < NPV) {
        const int j = u / OT, dt = u % OT;
        const short8v a8 = {vlo[u][0], vlo[u][1], vlo[u][2], vlo[u][3], vhi[u][0], vhi[u][1], vhi[u][2], vhi[u][3]};
        o[dt] = mfma32x32x16(__builtin_bit_cast(bf16x8, a8), pp[j], o[dt]);
      } else {
        const int ks = u - NPV;
        nxt = mfma32x32x16(kf[ks], qf[ks], ks == 0 ? floatx16{} : nxt);
      }
    };
    const float nm = -m;
    auto exp_i = [&](int r) {
      const float pr = (drop >> r) & 1 ? 0.f : fast_exp2(fmaf(cur[r], c, nm));
      lsum += pr;
      pc[r >> 3][r & 7] = f2bf(pr);
    };
    __builtin_amdgcn_sched_barrier(0);
    read_u(0);
    read_u(1);
    read_u(2);
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      if (u + 3 < NU) read_u(u + 3);
      mma_u(u);
      // the tile's 16 exponentials spread over the NU slots
#pragma unroll
      for (int r = u * 16 / NU; r < (u + 1) * 16 / NU; ++r) exp_i(r);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  constexpr std::true_type kMasked{};
  constexpr std::false_type kUnmasked{};

  if (nkt > 0) {
    if (!qpro) {
#pragma unroll
      for (int s = 0; s <= kAhead; ++s) issue(s);
    }
    // (with the q prologue, tiles 0 .. kAhead - 1 have landed and only tile
    // kAhead is in flight)
    q3::vm_wait<(kAhead - 1) * PERW>();
    __syncthreads();
    floatx16 sa, sb;
    bf16x8 pa[2] = {}, pb[2] = {};
    qk(sa, 0);
    qk(sb, 1);
    {
      const uint32_t drop = tile_mask(kMasked, 0);
      softmax_max(sa, drop, pb);
      softmax_exp(sa, drop, pa);
    }
    const int nfull = min(causal ? (q0 + off) / kKeys : nkt, Skb / kKeys);
    int t = 1;
    for (; t + 1 < nfull; t += 2) {
      step(kUnmasked, t, sb, sa, pa, pb);
      step(kUnmasked, t + 1, sa, sb, pb, pa);
    }
    for (; t + 1 < nkt; t += 2) {
      step(kMasked, t, sb, sa, pa, pb);
      step(kMasked, t + 1, sa, sb, pb, pa);
    }
    if (t < nkt) {
      step(kMasked, t, sb, sa, pa, pb);
      pv(t, pb);
    } else {
      pv(t - 1, pa);
    }
  }
  q3::vm_wait<0>();

  {
    const int qi = qw0 + l32;
    const float l = lsum + __shfl_xor(lsum, 32, 64);
    if (qi < Sq) {
      const float inv_l = l > 0.f ? 1.0f / l : 0.f;
      bf16* orow = p.o + ob_off + (int64_t)hq * p.oh + (int64_t)qi * p.os;
#pragma unroll
      for (int dt = 0; dt < OT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = dt * 32 + 8 * g + 4 * h;
          if (d >= D) continue;  // rows of O^T past D come from the zero padding
          bf16x4 v4;
#pragma unroll
          for (int e = 0; e < 4; ++e) v4[e] = f2bf(o[dt][4 * g + e] * inv_l);
          *reinterpret_cast<bf16x4*>(orow + d) = v4;
        }
      if (p.lse && h == 0 && !p.cu_seqlens)
        p.lse[((int64_t)b * p.Hq + hq) * Sq + qi] = (m + log2f(l)) * 0.6931471805599453f;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(128) void flash_generic_kernel(const AttnParams p, int D, const int* kv_lens) {
  const int64_t row = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.Hq * p.Sq;
  if (row >= total) return;
  const int i = (int)(row % p.Sq);
  const int hq = (int)((row / p.Sq) % p.Hq);
  const int b = (int)(row / ((int64_t)p.Sq * p.Hq));
  const int kvh = hq / p.groups;
  int64_t qb_off = (int64_t)b * p.qb, kb_off = (int64_t)b * p.kb, vb_off = (int64_t)b * p.vb,
          ob_off = (int64_t)b * p.ob;
  int Sk = p.Sk;
  if (p.cu_seqlens) {  // packed sequences: row i of sequence b is packed row cu_seqlens[b] + i
    const int row0 = p.cu_seqlens[b];
    Sk = p.cu_seqlens[b + 1] - row0;
    if (i >= Sk) return;
    qb_off = (int64_t)row0 * p.qs;
    kb_off = (int64_t)row0 * p.ks;
    vb_off = (int64_t)row0 * p.vs;
    ob_off = (int64_t)row0 * p.os;
  }
  const T* q = reinterpret_cast<const T*>(p.q) + qb_off + (int64_t)hq * p.qh + (int64_t)i * p.qs;
  const T* kb = reinterpret_cast<const T*>(p.k) + kb_off + (int64_t)kvh * p.kh;
  const T* vb = reinterpret_cast<const T*>(p.v) + vb_off + (int64_t)kvh * p.vh;
  const int off = p.q_off ? max(p.q_off[b], 0) : 0;
  int nk = kv_lens ? min(kv_lens[b] + p.len_add, Sk) : (p.q_off ? min(Sk, off + p.Sq) : Sk);
  if (p.causal) nk = min(nk, i + off + 1);
  float acc[256];
  for (int d = 0; d < D; ++d) acc[d] = 0.f;
  float m = -INFINITY, l = 0.f;
  const float scale = p.scale_log2 / kLog2e;
  for (int j = 0; j < nk; ++j) {
    const T* kr = kb + (int64_t)j * p.ks;
    float s = 0.f;
    for (int d = 0; d < D; ++d) s += to_f<T>(q[d]) * to_f<T>(kr[d]);
    s *= scale;
    const float mn = fmaxf(m, s);
    const float a = expf(m - mn);
    const float e = expf(s - mn);
    l = l * a + e;
    const T* vr = vb + (int64_t)j * p.vs;
    for (int d = 0; d < D; ++d) acc[d] = acc[d] * a + e * to_f<T>(vr[d]);
    m = mn;
  }
  T* o = reinterpret_cast<T*>(p.o) + ob_off + (int64_t)hq * p.oh + (int64_t)i * p.os;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  for (int d = 0; d < D; ++d) o[d] = from_f<T>(acc[d] * inv);
  if (p.lse) p.lse[((int64_t)b * p.Hq + hq) * p.Sq + i] = m + logf(l);
}

bool mfma_head_dim(int64_t D) { return D == 64 || D == 72 || D == 80 || D == 96 || D == 128; }

template <int D, bool MHA, bool PAGED = false>
int launch_fwd_pipe_t(const AttnParams& p, hipStream_t st) {
  const int n_qt = (int)q3_cdiv(p.Sq, MHA ? 4 * fwdp::kQ : fwdp::kQ);
  Q3_REQUIRE(n_qt <= 65535, Q3_ERR_UNSUPPORTED);
  dim3 grid((unsigned)(MHA ? p.B * p.Hq : p.B * p.Hkv * (p.groups / 4)), (unsigned)n_qt);
  hipLaunchKernelGGL((flash_fwd_pipe_kernel<D, MHA, PAGED>), grid, dim3(512), 0, st, p);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}

// The pipelined kernel takes GQA groups that are a multiple of 4 (a block per 4
// query heads of a KV head), and a block per query head (MHA, groups 1) when the
// (longest) sequence fills most of its 256-query blocks.
bool pipe_eligible(const AttnParams& p) { return p.groups % 4 == 0 || (p.groups == 1 && p.Sq >= 192); }

template <int D>
int launch_fwd_pipe(const AttnParams& p, hipStream_t st) {
  return p.groups % 4 != 0 ? launch_fwd_pipe_t<D, true>(p, st) : launch_fwd_pipe_t<D, false>(p, st);
}

template <int D>
int launch_fwd(const AttnParams& p, hipStream_t st) {
  const int WH = (p.groups % 4 == 0) ? 4 : (p.groups % 2 == 0 ? 2 : 1);
  const int QB = 32 * (4 / WH);
  Q3_REQUIRE(q3_cdiv(p.Sq, QB) <= 65535, Q3_ERR_UNSUPPORTED);
  dim3 grid((unsigned)(p.B * p.Hkv * (p.groups / WH)), (unsigned)q3_cdiv(p.Sq, QB));
  if (WH == 4)
    hipLaunchKernelGGL((flash_fwd_kernel<D, 4>), grid, dim3(256), 0, st, p);
  else if (WH == 2)
    hipLaunchKernelGGL((flash_fwd_kernel<D, 2>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((flash_fwd_kernel<D, 1>), grid, dim3(256), 0, st, p);
  Q3_LAUNCH_CHECK();
  return Q3_OK;
}


bool strides_aligned8(const int64_t* s, int n) {
  for (int i = 0; i < n; ++i)
    if (s[i] % 8 != 0) return false;
  return true;
}

constexpr int64_t kDecHdrBytes = (kDecMaxBatch + 1 + 63) / 64 * 256;  // unit prefix, 256-byte aligned

int64_t decode_ws_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t D) {
  (void)max_len;
  // header, then one record per (wave, pair) piece: at most one per pair plus
  // one per boundary between waves
  return kDecHdrBytes + (kDecWavesMax + B * Hkv) *
                            (int64_t)dec_partial_floats((int)(Hq / std::max<int64_t>(Hkv, 1)), (int)D) *
                            (int64_t)sizeof(float);
}

__global__ void lens_inc_kernel(int* lens, int B, int add) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < B) lens[i] += add;
}

// q, k, v, o: (B, H, S, D) with element strides (b, h, s) given in `strides`
// as [qb, qh, qs, kb, kh, ks, vb, vh, vs, ob, oh, os]; the head dim is contiguous.
// q_off (B) int32 on the device or null: per-sequence query offset (see
// AttnParams::q_off). lens_add: if set, lens_add[b] += Sq after the attention.
int fwd_impl(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t Hq, int64_t Hkv,
             int64_t Sq, int64_t Sk, int64_t D, const int64_t* strides, float scale, int is_causal, int dtype,
             const int* q_off, int* lens_add, void* stream, const int* cu_seqlens = nullptr,
             const bf16* qn_w = nullptr, const float* rope_tab = nullptr, float qn_eps = 0.f,
             const int* block_table = nullptr, int64_t max_pages = 0, int64_t page_rows = 0, int64_t num_pages = 0,
             int* status = nullptr) {
  Q3_REQUIRE(q && k && v && o && strides, Q3_ERR_NULL);
  Q3_REQUIRE(B >= 0 && Hq >= 1 && Hkv >= 1 && Sq >= 0 && Sk >= 0 && D >= 1, Q3_ERR_SHAPE);
  Q3_REQUIRE(Hq % Hkv == 0, Q3_ERR_SHAPE);
  Q3_REQUIRE(D <= 256, Q3_ERR_UNSUPPORTED);
  if (B == 0 || Sq == 0) return Q3_OK;
  AttnParams p{};
  p.q = static_cast<const bf16*>(q);
  p.k = static_cast<const bf16*>(k);
  p.v = static_cast<const bf16*>(v);
  p.o = static_cast<bf16*>(o);
  p.lse = lse;
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.Sq = (int)Sq;
  p.Sk = (int)Sk;
  p.qb = strides[0];
  p.qh = strides[1];
  p.qs = strides[2];
  p.kb = strides[3];
  p.kh = strides[4];
  p.ks = strides[5];
  p.vb = strides[6];
  p.vh = strides[7];
  p.vs = strides[8];
  p.ob = strides[9];
  p.oh = strides[10];
  p.os = strides[11];
  p.scale_log2 = scale * kLog2e;
  p.causal = is_causal ? 1 : 0;
  p.groups = (int)(Hq / Hkv);
  p.q_off = q_off;
  p.cu_seqlens = cu_seqlens;
  p.qn_w = qn_w;
  p.rope_tab = rope_tab;
  p.qn_eps = qn_eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool aligned = q3_aligned(q, 16) && q3_aligned(k, 16) && q3_aligned(v, 16) && q3_aligned(o, 8) &&
                       strides_aligned8(strides, 12);
  int rc = Q3_OK;
  if (block_table) {  // paged cache: the pipelined kernel at D = 128 only
    Q3_REQUIRE(dtype == Q3_BF16, Q3_ERR_DTYPE);
    Q3_REQUIRE(aligned, Q3_ERR_ALIGN);
    Q3_REQUIRE(D == 128 && q_off != nullptr && rope_tab == nullptr && cu_seqlens == nullptr &&
                   max_pages <= 64 * fwdp::kPagedPrefillRegs,
               Q3_ERR_UNSUPPORTED);
    p.block_table = block_table;
    p.max_pages = (int)max_pages;
    p.page_rows = (int)page_rows;
    p.num_pages = (int)num_pages;
    p.status = status;
    // GQA groups of 4k: a block serves 4 query heads of a KV head; other groups:
    // a block per query head (each reads its KV head's pages).
    rc = p.groups % 4 == 0 ? launch_fwd_pipe_t<128, false, true>(p, st) : launch_fwd_pipe_t<128, true, true>(p, st);
    if (rc != Q3_OK) return rc;
    if (lens_add) {
      hipLaunchKernelGGL(lens_inc_kernel, dim3((unsigned)q3_cdiv(B, 256)), dim3(256), 0, st, lens_add, (int)B,
                         (int)Sq);
      Q3_LAUNCH_CHECK();
    }
    return Q3_OK;
  }
  if (rope_tab) {  // the fused q prologue exists in the pipelined GQA kernel only (D = 64 or 128)
    Q3_REQUIRE(dtype == Q3_BF16, Q3_ERR_DTYPE);
    Q3_REQUIRE(aligned && q3_aligned(qn_w, 16), Q3_ERR_ALIGN);
    Q3_REQUIRE((D == 64 || D == 128) && p.groups % 4 == 0 && q_off == nullptr && cu_seqlens == nullptr &&
                   (Sk + 1) * strides[5] * 2 < 0x7fffffffLL,
               Q3_ERR_UNSUPPORTED);
  }
  // The MFMA path addresses K with 32-bit buffer offsets.
  if (dtype == Q3_BF16 && mfma_head_dim(D) && aligned && Sk > 0 && (Sk + 1) * strides[5] * 2 < 0x7fffffffLL) {
    // A prefill over a KV cache always runs the pipelined kernel (a block per
    // query head when the groups are not a multiple of 4), the kernel of its
    // paged form, so paged and contiguous caches give the same output.
    const bool pipe = pipe_eligible(p) || q_off != nullptr;
    switch (D) {
      case 64:
        rc = pipe ? launch_fwd_pipe<64>(p, st) : launch_fwd<64>(p, st);
        break;
      case 72:
        rc = pipe ? launch_fwd_pipe<72>(p, st) : launch_fwd<72>(p, st);
        break;
      case 80:
        rc = pipe ? launch_fwd_pipe<80>(p, st) : launch_fwd<80>(p, st);
        break;
      case 96:
        rc = pipe ? launch_fwd_pipe<96>(p, st) : launch_fwd<96>(p, st);
        break;
      default:
        rc = pipe ? launch_fwd_pipe<128>(p, st) : launch_fwd<128>(p, st);
    }
  } else {
    const int64_t rows = B * Hq * Sq;
    if (dtype == Q3_F32)
      hipLaunchKernelGGL(flash_generic_kernel<float>, dim3((unsigned)q3_cdiv(rows, 128)), dim3(128), 0, st, p,
                         (int)D, nullptr);
    else if (dtype == Q3_BF16)
      hipLaunchKernelGGL(flash_generic_kernel<bf16>, dim3((unsigned)q3_cdiv(rows, 128)), dim3(128), 0, st, p,
                         (int)D, nullptr);
    else
      return Q3_ERR_DTYPE;
    Q3_LAUNCH_CHECK();
  }
  if (rc != Q3_OK) return rc;
  if (lens_add) {
    hipLaunchKernelGGL(lens_inc_kernel, dim3((unsigned)q3_cdiv(B, 256)), dim3(256), 0, st, lens_add, (int)B, (int)Sq);
    Q3_LAUNCH_CHECK();
  }
  return Q3_OK;
}

}  // namespace

namespace q3 {
int k_norm_rope_table(void* k, const void* q_weight, const void* k_weight, const int* positions,
                      const float* inv_freq, float* tab, int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                      const int64_t* section, float eps, const int64_t* kst, hipStream_t st);
}

extern "C" {

int64_t q3_qk_norm_rope_attention_workspace_bytes(int64_t B, int64_t S, int64_t D) {
  if (B < 0 || S < 0 || D < 0) return 0;
  return B * S * D * (int64_t)sizeof(float);
}

int q3_qk_norm_rope_attention(const void* q_in, void* k, const void* v, void* o, const void* q_weight,
                              const void* k_weight, const int* positions, const float* inv_freq, int64_t B,
                              int64_t S, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* section, float eps,
                              const int64_t* strides, float scale, int is_causal, int dtype, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  Q3_REQUIRE(q_in && k && v && o && q_weight && k_weight && positions && inv_freq && section && strides, Q3_ERR_NULL);
  Q3_REQUIRE(B >= 0 && S >= 0 && Hq >= 1 && Hkv >= 1 && Hq % Hkv == 0 && D >= 1, Q3_ERR_SHAPE);
  Q3_REQUIRE(section[0] >= 0 && section[1] >= 0 && section[2] >= 0 && section[0] + section[1] + section[2] == D / 2,
             Q3_ERR_SHAPE);
  Q3_REQUIRE(dtype == Q3_BF16, Q3_ERR_DTYPE);
  Q3_REQUIRE(D == 64 || D == 128, Q3_ERR_UNSUPPORTED);  // the k kernel's lane groups: D / 8 in {8, 16}
  Q3_REQUIRE((Hq / Hkv) % 4 == 0, Q3_ERR_UNSUPPORTED);
  Q3_REQUIRE(B * S < (1ll << 31), Q3_ERR_SHAPE);
  const int64_t need = q3_qk_norm_rope_attention_workspace_bytes(B, S, D);
  Q3_REQUIRE(workspace != nullptr && workspace_bytes >= need, Q3_ERR_WORKSPACE);
  Q3_REQUIRE(q3_aligned(workspace, 16) && q3_aligned(k_weight, 16), Q3_ERR_ALIGN);
  if (B == 0 || S == 0) return Q3_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* tab = static_cast<float*>(workspace);
  // Validate the attention call before the k rows are rewritten in place.
  {
    AttnParams probe{};
    probe.groups = (int)(Hq / Hkv);
    probe.Sq = (int)S;
    const bool aligned = q3_aligned(q_in, 16) && q3_aligned(k, 16) && q3_aligned(v, 16) && q3_aligned(o, 8) &&
                         q3_aligned(q_weight, 16) && strides_aligned8(strides, 12);
    Q3_REQUIRE(aligned, Q3_ERR_ALIGN);
    Q3_REQUIRE(pipe_eligible(probe) && (S + 1) * strides[5] * 2 < 0x7fffffffLL, Q3_ERR_UNSUPPORTED);
  }
  const int64_t kst[3] = {strides[3], strides[5], strides[4]};  // (b, s, h)
  const int rc = q3::k_norm_rope_table(k, q_weight, k_weight, positions, inv_freq, tab, B, S, Hq, Hkv, D, section,
                                       eps, kst, st);
  if (rc != Q3_OK) return rc;
  return fwd_impl(q_in, k, v, o, nullptr, B, Hq, Hkv, S, S, D, strides, scale, is_causal, dtype, nullptr, nullptr,
                  stream, nullptr, static_cast<const bf16*>(q_weight), tab, eps);
}

int q3_flash_attention(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t Hq,
                       int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, const int64_t* strides, float scale,
                       int is_causal, int dtype, void* stream) {
  return fwd_impl(q, k, v, o, lse, B, Hq, Hkv, Sq, Sk, D, strides, scale, is_causal, dtype, nullptr, nullptr,
                  stream);
}

// Packed variable-length sequences (the vision tower's images): q/k/v/o are
// (H, total, D) views with strides [h, s] each (strides = [qh, qs, kh, ks, vh,
// vs, oh, os]); sequence b is rows [cu_seqlens[b], cu_seqlens[b + 1]) (int32
// on the device, cu_seqlens[0] = 0), attending only within itself;
// max_seqlen >= every sequence's length.
int q3_flash_attention_varlen(const void* q, const void* k, const void* v, void* o, const int* cu_seqlens,
                              int64_t n_seqs, int64_t total, int64_t max_seqlen, int64_t Hq, int64_t Hkv, int64_t D,
                              const int64_t* strides, float scale, int is_causal, int dtype, void* stream) {
  Q3_REQUIRE(q && k && v && o && cu_seqlens && strides, Q3_ERR_NULL);
  Q3_REQUIRE(n_seqs >= 0 && total >= 0 && max_seqlen >= 0 && max_seqlen <= total, Q3_ERR_SHAPE);
  if (n_seqs == 0 || total == 0) return Q3_OK;
  const int64_t st12[12] = {0, strides[0], strides[1], 0, strides[2], strides[3],
                            0, strides[4], strides[5], 0, strides[6], strides[7]};
  // Sk = total: keys are addressed within the packed rows (buffer bounds).
  return fwd_impl(q, k, v, o, nullptr, n_seqs, Hq, Hkv, max_seqlen, total, D, st12, scale, is_causal, dtype,
                  nullptr, nullptr, stream, cu_seqlens);
}

// Prefill of Sq new tokens per sequence over a ragged KV cache whose rows
// [kv_lens[b], kv_lens[b] + Sq) already hold the new tokens' K/V: query i of
// sequence b attends causally to rows [0, kv_lens[b] + i]; kv_lens[b] += Sq
// afterwards when `advance` is non-zero. strides as q3_flash_attention's with
// k/v the (B, Hkv, cap, D) caches.
int q3_flash_attention_cache(const void* q, const void* k_cache, const void* v_cache, int* kv_lens, void* o,
                             int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t cap, int64_t D,
                             const int64_t* strides, float scale, int advance, int dtype, void* stream) {
  Q3_REQUIRE(kv_lens, Q3_ERR_NULL);
  Q3_REQUIRE(Sq <= cap, Q3_ERR_SHAPE);
  return fwd_impl(q, k_cache, v_cache, o, nullptr, B, Hq, Hkv, Sq, cap, D, strides, scale, 1, dtype, kv_lens,
                  advance ? kv_lens : nullptr, stream);
}

// The same over a paged cache: cache row r of sequence b is row r % page_rows
// of page block_table[b * max_pages + r / page_rows] of k_pages / v_pages
// (num_pages, Hkv, page_rows, D). strides = [qb, qh, qs, k page, kh, ks,
// v page, vh, vs, ob, oh, os]. bf16, D = 128,
// max_pages <= 512, fewer than 65535 pages, pools under 2 GiB (32-bit
// offsets); else
// Q3_ERR_UNSUPPORTED. A page id outside [0, num_pages) reads as zero rows and
// sets bit 1 of *status (a device int32, or null).
int q3_flash_attention_cache_paged(const void* q, const void* k_pages, const void* v_pages, const int* block_table,
                                   int64_t max_pages, int64_t page_rows, int64_t num_pages, int* kv_lens, void* o,
                                   int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D, const int64_t* strides,
                                   float scale, int advance, int dtype, int* status, void* stream) {
  Q3_REQUIRE(q && k_pages && v_pages && block_table && kv_lens && o && strides, Q3_ERR_NULL);
  Q3_REQUIRE(max_pages >= 1 && num_pages >= 1 && page_rows >= 32 && page_rows % 32 == 0, Q3_ERR_SHAPE);
  Q3_REQUIRE(max_pages * page_rows < (1ll << 31) && Sq <= max_pages * page_rows, Q3_ERR_SHAPE);
  Q3_REQUIRE(num_pages < 0xffff && num_pages * strides[3] * 2 < 0x7fffffffLL &&
                 num_pages * strides[6] * 2 < 0x7fffffffLL,
             Q3_ERR_UNSUPPORTED);
  Q3_REQUIRE(strides[3] >= Hkv * page_rows * D && strides[6] >= Hkv * page_rows * D, Q3_ERR_SHAPE);
  return fwd_impl(q, k_pages, v_pages, o, nullptr, B, Hq, Hkv, Sq, max_pages * page_rows, D, strides, scale, 1, dtype,
                  kv_lens, advance ? kv_lens : nullptr, stream, nullptr, nullptr, nullptr, 0.f, block_table, max_pages,
                  page_rows, num_pages, status);
}

int64_t q3_decode_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t D) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || max_len <= 0 || D <= 0) return 0;
  return decode_ws_bytes(B, Hq, Hkv, max_len, D);
}

// One query token per sequence over a ragged KV cache.
// q: (B, Hq, D) strides [qb, qh]; caches: (B, Hkv, cap, D) strides [b, h, s];
// o: (B, Hq, D) strides [ob, oh]; kv_lens (B) int32 on device: sequence b
// attends to cache positions [0, kv_lens[b]); max_len >= max(kv_lens).
// strides = [qb, qh, kb, kh, ks, vb, vh, vs, ob, oh].
}  // extern "C"

namespace {

// Whether decode_impl takes the MFMA split-K path (the one that uses the
// workspace) for these arguments.
bool dec_fast_path(const void* q, const void* k_cache, const void* v_cache, int64_t B, int64_t Hq, int64_t Hkv,
                   int64_t D, int64_t max_len, const int64_t* strides, int dtype) {
  const bool aligned = q3_aligned(q, 16) && q3_aligned(k_cache, 16) && q3_aligned(v_cache, 16) &&
                       strides_aligned8(strides, 8);
  // The MFMA path addresses the cache with 32-bit buffer offsets.
  return dtype == Q3_BF16 && D == 128 && Hq / Hkv <= 32 && B <= kDecMaxBatch && aligned &&
         (max_len + 1) * strides[4] * 2 < 0x7fffffffLL && (max_len + 1) * strides[7] * 2 < 0x7fffffffLL;
}

// Paged cache (block_table set): kb / vb in `strides` are the page strides and
// max_len = max_pages * page_rows; only the MFMA path reads pages.
int decode_impl(const void* q, const void* k_cache, const void* v_cache, const int* kv_lens, int len_add,
                int* lens_inc, void* o, int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len,
                const int64_t* strides, float scale, int dtype, void* workspace, int64_t workspace_bytes,
                void* stream, const int* block_table = nullptr, int64_t max_pages = 0, int64_t page_rows = 0,
                int64_t num_pages = 0, int* status = nullptr) {
  Q3_REQUIRE(q && k_cache && v_cache && kv_lens && o && strides, Q3_ERR_NULL);
  Q3_REQUIRE(B >= 0 && Hq >= 1 && Hkv >= 1 && Hq % Hkv == 0 && D >= 1 && max_len >= 1, Q3_ERR_SHAPE);
  if (block_table) {
    const bool fast = dtype == Q3_BF16 && D == 128 && Hq / Hkv <= 32 && B <= kDecMaxBatch && q3_aligned(q, 16) &&
                      q3_aligned(k_cache, 16) && q3_aligned(v_cache, 16) && strides_aligned8(strides, 8) &&
                      page_rows * strides[4] * 2 < 0x7fffffffLL && page_rows * strides[7] * 2 < 0x7fffffffLL;
    Q3_REQUIRE(fast, Q3_ERR_UNSUPPORTED);
  }
  if (B == 0) return Q3_OK;
  AttnParams p{};
  p.q = static_cast<const bf16*>(q);
  p.k = static_cast<const bf16*>(k_cache);
  p.v = static_cast<const bf16*>(v_cache);
  p.o = static_cast<bf16*>(o);
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.Sq = 1;
  p.Sk = (int)max_len;
  p.qb = strides[0];
  p.qh = strides[1];
  p.qs = 0;
  p.kb = strides[2];
  p.kh = strides[3];
  p.ks = strides[4];
  p.vb = strides[5];
  p.vh = strides[6];
  p.vs = strides[7];
  p.ob = strides[8];
  p.oh = strides[9];
  p.os = 0;
  p.scale_log2 = scale * kLog2e;
  p.causal = 0;
  p.groups = (int)(Hq / Hkv);
  p.kv_lens = kv_lens;
  p.len_add = len_add;
  p.block_table = block_table;
  p.max_pages = (int)max_pages;
  p.page_rows = (int)page_rows;
  p.num_pages = (int)num_pages;
  p.status = status;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (block_table || dec_fast_path(q, k_cache, v_cache, B, Hq, Hkv, D, max_len, strides, dtype)) {
    Q3_REQUIRE(workspace != nullptr && workspace_bytes >= decode_ws_bytes(B, Hq, Hkv, max_len, D), Q3_ERR_WORKSPACE);
    Q3_REQUIRE(q3_aligned(workspace, 16), Q3_ERR_ALIGN);
    p.dec_hdr = static_cast<int*>(workspace);
    p.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kDecHdrBytes);
    p.lens_inc = lens_inc;
    // Four waves per CU with two ring slots each where a slot fits (groups
    // <= 8), else two waves with three slots (the LDS holds ~150 KB of ring).
    const dim3 grid(kDecBlocks);
    p.dec_waves = kDecBlocks * (p.groups <= 8 ? 4 : 2);
    if (p.groups <= 4)
      hipLaunchKernelGGL((flash_decode_kernel<1, 2, 4>), grid, dim3(256), 0, st, p);
    else if (p.groups <= 8)
      hipLaunchKernelGGL((flash_decode_kernel<2, 2, 4>), grid, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((flash_decode_kernel<8, 3, 2>), grid, dim3(128), 0, st, p);
    Q3_LAUNCH_CHECK();
    hipLaunchKernelGGL(flash_decode_combine<128>, dim3((unsigned)(B * Hkv)), dim3(256), 0, st, p);
    Q3_LAUNCH_CHECK();
    return Q3_OK;
  }
  const int64_t rows = B * Hq;
  if (dtype == Q3_F32)
    hipLaunchKernelGGL(flash_generic_kernel<float>, dim3((unsigned)q3_cdiv(rows, 128)), dim3(128), 0, st, p, (int)D,
                       kv_lens);
  else if (dtype == Q3_BF16)
    hipLaunchKernelGGL(flash_generic_kernel<bf16>, dim3((unsigned)q3_cdiv(rows, 128)), dim3(128), 0, st, p, (int)D,
                       kv_lens);
  else
    return Q3_ERR_DTYPE;
  Q3_LAUNCH_CHECK();
  if (lens_inc) {
    hipLaunchKernelGGL(lens_inc_kernel, dim3((unsigned)q3_cdiv(B, 256)), dim3(256), 0, st, lens_inc, (int)B, 1);
    Q3_LAUNCH_CHECK();
  }
  return Q3_OK;
}

}  // namespace

extern "C" {

int q3_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int* kv_lens, void* o,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len, const int64_t* strides,
                        float scale, int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  return decode_impl(q, k_cache, v_cache, kv_lens, 0, nullptr, o, B, Hq, Hkv, D, max_len, strides, scale, dtype,
                     workspace, workspace_bytes, stream);
}

int q3_decode_attention_step(const void* q, const void* k_cache, const void* v_cache, int* kv_lens, void* o,
                             int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len, const int64_t* strides,
                             float scale, int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  return decode_impl(q, k_cache, v_cache, kv_lens, 1, kv_lens, o, B, Hq, Hkv, D, max_len, strides, scale, dtype,
                     workspace, workspace_bytes, stream);
}

int q3_decode_attention_paged(const void* q, const void* k_pages, const void* v_pages, const int* block_table,
                              int64_t max_pages, int64_t page_rows, int64_t num_pages, int* kv_lens, int advance,
                              void* o, int64_t B, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides,
                              float scale, int dtype, void* workspace, int64_t workspace_bytes, int* status,
                              void* stream) {
  Q3_REQUIRE(block_table, Q3_ERR_NULL);
  Q3_REQUIRE(max_pages >= 1 && num_pages >= 1 && page_rows >= kDecUnit && page_rows % kDecUnit == 0, Q3_ERR_SHAPE);
  Q3_REQUIRE(max_pages * page_rows < (1ll << 31) && num_pages < (1ll << 31), Q3_ERR_SHAPE);
  return decode_impl(q, k_pages, v_pages, kv_lens, advance ? 1 : 0, advance ? kv_lens : nullptr, o, B, Hq, Hkv, D,
                     max_pages * page_rows, strides, scale, dtype, workspace, workspace_bytes, stream, block_table,
                     max_pages, page_rows, num_pages, status);
}

}  // extern "C"

// ----------------------------------------------------------------- allocation-free decode step
// The decode step's workspace (unit-prefix header + split-K records) in a
// static device array instead of a caller allocation. Every GPU the library
// runs on holds its own copy for the life of the process; calls on one GPU
// share it, so calls that overlap in time on one GPU race (stream-ordered
// calls are fine: each call writes every byte it reads before reading it, so
// nothing needs clearing between calls).
namespace {

constexpr int64_t kDecScratchBytes = 32ll << 20;
constexpr int kScratchMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kDecScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchMaxDevices] = {};

// The device address of `scratch` on the current device (looked up once per
// device, with that device current): host code never passes the symbol
// itself, which names a host-side shadow, to a kernel.
int scratch_for_current_device(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (stream) {
    int sdev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) return (int)e;
    if (sdev != dev) return Q3_ERR_UNSUPPORTED;  // the stream must belong to the current device
  }
  if (dev < 0 || dev >= kScratchMaxDevices) return Q3_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr) return (int)hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return Q3_OK;
}

}  // namespace

extern "C" {

int64_t q3_decode_attention_step_noalloc_max_bytes(void) { return kDecScratchBytes; }

int q3_decode_attention_step_noalloc(const void* q, const void* k_cache, const void* v_cache, int* kv_lens, void* o,
                                     int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len,
                                     const int64_t* strides, float scale, int dtype, void* stream) {
  Q3_REQUIRE(q && k_cache && v_cache && kv_lens && o && strides, Q3_ERR_NULL);
  Q3_REQUIRE(B >= 0 && Hq >= 1 && Hkv >= 1 && Hq % Hkv == 0 && D >= 1 && max_len >= 1, Q3_ERR_SHAPE);
  if (B == 0) return Q3_OK;
  // Sizes whose workspace would not fit the static array are refused before
  // anything touches the device.
  const bool fast = dec_fast_path(q, k_cache, v_cache, B, Hq, Hkv, D, max_len, strides, dtype);
  Q3_REQUIRE(!fast || decode_ws_bytes(B, Hq, Hkv, max_len, D) <= kDecScratchBytes, Q3_ERR_SCRATCH);
  void* ws = nullptr;
  if (fast) {
    const int rc = scratch_for_current_device(stream, &ws);
    if (rc != Q3_OK) return rc;
  }
  return decode_impl(q, k_cache, v_cache, kv_lens, 1, kv_lens, o, B, Hq, Hkv, D, max_len, strides, scale, dtype,
                     ws, fast ? kDecScratchBytes : 0, stream);
}

}  // extern "C"
