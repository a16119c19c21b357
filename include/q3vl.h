/* C-ABI of libq3vl.so: the MI355X (gfx950) kernels of the Qwen3-VL operator layer.
 *
 * Conventions (all entry points):
 *  - Plain device pointers, int64 sizes and element strides; the innermost
 *    dimension of every tensor is contiguous.
 *  - `dtype` is a q3_dtype; every tensor of a call shares it unless stated.
 *  - `stream` is a hipStream_t passed as void*; work is enqueued on it and the
 *    call never synchronises.
 *  - Return 0 on success; a negative q3_status when argument validation
 *    failed (checked on the host before anything touches the device, so these
 *    paths work without a GPU); a positive value is the hipError_t of a failed
 *    launch.
 *  - The library allocates nothing: callers pass outputs and, where a
 *    *_workspace_bytes query says so, a device workspace. It keeps no pointer
 *    after returning and has no global state, except the static device
 *    scratch array of the allocation-free entry point (one per GPU, with its
 *    device address cached per device on first use).
 *
 * Reference interfaces replaced (paths relative to the reference's
 * CUDA_qwen3_5-main/CUDA_qwen3_5-main/cuda_qwen3_vl/): the torch-op schemas
 * registered in csrc/<op>_op.cpp and called by kernels/<op>.py.
 */
#ifndef Q3VL_H
#define Q3VL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q3VL_ABI_VERSION 2

typedef enum { Q3_F32 = 0, Q3_BF16 = 1 } q3_dtype;

typedef enum {
  Q3_OK = 0,
  Q3_ERR_NULL = -1,        /* a required pointer is null */
  Q3_ERR_SHAPE = -2,       /* inconsistent or negative sizes */
  Q3_ERR_DTYPE = -3,       /* dtype not supported by this op */
  Q3_ERR_ALIGN = -4,       /* pointer / stride alignment violated */
  Q3_ERR_UNSUPPORTED = -5, /* valid request outside what the kernels cover */
  Q3_ERR_WORKSPACE = -6,   /* workspace missing or smaller than *_workspace_bytes */
  Q3_ERR_SCRATCH = -7      /* request larger than a static scratch buffer (allocation-free entry points) */
} q3_status;

int q3_abi_version(void);
const char* q3_error_string(int code);

/* ---------------------------------------------------------------- GEMM
 * y[m, n] = sum_k x[m, k] * w[n, k] (+ bias[n]) (+ residual[m, n]), one rounding.
 * Replaces matmul_forward(Tensor x, Tensor weight, Tensor? bias)
 * (csrc/matmul_op.cpp:12, called from kernels/matmul.py:72). The residual
 * operand fuses residual_add (csrc/residual_add_op.cpp:6) into the epilogue.
 * bias/residual may be null. M <= 32 (bf16) runs the weight-streaming path,
 * which needs a workspace (q3_matmul_workspace_bytes): its first 16 KiB hold
 * tile counters that must be zero before the workspace's first use (allocate
 * it zero-filled) and that every call leaves zero. A few-tile, long-K plain
 * GEMM (q3_matmul, M > 32) may also ask for one: the query then returns 16 KiB
 * plus fp32 partial planes of a split over K (behind the counters, never
 * touching them); given a smaller workspace, or none, the call runs unsplit.
 * Calls that may run at the same time must not share a workspace; any number
 * of stream-ordered calls, of any shape, may. */
int64_t q3_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K, int dtype, int swiglu);
int q3_matmul(const void* x, const void* w, const void* bias, const void* residual, void* y, int64_t M, int64_t N,
              int64_t K, int64_t ldx, int64_t ldw, int64_t ldr, int64_t ldc, int dtype, void* workspace,
              int64_t workspace_bytes, void* stream);

/* Several weight matrices over the same input in one launch: y[:, c_i + j] =
 * x . w[i][j] (+ bias[i][j]) with c_i = n[0] + ... + n[i-1], 1 <= nseg <= 4,
 * every w[i] (n[i], K) with row stride ldw. Replaces the three
 * matmul_forward calls of CudaFullAttention's q/k/v projections
 * (modules/attention.py:82-84, csrc/matmul_op.cpp:12) with one GEMM over the
 * stacked weights, without copying them. bias may be null, or hold null
 * entries. Workspace: q3_matmul_segments_workspace_bytes. */
int64_t q3_matmul_segments_workspace_bytes(int64_t M, const int64_t* n, int64_t nseg, int64_t K, int dtype);
int q3_matmul_segments(const void* x, const void* const* w, const void* const* bias, const int64_t* n, int64_t nseg,
                       void* y, int64_t M, int64_t K, int64_t ldx, int64_t ldw, int64_t ldc, int dtype,
                       void* workspace, int64_t workspace_bytes, void* stream);

/* y[m, n] = silu(x . w_gate[n]) * (x . w_up[n]). Fuses the gate/up projections
 * and swiglu_forward (csrc/swiglu_op.cpp:9) of CudaSwiGLUMLP
 * (modules/mlp.py:19-22). */
int q3_matmul_swiglu(const void* x, const void* w_gate, const void* w_up, void* y, int64_t M, int64_t N, int64_t K,
                     int64_t ldx, int64_t ldw, int64_t ldc, int dtype, void* workspace, int64_t workspace_bytes,
                     void* stream);

/* y = gelu_tanh(x . w^T + bias): the fc1 projection and gelu_tanh_forward
 * (csrc/gelu_tanh_op.cpp:7) of CudaVisionMLP (modules/mlp.py:33-34) and of
 * CudaVisionPatchMerger (modules/vision_patch.py:68) in one GEMM, the
 * activation applied in fp32 before the single rounding. bias may be null. */
int q3_matmul_gelu(const void* x, const void* w, const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                   int64_t ldx, int64_t ldw, int64_t ldc, int dtype, void* stream);

/* Decode-shaped (1 <= M <= 32 rows, bf16) RMSNorm fused into the projection
 * that consumes it: y = rmsnorm(x; norm_w, eps) . w^T, per segment (+ bias),
 * or silu(. w_gate) * (. w_up). The rows are normalised as X is staged into
 * the weight-streaming kernel (x * norm_w rounded to bf16 once, rows scaled
 * by rsqrt(mean(x^2) + eps) in fp32 after the dot products), so the
 * normalised rows never go to memory. Equals q3_rmsnorm followed by
 * q3_matmul_segments / q3_matmul_swiglu to bf16 rounding. No counterpart in
 * the reference (CudaTextDecoderLayer.forward, modules/text_decoder.py:56-58,
 * runs the RMSNorm and then the projections); used by this library's
 * decoder-layer composition for decode steps. Needs x,
 * norm_w and each weight 16-byte aligned, ldx, ldw and K multiples of 8
 * (else Q3_ERR_ALIGN); M > 32 gives Q3_ERR_UNSUPPORTED. No workspace. */
int q3_rmsnorm_matmul_segments(const void* x, const void* norm_w, float eps, const void* const* w,
                               const void* const* bias, const int64_t* n, int64_t nseg, void* y, int64_t M, int64_t K,
                               int64_t ldx, int64_t ldw, int64_t ldc, int dtype, void* stream);
int q3_rmsnorm_matmul_swiglu(const void* x, const void* norm_w, float eps, const void* w_gate, const void* w_up,
                             void* y, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldc,
                             int dtype, void* stream);

/* y[e] = x[e] . w[e]^T for x (E, M, K), w (E, N, K), y (E, M, N), contiguous.
 * Replaces batched_gemm_forward(Tensor x, Tensor weight)
 * (csrc/moe_routing_op.cpp:12, kernels/moe_routing.py:126-181). */
int q3_batched_gemm(const void* x, const void* w, void* y, int64_t E, int64_t M, int64_t N, int64_t K, int dtype,
                    void* stream);

/* ---------------------------------------------------------------- elementwise (n elements, contiguous)
 * residual_add_forward(Tensor a, Tensor b)   csrc/residual_add_op.cpp:6
 * swiglu_forward(Tensor gate, Tensor up)     csrc/swiglu_op.cpp:9
 * gelu_tanh_forward(Tensor x)                csrc/gelu_tanh_op.cpp:7 */
int q3_residual_add(const void* a, const void* b, void* y, int64_t n, int dtype, void* stream);
int q3_swiglu(const void* gate, const void* up, void* y, int64_t n, int dtype, void* stream);
int q3_gelu_tanh(const void* x, void* y, int64_t n, int dtype, void* stream);

/* ---------------------------------------------------------------- row reductions (rows x cols, contiguous)
 * rmsnorm_forward(Tensor x, Tensor weight, float eps)               csrc/rmsnorm_op.cpp:10
 * layernorm_forward(Tensor x, Tensor weight, Tensor? bias, float eps) csrc/layernorm_op.cpp:8
 * softmax_forward(Tensor x)                                          csrc/softmax_op.cpp:7
 * topk_forward(Tensor x, int k) -> (vals in x dtype, idx int64), ties to the lowest
 *   index                                                            csrc/moe_routing_op.cpp:10 */
int q3_rmsnorm(const void* x, const void* weight, void* y, int64_t rows, int64_t cols, float eps, int dtype,
               void* stream);
int q3_layernorm(const void* x, const void* weight, const void* bias, void* y, int64_t rows, int64_t cols, float eps,
                 int dtype, void* stream);
int q3_softmax(const void* x, void* y, int64_t rows, int64_t cols, int dtype, void* stream);
int q3_topk(const void* x, void* vals, int64_t* idx, int64_t rows, int64_t cols, int64_t k, int dtype, void* stream);

/* ---------------------------------------------------------------- rotary
 * x, y: (B, H, S, D) with element strides [b, h, s]; rotate-half over the first
 * D_rope dims, the rest copied. cos/sin dtype: cos_dtype (Q3_F32 or Q3_BF16).
 * q3_rope replaces rope_forward(Tensor x, Tensor cos, Tensor sin) (csrc/rope_op.cpp:6):
 *   cos element (b, s, i) at b * cos_batch_stride + s * cos_seq_stride + i
 *   (cos_batch_stride 0 broadcasts one table over the batch).
 * q3_mrope replaces apply_mrope (kernels/mrope.py:80-104, mrope_forward csrc/mrope_op.cpp:6)
 *   with cos3d/sin3d (3, B, S, D_rope) read in place: cos_strides = [axis, b, s],
 *   section = 3 ints summing to D_rope / 2 (the chunked section layout). */
int q3_rope(const void* x, const void* cos, const void* sin, void* y, int64_t B, int64_t H, int64_t S, int64_t D,
            int64_t D_rope, const int64_t* x_strides, const int64_t* y_strides, int64_t cos_batch_stride,
            int64_t cos_seq_stride, int dtype, int cos_dtype, void* stream);
int q3_mrope(const void* x, const void* cos3d, const void* sin3d, void* y, int64_t B, int64_t H, int64_t S, int64_t D,
             int64_t D_rope, const int64_t* section, const int64_t* x_strides, const int64_t* y_strides,
             const int64_t* cos_strides, int dtype, int cos_dtype, void* stream);

/* Fused attention prologue of CudaFullAttention.forward (modules/attention.py:82-88):
 * q_norm/k_norm RMSNorm over the head dim, mRoPE of q and k (angles
 * positions[axis, b, s] * inv_freq[i] in fp32, modules/rotary.py:43-55; chunked
 * section layout, kernels/mrope.py:19-35), and a copy of v. Inputs and outputs
 * are (B, S, H, D) views with element strides; strides = 18 values, (b, s, h)
 * for q_in, k_in, v_in, q_out, k_out, v_out. positions: (3, B, S) int32,
 * inv_freq: (D / 2) fp32, both on the device. dst_seq_offset (B) int32 or null
 * shifts the sequence index of k_out / v_out rows (KV-cache append); rows whose
 * shifted index is >= dst_seq_cap (when > 0) are not written.
 * q_weight/k_weight both null: no normalisation (rotary only); v_in/v_out both
 * null: no v copy. */
int q3_qk_norm_rope(const void* q_in, const void* k_in, const void* v_in, void* q_out, void* k_out, void* v_out,
                    const void* q_weight, const void* k_weight, const int* positions, const float* inv_freq,
                    const int* dst_seq_offset, int64_t dst_seq_cap, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                    int64_t D, const int64_t* section, float eps, const int64_t* strides, int dtype, void* stream);

/* ---------------------------------------------------------------- attention
 * Replaces flash_attention_forward(Tensor q, Tensor k, Tensor v, float scale,
 * bool is_causal, int num_kv_groups) (csrc/flash_attention_op.cpp:14,
 * kernels/flash_attention.py:82-100). q (B, Hq, Sq, D), k/v (B, Hkv, Sk, D),
 * o (B, Hq, Sq, D); strides = [qb, qh, qs, kb, kh, ks, vb, vh, vs, ob, oh, os].
 * Query head h uses KV head h / (Hq / Hkv). Causal masks key j > query i
 * (top-left aligned). lse (B, Hq, Sq) fp32 natural-log LSE, or null. */
int q3_flash_attention(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t Hq,
                       int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, const int64_t* strides, float scale,
                       int is_causal, int dtype, void* stream);

/* The attention half of CudaFullAttention.forward without a cache (reference
 * modules/attention.py:83-96: q_norm / k_norm, mRoPE, attention) in two
 * launches: k is RMS-normalised and rotated in place (the layer returns it),
 * and q, read raw from the projection output, is normalised and rotated
 * inside the attention kernel as it is loaded; q_in is not modified. q_in,
 * k, v, o are (B, H, S, D) views with strides = [qb, qh, qs, kb, kh, ks, vb,
 * vh, vs, ob, oh, os] (Sq = Sk = S); positions (3, B, S) int32; inv_freq
 * (D/2) fp32; section as q3_qk_norm_rope; weights (D). The workspace holds
 * the per-token rotary table: q3_qk_norm_rope_attention_workspace_bytes.
 * Results equal q3_qk_norm_rope followed by q3_flash_attention up to the
 * order of the q row's sum of squares. bf16, D in {64, 128}, Hq / Hkv a
 * multiple of 4 only (else Q3_ERR_UNSUPPORTED, checked before any launch). */
int64_t q3_qk_norm_rope_attention_workspace_bytes(int64_t B, int64_t S, int64_t D);
int q3_qk_norm_rope_attention(const void* q_in, void* k, const void* v, void* o, const void* q_weight,
                              const void* k_weight, const int* positions, const float* inv_freq, int64_t B,
                              int64_t S, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* section, float eps,
                              const int64_t* strides, float scale, int is_causal, int dtype, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* Attention over packed variable-length sequences (the vision tower's images,
 * each attending only within itself: HF's cu_seqlens form of the attention
 * the reference runs over one concatenated sequence, models/common.py:198).
 * q/k/v/o are (H, total, D) views with strides = [qh, qs, kh, ks, vh, vs, oh,
 * os]; sequence b is rows [cu_seqlens[b], cu_seqlens[b + 1]) (n_seqs + 1
 * int32 on the device, cu_seqlens[0] = 0, last = total); max_seqlen >= every
 * sequence's length. is_causal applies within each sequence. */
int q3_flash_attention_varlen(const void* q, const void* k, const void* v, void* o, const int* cu_seqlens,
                              int64_t n_seqs, int64_t total, int64_t max_seqlen, int64_t Hq, int64_t Hkv, int64_t D,
                              const int64_t* strides, float scale, int is_causal, int dtype, void* stream);

/* A prefill chunk of Sq tokens per sequence over a ragged KV cache: the
 * S > 1 case of CudaFullAttention.forward with a cache
 * (modules/attention.py:89-96) without the torch.cat growth. k/v cache
 * (B, Hkv, cap, D) whose rows [kv_lens[b], kv_lens[b] + Sq) already hold the
 * chunk's keys/values; query i of sequence b is the token at position
 * kv_lens[b] + i and attends to rows [0, kv_lens[b] + i] (causal over the
 * whole sequence). kv_lens[b] += Sq afterwards when `advance` is non-zero.
 * strides as q3_flash_attention's (k/v = the caches). Keys past cap are never
 * read. The reference's past_kv form runs such a chunk non-causally
 * (is_causal = Sq == Sk); this entry point is for the in-place cache. */
int q3_flash_attention_cache(const void* q, const void* k_cache, const void* v_cache, int* kv_lens, void* o,
                             int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t cap, int64_t D,
                             const int64_t* strides, float scale, int advance, int dtype, void* stream);

/* Decode step over a ragged KV cache: the Sq = 1 case of the same op
 * (modules/attention.py:89-96) without the torch.cat cache growth. q (B, Hq, D)
 * strides [qb, qh]; k/v cache (B, Hkv, cap, D) strides [b, h, s]; o (B, Hq, D)
 * strides [ob, oh]; strides = [qb, qh, kb, kh, ks, vb, vh, vs, ob, oh].
 * Sequence b attends to cache rows [0, kv_lens[b]) (int32 on the device);
 * max_len >= every kv_lens[b]. */
int64_t q3_decode_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t D);
int q3_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int* kv_lens, void* o,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len, const int64_t* strides,
                        float scale, int dtype, void* workspace, int64_t workspace_bytes, void* stream);

/* The decode step of CudaFullAttention.forward with a KV cache
 * (modules/attention.py:89-96: cache concat, then attention of the new token):
 * the new token's K/V row is already at cache row kv_lens[b]; sequence b
 * attends to rows [0, kv_lens[b] + 1) and kv_lens[b] is then incremented in
 * place (the reference's torch.cat growth of the cache). Same arguments and
 * workspace as q3_decode_attention; max_len >= every kv_lens[b] + 1. */
int q3_decode_attention_step(const void* q, const void* k_cache, const void* v_cache, int* kv_lens, void* o,
                             int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len, const int64_t* strides,
                             float scale, int dtype, void* workspace, int64_t workspace_bytes, void* stream);

/* Paged KV cache (no counterpart in the reference, whose cache grows by
 * torch.cat, modules/attention.py:89-92; serves the preallocated, optionally
 * paged cache of the decode loop): each KV head's rows live in pages of page_rows rows (a multiple of
 * 32) in pools k_pages / v_pages (num_pages, Hkv, page_rows, D); cache row r
 * of sequence b is row r % page_rows of page block_table[b * max_pages +
 * r / page_rows] (int32 on the device). A page id outside [0, num_pages)
 * reads as zero rows / drops the write and sets bit 1 of *status (a device
 * int32, or null; never cleared here).
 *
 * q3_qk_norm_rope_paged: q3_qk_norm_rope whose k/v outputs are the page pools,
 * rows appended at cache rows kv_lens[b] + s (< max_pages * page_rows).
 * strides = q3_qk_norm_rope's, with the k/v output (b, s, h) strides replaced
 * by (page, row, head) strides of the pools. */
int q3_qk_norm_rope_paged(const void* q_in, const void* k_in, const void* v_in, void* q_out, void* k_pages,
                          void* v_pages, const void* q_weight, const void* k_weight, const int* positions,
                          const float* inv_freq, const int* block_table, int64_t max_pages, int64_t page_rows,
                          int64_t num_pages, const int* kv_lens, int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                          int64_t D, const int64_t* section, float eps, const int64_t* strides, int dtype,
                          int* status, void* stream);

/* Decode attention over a paged cache: sequence b attends to its cache rows
 * [0, kv_lens[b] + advance) (advance = 1: the step, whose new K/V row is
 * already appended; kv_lens[b] is then incremented in place). strides = [qb,
 * qh, k page, kh, ks, v page, vh, vs, ob, oh]; workspace as
 * q3_decode_attention with max_len = max_pages * page_rows. bf16, D = 128,
 * Hq / Hkv <= 32, B <= 1024 only (else Q3_ERR_UNSUPPORTED). */
int q3_decode_attention_paged(const void* q, const void* k_pages, const void* v_pages, const int* block_table,
                              int64_t max_pages, int64_t page_rows, int64_t num_pages, int* kv_lens, int advance,
                              void* o, int64_t B, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides,
                              float scale, int dtype, void* workspace, int64_t workspace_bytes, int* status,
                              void* stream);

/* q3_flash_attention_cache over a paged cache (no counterpart in the
 * reference, whose cache grows by torch.cat, modules/attention.py:89-96): cache
 * row r of sequence b is row r % page_rows of page block_table[b * max_pages +
 * r / page_rows] of k_pages / v_pages (num_pages, Hkv, page_rows, D), read in
 * place. strides = [qb, qh, qs, k page, kh, ks, v page, vh, vs, ob, oh, os].
 * Same kernel and arithmetic as q3_flash_attention_cache (bit-identical
 * output). bf16, D = 128, max_pages <= 512, fewer
 * than 65535 pages, each pool under 2 GiB; else Q3_ERR_UNSUPPORTED. A page id
 * outside [0, num_pages) reads as zero rows and sets bit 1 of *status. */
int q3_flash_attention_cache_paged(const void* q, const void* k_pages, const void* v_pages, const int* block_table,
                                   int64_t max_pages, int64_t page_rows, int64_t num_pages, int* kv_lens, void* o,
                                   int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D, const int64_t* strides,
                                   float scale, int advance, int dtype, int* status, void* stream);

/* q3_decode_attention_step without a workspace argument, for callers that
 * cannot allocate (code under HIP-graph capture, tight serving loops). No
 * counterpart in the reference. The workspace lives in a static device array
 * of q3_decode_attention_step_noalloc_max_bytes() bytes (32 MiB), one per GPU,
 * held until the process ends; a request whose workspace
 * (q3_decode_attention_workspace_bytes) exceeds it returns Q3_ERR_SCRATCH
 * before touching the device. All calls on one GPU share the array: calls
 * that may run at the same time on one GPU race (stream-ordered calls are
 * safe; no call relies on its previous contents). The stream must belong to
 * the current device. Makes no allocation of any kind. */
int64_t q3_decode_attention_step_noalloc_max_bytes(void);
int q3_decode_attention_step_noalloc(const void* q, const void* k_cache, const void* v_cache, int* kv_lens, void* o,
                                     int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len,
                                     const int64_t* strides, float scale, int dtype, void* stream);

/* ---------------------------------------------------------------- model edges and vision-tower glue
 * q3_embedding replaces embedding_forward(Tensor ids, Tensor weight)
 * (csrc/embedding_op.cpp, csrc/embedding_op.cu:40-70, kernels/embedding.py):
 * out (n, dim) = weight[ids] for int64 ids; an id outside [0, rows) gives a
 * zero row and sets bit 0 of *status (a device int32, or null).
 *
 * Images are described by an (n_img, 4) int32 table of (t, h, w, first token)
 * in patch units (first token = running sum of t*h*w), passed both on the
 * device (`images`, read by the kernel) and on the host (`images_host`,
 * validated before any launch: h and w multiples of `merge`, consistent
 * first tokens). Tokens of an image are frame-major, then merge blocks of
 * merge x merge patches row-major, then the patches of a block row-major (the
 * Qwen2/3-VL processor's order).
 * q3_vision_rope_tables replaces CudaVisionTower._rot_pos_emb and the cos/sin
 * of its forward (models/common.py:85-120, 192-195): cos/sin (total, head_dim)
 * fp32 with angles row * inv_freq[j] (j < head_dim/4) and col * inv_freq[j -
 * head_dim/4] (j < head_dim/2), repeated over both halves; inv_freq (head_dim/4)
 * fp32 on the device.
 * q3_vision_pos_embed replaces CudaVisionTower._fast_pos_embed_interpolate and
 * the add that follows it (models/common.py:122-174, 180-181): y = x +
 * bilinear(table) with table (grid_side^2, hidden), coordinates
 * linspace(0, grid_side - 1, h or w) per image; x and y (total, hidden) may
 * alias. */
int q3_embedding(const int64_t* ids, const void* weight, void* out, int64_t n, int64_t rows, int64_t dim, int dtype,
                 int* status, void* stream);
int q3_vision_rope_tables(const int* images, const int* images_host, int64_t n_img, int64_t merge, int64_t head_dim,
                          const float* inv_freq, float* cos_out, float* sin_out, void* stream);
int q3_vision_pos_embed(const int* images, const int* images_host, int64_t n_img, int64_t merge, int64_t grid_side,
                        const void* table, const void* x, void* y, int64_t hidden, int dtype, void* stream);

/* ---------------------------------------------------------------- MoE
 * Router of CudaSparseMoE.forward (modules/moe.py:60-65): softmax over the
 * (bf16) logits (softmax_forward, csrc/softmax_op.cpp:7), top-k
 * (topk_forward, csrc/moe_routing_op.cpp:10; lowest index wins ties),
 * renormalise and cast to bf16. top_idx (T, k) int32; top_w (T, k) bf16;
 * top_p (T, k) fp32 selected probabilities or null. */
int q3_moe_route(const void* logits, int* top_idx, void* top_w, float* top_p, int64_t T, int64_t E, int64_t k,
                 int norm, void* stream);

/* The router whole (modules/moe.py:60-65 with the gate projection of
 * modules/moe.py:59, matmul_forward, csrc/matmul_op.cpp:10): logits (T, E)
 * bf16 = x (T, H) . gate_w (E, H)^T, computed as fp32 partial products over
 * K splits (q3_moe_router_workspace_bytes: splits x T x E fp32) summed in
 * split order and rounded once, then q3_moe_route on those logits. For
 * prefill-sized T, where a (T, 128) output has too few tiles to occupy the
 * GPU (4096 x 128: 32 tiles). bf16 only; H a multiple of 8, x and gate_w
 * 16-byte aligned. */
int64_t q3_moe_router_workspace_bytes(int64_t T, int64_t H, int64_t E);
int q3_moe_router(const void* x, const void* gate_w, void* logits, int* top_idx, void* top_w, float* top_p,
                  int64_t T, int64_t H, int64_t E, int64_t k, int norm, void* workspace, int64_t workspace_bytes,
                  void* stream);

/* Expert dispatch, SwiGLU experts and combine of CudaSparseMoE.forward
 * (modules/moe.py:70-83): replaces the per-expert loop of matmul_forward,
 * swiglu_forward and index_add_forward (csrc/moe_routing_op.cpp:11) with a
 * permute + two grouped GEMMs + an expert-ordered combine. x (T, H);
 * gate_up (E, 2I, H); down (E, H, I); out (T, H) (+ residual (T, H) or null). */
int64_t q3_moe_experts_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k);
int q3_moe_experts(const void* x, const void* gate_up, const void* down, const int* top_idx, const void* top_w,
                   const void* residual, void* out, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                   void* workspace, int64_t workspace_bytes, void* stream);

/* The dispatch step of q3_moe_experts on its own: the per-expert token
 * lists that CudaSparseMoE.forward builds with `(top_idx == e).nonzero()` for
 * each expert e (modules/moe.py:70-76). Rows of expert e are
 * [offsets[e], offsets[e + 1]) (offsets (E + 1) int32, offsets[0] = 0); within
 * them the (token, slot) entries routed to e in ascending (token, slot) order:
 * sorted_token (T * k) int32 and sorted_w (T * k) bf16 (the entry's routing
 * weight). pos_of (T, k) int32 is the inverse (the row of each entry). Ids
 * outside [0, E) are not dispatched (their pos_of entry is left unwritten).
 * Workspace: q3_moe_permute_workspace_bytes. */
int64_t q3_moe_permute_workspace_bytes(int64_t T, int64_t E, int64_t k);
int q3_moe_permute(const int* top_idx, const void* top_w, int* offsets, int* sorted_token, void* sorted_w,
                   int* pos_of, int64_t T, int64_t E, int64_t k, void* workspace, int64_t workspace_bytes,
                   void* stream);

/* Deterministic target[idx[i]] += src[i] (in place): replaces
 * index_add_forward(Tensor(a!) target, Tensor source, Tensor index)
 * (csrc/moe_routing_op.cpp:11). Each target row adds its sources in ascending
 * i in fp32, starting from the target value, and rounds to dtype once (the
 * semantics of torch's index_add_, kernels/moe_routing.py:111-115).
 * idx int64; entries outside [0, n_target) are skipped and set bit 0 of
 * *status (a device int32, or null), which the call never clears: the index
 * check needs no host synchronisation (the reference's kernel,
 * csrc/moe_routing_op.cu:90-102, writes out of bounds instead). */
int64_t q3_index_add_workspace_bytes(int64_t n_src, int64_t n_target);
int q3_index_add(void* target, const void* src, const int64_t* idx, int64_t n_src, int64_t n_target, int64_t D,
                 int dtype, void* workspace, int64_t workspace_bytes, int* status, void* stream);

/* ---------------------------------------------------------------- the rest of the op namespace
 * q3_sigmoid_mul replaces sigmoid_mul_forward(Tensor x, Tensor gate)
 * (csrc/sigmoid_mul_op.cpp:9, csrc/sigmoid_mul_op.cu:5-16): y = x * sigmoid(gate)
 * in fp32, one rounding; n contiguous elements.
 * q3_cross_entropy replaces cross_entropy_forward(Tensor logits, Tensor targets,
 * int ignore_index) -> [loss_per_token, lse] (csrc/cross_entropy_op.cpp:11,
 * csrc/cross_entropy_op.cu:10-62) and the mean that kernels/cross_entropy.py:60-64
 * takes after it: logits (N, V) contiguous, targets (N) int64; loss_per_token
 * and lse (N) fp32 (both 0 for a target equal to ignore_index), *loss (fp32) =
 * sum(loss_per_token) / max(#valid targets, 1), *n_valid (int32, or null) = the
 * count. A target outside [0, V) other than ignore_index counts as ignored and
 * sets bit 0 of *status (a device int32, or null). Nothing synchronises. */
int q3_sigmoid_mul(const void* x, const void* gate, void* y, int64_t n, int dtype, void* stream);
int q3_cross_entropy(const void* logits, const int64_t* targets, float* loss_per_token, float* lse, float* loss,
                     int* n_valid, int64_t N, int64_t V, int64_t ignore_index, int dtype, int* status, void* stream);

/* ---------------------------------------------------------------- backward
 * Gradients of the ops the reference wraps in torch.autograd.Function. Every
 * reduction runs in a fixed order (no atomics): results are bitwise
 * reproducible. fp32 and bf16; fp32 math, one rounding per output.
 *
 * Elementwise (n contiguous elements), replacing
 *   sigmoid_mul_backward(x, gate, grad_out) -> [gx, gg] (csrc/sigmoid_mul_op.cpp:10, .cu:18-34),
 *   swiglu_backward(gate, up, grad_out) -> [gg, gu] (csrc/swiglu_op.cpp:10, .cu:20-39),
 *   gelu_tanh_backward(x, grad_out) (csrc/gelu_tanh_op.cpp:8, .cu:20-36).
 * Softmax rows (rows, cols): gx = out * (dy - sum(out * dy)), replacing
 *   softmax_backward(out, grad_out) (csrc/softmax_op.cpp:8, .cu:55-88). */
int q3_sigmoid_mul_backward(const void* x, const void* gate, const void* grad_out, void* grad_x, void* grad_gate,
                            int64_t n, int dtype, void* stream);
int q3_swiglu_backward(const void* gate, const void* up, const void* grad_out, void* grad_gate, void* grad_up,
                       int64_t n, int dtype, void* stream);
int q3_gelu_tanh_backward(const void* x, const void* grad_out, void* grad_x, int64_t n, int dtype, void* stream);
int q3_softmax_backward(const void* out, const void* grad_out, void* grad_x, int64_t rows, int64_t cols, int dtype,
                        void* stream);

/* RMSNorm / LayerNorm rows (rows, cols), contiguous. q3_rmsnorm_backward
 * replaces rmsnorm_backward(x, weight, grad_out, eps) -> [gx, gw]
 * (csrc/rmsnorm_op.cpp:11, csrc/rmsnorm_op.cu:63-130,158-186);
 * q3_layernorm_backward has no CUDA counterpart (the reference differentiates
 * F.layer_norm with torch autograd, kernels/layernorm.py:35-52). grad_weight /
 * grad_bias may be null; when set, the call needs a workspace of
 * q3_norm_backward_workspace_bytes(rows, cols) (per-block partial column sums,
 * summed in block order). */
int64_t q3_norm_backward_workspace_bytes(int64_t rows, int64_t cols);
int q3_rmsnorm_backward(const void* x, const void* weight, const void* grad_out, void* grad_x, void* grad_weight,
                        int64_t rows, int64_t cols, float eps, int dtype, void* workspace, int64_t workspace_bytes,
                        void* stream);
int q3_layernorm_backward(const void* x, const void* weight, const void* grad_out, void* grad_x, void* grad_weight,
                          void* grad_bias, int64_t rows, int64_t cols, float eps, int dtype, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* Cross entropy, replacing cross_entropy_backward(logits, targets, lse,
 * grad_scale, ignore_index) (csrc/cross_entropy_op.cpp:12, .cu:66-116):
 * grad = (exp(logits - lse) - onehot(target)) * (*grad_loss) / max(*n_valid, 1),
 * zero rows for ignored targets; grad_loss (fp32) and n_valid (int32, from
 * q3_cross_entropy) are read on the device. */
int q3_cross_entropy_backward(const void* logits, const int64_t* targets, const float* lse, const float* grad_loss,
                              const int* n_valid, void* grad_logits, int64_t N, int64_t V, int64_t ignore_index,
                              int dtype, void* stream);

/* Top-k: grad_x (rows, cols) = grad_vals (rows, k) scattered to idx (int64),
 * zeros elsewhere (the reference's scatter_add_, kernels/moe_routing.py:44-52). */
int q3_topk_backward(const void* grad_vals, const int64_t* idx, void* grad_x, int64_t rows, int64_t cols, int64_t k,
                     int dtype, void* stream);

/* (E, R, C) -> (E, C, R), contiguous (operand layouts of the GEMM backward). */
int q3_transpose(const void* a, void* b, int64_t E, int64_t R, int64_t C, int dtype, void* stream);

/* GEMM backward, replacing matmul_backward(x, weight, grad_out,
 * needs_bias_grad) -> [gx, gw, gb] (csrc/matmul_op.cpp:13, .cu:151-233): for
 * y = x . w^T (+ b) with x (M, K), w (N, K), dy (M, N), all contiguous:
 * gx = dy . w (M, K), gw = dy^T . x (N, K), gb = sum over rows of dy (N); any of
 * the three may be null. The operands are transposed into `workspace`
 * (q3_matmul_backward_workspace_bytes) and multiplied by q3_matmul, which may
 * use `gemm_ws` as q3_matmul's workspace (zero-filled before first use, as
 * there; size at least q3_matmul_workspace_bytes of both products). */
int64_t q3_matmul_backward_workspace_bytes(int64_t M, int64_t N, int64_t K, int dtype);
int q3_matmul_backward(const void* x, const void* w, const void* dy, void* gx, void* gw, void* gb, int64_t M,
                       int64_t N, int64_t K, int dtype, void* workspace, int64_t workspace_bytes, void* gemm_ws,
                       int64_t gemm_ws_bytes, void* stream);

/* Batched GEMM backward (the reference's _BatchedGemmFunction,
 * kernels/moe_routing.py:146-181): for y[e] = x[e] . w[e]^T with x (E, M, K),
 * w (E, N, K), dy (E, M, N): gx[e] = dy[e] . w[e], gw[e] = dy[e]^T . x[e];
 * either may be null. */
int64_t q3_batched_gemm_backward_workspace_bytes(int64_t E, int64_t M, int64_t N, int64_t K, int dtype);
int q3_batched_gemm_backward(const void* x, const void* w, const void* dy, void* gx, void* gw, int64_t E, int64_t M,
                             int64_t N, int64_t K, int dtype, void* workspace, int64_t workspace_bytes,
                             void* stream);

/* Flash-attention backward, replacing flash_attention_backward(q, k, v, o, lse,
 * grad_o, scale, is_causal, num_kv_groups) -> [dq, dk, dv]
 * (csrc/flash_attention_op.cpp:15, .cu:235-390): q, o, grad_out, grad_q
 * (B, Hq, Sq, D), k, v, grad_k, grad_v (B, Hkv, Sk, D), all contiguous; lse
 * (B, Hq, Sq) fp32 natural-log row log-sum-exp of the scaled scores (as
 * q3_flash_attention writes it); D <= 128; causal masks key j > query i.
 * Workspace: q3_flash_attention_backward_workspace_bytes (one fp32 per query
 * row). */
int64_t q3_flash_attention_backward_workspace_bytes(int64_t B, int64_t Hq, int64_t Sq);
int q3_flash_attention_backward(const void* q, const void* k, const void* v, const void* o, const float* lse,
                                const void* grad_out, void* grad_q, void* grad_k, void* grad_v, int64_t B, int64_t Hq,
                                int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, float scale, int is_causal,
                                int dtype, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* Q3VL_H */
