// Host interface of the weight-streaming GEMV (M <= 32 rows: decode
// projections), used by the GEMM entry points in gemm.hip.
#pragma once

#include "gemm_kernels.h"

namespace q3 {

constexpr int kGemvMaxRows = 32;

struct GemvArgs {
  const bf16* X;
  int64_t ldx;
  WeightSegments seg;  // W matrices stacked along the output columns (seg.n >= 1)
  const bf16* W2;      // SwiGLU up weight (seg.w[0] is the gate weight), else null
  const bf16* R;       // residual (M, N) or null
  int64_t ldr;
  bf16* C;
  int64_t ldc;
  int M, N, K;
  int64_t ldw;
  const bf16* nw;  // RMSNorm weight (K) applied to the X rows first (row-owned kernel), or null
  float eps;       // RMSNorm epsilon when nw is set
};

// True when the GEMV path takes the problem (bf16 rows 16-byte aligned,
// segment starts on 128-column tiles, 32-bit buffer offsets).
bool gemv_eligible(const GemvArgs& a);
// Workspace: none where the row-owned kernel runs (M <= 8 or K <= 16384);
// else a fixed 16 KiB region of tile counters (zero before the first call;
// every call leaves it zero) followed by fp32 split-K partials.
int64_t gemv_workspace_bytes(int64_t M, int64_t N, int64_t K, bool swiglu);
int gemv_launch(const GemvArgs& a, void* ws, int64_t ws_bytes, hipStream_t st);

}  // namespace q3
