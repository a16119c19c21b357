"""CPU oracle for the Qwen3-VL operator layer — TEST INFRASTRUCTURE ONLY.

This package restates, on CPU in float32, the reference's own PyTorch
implementations of every op and module on the hot path
(`cuda_qwen3_vl/kernels/*.py` fallbacks and `cuda_qwen3_vl/modules/*.py`
compositions of luozoupi/Qwen3_5_VL_CUDA_CUSTOM). Each function cites the
reference file:line it follows (paths relative to the reference's
`CUDA_qwen3_5-main/CUDA_qwen3_5-main/` root).

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only as the checker or the timed CPU
baseline. The product (`qwen3_5_vl_cuda_custom_amd`) never imports it and has
no CPU fallback.

Pinning (how each function is checked independently of its own formula):
  ops.linear / batched_gemm / conv3d_patch   numpy float64 brute force (tests/test_oracle_pins.py)
  ops.flash_attention (+ decode form)        numpy float64 per-row softmax loop; causal row 0 == v0
  ops.chunk_attention                        numpy float64 masked loop; equals the last rows of causal
                                             ops.flash_attention over the whole sequence; offset 0 is causal
  ops.interleave_cos_sin / mrope_cos_sin     per-element closed form with distinct T/H/W positions;
                                             HF Qwen3-VL rotary for identical axes
  ops.rotate_half_apply                      identity at theta=0, per-pair norm preservation, numpy loop
  ops.rmsnorm / layernorm / swiglu / gelu    numpy float64 closed forms; constant-row invariants
  ops.softmax / topk                         numpy float64 softmax; brute-force lexicographic top-k
                                             with planted ties (lowest index wins)
  ops.index_add                              numpy sequential loop; unique-index scatter
  layers.text_decoder_layer                  HF transformers Qwen3VLTextDecoderLayer (fp32, C1 shape)
  layers.sparse_moe                          numpy per-token loop; single-expert reduces to SwiGLU MLP
  layers.vision_block / vision_rope_tables   HF Qwen3VLVisionBlock with cu_seqlens; HF vision position ids
  C1 golden fixture                          tests/golden/c1_layer.npz (regression pin of the whole layer)
"""
