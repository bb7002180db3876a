"""MI355X-native DeepSeek-sparse-attention decode path (gfx950 HIP kernels).

Modules mirror the reference interfaces they replace:
  deep_gemm    - fp8_paged_mqa_logits / get_paged_mqa_logits_metadata / get_num_sms
  deepseek_v4  - topk_transform / topk_transform_ragged
  mla_utils    - topk_indices_to_physical / merge_attention_states
  flash_mla    - flash_mla_with_kvcache (sparse fp8) / get_mla_metadata
  indexer      - the decode selection of Indexer.forward, IndexerCache
  mla_backend  - MlaAttentionBase-compatible sparse MLA backend + "mi355x" tier
  pipeline     - the fused three-launch decode step
The kernels live in libdsa_amd.so (C ABI in include/dsa_amd.h); there is no
CPU fallback.
"""
__version__ = "0.1.0"
