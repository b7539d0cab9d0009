"""MI355X-native speculative verify/accept path and paged KV cache.

gfx950 HIP kernels (libcoopt_amd.so, C ABI in include/coopt_amd.h) behind the Python call
surface of mohsinmubarak/iitj-llm-coopt's engine:
  spec_decode   sample / verify / batched accept      (engine/spec_decode.py)
  kv_cache      quantize / dequantize / paged write   (engine/kv_tier_manager.py, model.py:242)
  kv_tier       KVTierManager swap_out / swap_in      (engine/kv_tier_manager.py:44-131)
  kv_blocks     block-major KV buffer, batched block migration copy (engine/elastic.py:74-77,
                131; engine/block_manager.py:165-187)
  attention     flash_attn_varlen_func-compatible paged verification attention (model.py:244)
  block_manager BlockManager slot / block-table contract (engine/block_manager.py)
  batch         WorkItem / Batch / build_batch varlen layout (engine/batch.py)
"""
from . import _lib  # noqa: F401  (imports torch first, then binds the library lazily)
from . import fused  # noqa: F401  (rms_norm / rope_ / silu_and_mul forward stages)
from .attention import (flash_attn_varlen_func, paged_attention, paged_attention_qkv,
                        qkv_attention_supported)
from .batch import Batch, WorkItem, build_batch, build_padded_batch
from .block_manager import BlockManager, OutOfBlocks
from .kv_blocks import allocate_block_major_kv, copy_blocks, migrate_out_of
from .kv_cache import (allocate_kv_cache, dequantize, qkv_rope_and_cache, quantize,
                       reshape_and_cache_flash)
from .kv_tier import (KVTierManager, SwappedKV, swap_in_blocks, swap_in_caches, swap_out_blocks,
                      swap_out_caches)
from .spec_decode import AcceptResult, accept, sample, softmax, verify

__all__ = [
    "flash_attn_varlen_func", "paged_attention", "paged_attention_qkv", "qkv_attention_supported", "Batch", "WorkItem", "build_batch",
    "build_padded_batch", "BlockManager", "OutOfBlocks", "allocate_kv_cache", "dequantize",
    "quantize", "reshape_and_cache_flash", "AcceptResult", "accept", "sample", "softmax",
    "verify", "KVTierManager", "SwappedKV", "swap_in_blocks", "swap_out_blocks",
    "allocate_block_major_kv", "copy_blocks", "migrate_out_of", "qkv_rope_and_cache",
    "swap_out_caches", "swap_in_caches",
]
