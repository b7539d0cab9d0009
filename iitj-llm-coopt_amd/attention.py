"""Paged GQA verification attention on gfx950.

Drop-in for the call at engine/model.py:244-247 (and :204-207):
    flash_attn_varlen_func(q=q, k=k_cache, v=v_cache, cu_seqlens_q=..., max_seqlen_q=...,
                           seqused_k=seq_lens, max_seqlen_k=..., softmax_scale=...,
                           causal=True, block_table=..., fa_version=2)
Sequence b owns query rows cu_seqlens_q[b]:cu_seqlens_q[b+1] and seq_lens[b] cached keys
(its new tokens' K/V already written, engine/model.py:242 precedes :244); query j attends to
keys [0, seq_len - q_len + j] (causal mask aligned bottom-right, engine/model.py:8-10).
For INT8 caches (codes + fp16 per-token scales from reshape_and_cache_flash(..., "int8"))
pass k_scale/v_scale; dequantisation is fused into the kernel.

Supported: head_dim 64 or 128, (Hq/Hkv) * max_seqlen_q <= 64 (speculative verify and decode
shapes); prefill-sized queries are outside this kernel's scope.
"""
import math

import torch

from . import _lib

__all__ = ["flash_attn_varlen_func", "paged_attention", "workspace_bytes"]

_WS = _lib.WorkspaceCache()


def workspace_bytes(batch: int, num_heads: int, num_kv_heads: int, head_dim: int,
                    max_seqlen_q: int, max_seqlen_k: int) -> int:
    return int(_lib.load().coopt_verify_attention_workspace(batch, num_heads, num_kv_heads,
                                                            head_dim, max_seqlen_q, max_seqlen_k))


def paged_attention(q, k_cache, v_cache, cu_seqlens_q, seq_lens, block_table, max_seqlen_q,
                    max_seqlen_k, softmax_scale=None, k_scale=None, v_scale=None, out=None,
                    workspace=None):
    """out [T, Hq, D] bf16 = causal paged attention; see the module docstring."""
    _lib.require_cuda(q, k_cache, v_cache, cu_seqlens_q, seq_lens, block_table)
    if q.dtype != torch.bfloat16 or q.dim() != 3 or q.stride(-1) != 1:
        raise ValueError("q must be bf16 [T, Hq, D] with contiguous D")
    T, Hq, D = q.shape
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride() or \
            k_cache.dim() != 4 or k_cache.stride(-1) != 1:
        raise ValueError("k/v caches must be [num_blocks, block_size, Hkv, D] alike")
    NB, bs, Hkv, cD = k_cache.shape
    if cD != D or Hq % Hkv:
        raise ValueError(f"q {tuple(q.shape)} does not match cache {tuple(k_cache.shape)}")
    B = seq_lens.numel()
    if cu_seqlens_q.numel() != B + 1:
        raise ValueError("cu_seqlens_q must have batch + 1 entries")
    for name, t in (("cu_seqlens_q", cu_seqlens_q), ("seq_lens", seq_lens),
                    ("block_table", block_table)):
        if t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32")
    if block_table.dim() != 2 or block_table.shape[0] != B or block_table.stride(1) != 1:
        raise ValueError("block_table must be [batch, width] int32, row-major")
    if k_cache.dtype == torch.bfloat16:
        code, ks, vs, sstr = _lib.DT_BF16, None, None, (0, 0, 0)
    elif k_cache.dtype == torch.int8:
        if k_scale is None or v_scale is None:
            raise ValueError("INT8 caches need k_scale and v_scale")
        if k_scale.shape != (NB, bs, Hkv) or k_scale.dtype != torch.float16 or \
                v_scale.shape != k_scale.shape or v_scale.stride() != k_scale.stride():
            raise ValueError("scale caches must be fp16 [num_blocks, block_size, Hkv] alike")
        _lib.require_cuda(k_scale, v_scale)
        code, ks, vs, sstr = _lib.DT_I8, k_scale, v_scale, k_scale.stride()
    else:
        raise ValueError(f"unsupported cache dtype {k_cache.dtype}")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty((T, Hq, D), dtype=torch.bfloat16, device=q.device)
    elif out.shape != (T, Hq, D) or out.dtype != torch.bfloat16 or out.stride(-1) != 1:
        raise ValueError("out must be bf16 [T, Hq, D] with contiguous D")
    if B == 0 or T == 0:
        return out
    cu = cu_seqlens_q.contiguous()
    sl = seq_lens.contiguous()
    lib = _lib.load()
    need = workspace_bytes(B, Hq, Hkv, D, int(max_seqlen_q), int(max_seqlen_k))
    if workspace is None:
        workspace = _WS.get(need, q.device)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} "
                         f"bytes, {need} needed")
    cs = k_cache.stride()
    _lib.check(lib.coopt_verify_attention(
        code, _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k_cache), _lib.ptr(v_cache),
        cs[0], cs[1], cs[2], _lib.ptr(ks), _lib.ptr(vs), sstr[0], sstr[1], sstr[2],
        _lib.ptr(block_table), block_table.stride(0), _lib.ptr(cu), _lib.ptr(sl),
        B, Hq, Hkv, D, bs, NB, int(max_seqlen_q), int(max_seqlen_k), float(softmax_scale),
        _lib.ptr(out), out.stride(0), out.stride(1), _lib.ptr(workspace),
        workspace.numel() * workspace.element_size(), _lib.stream_handle(q.device)),
        "coopt_verify_attention")
    return out


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, max_seqlen_q, seqused_k, max_seqlen_k,
                           softmax_scale=None, causal=True, block_table=None, fa_version=2,
                           k_scale=None, v_scale=None, out=None):
    """Keyword-compatible with the vLLM call the reference makes (engine/model.py:244-247)."""
    if not causal:
        raise ValueError("only causal=True is supported (the reference always passes it)")
    if block_table is None:
        raise ValueError("block_table is required: this is the paged-KV path")
    del fa_version
    return paged_attention(q, k, v, cu_seqlens_q, seqused_k, block_table, max_seqlen_q,
                           max_seqlen_k, softmax_scale, k_scale, v_scale, out)
