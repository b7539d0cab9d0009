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

Supported: head_dim 64 or 128, any q_len.  Items of up to 64 rows per KV head, (Hq/Hkv) *
max_seqlen_q <= 64 (speculative verify and decode), take the tuned path; longer ones (the
prefill chunks engine/engine.py:414-420 mixes into the same batch) run in query windows of
64/(Hq/Hkv) rows, one block per window and KV head -- correct at any length, not tuned.
"""
import math

import torch

from . import _lib

__all__ = ["flash_attn_varlen_func", "paged_attention", "paged_attention_qkv",
           "qkv_attention_supported", "workspace_bytes"]

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


def qkv_attention_supported(kv_cache_dtype, batch, num_heads, num_kv_heads, head_dim,
                            max_seqlen_q, max_seqlen_k) -> bool:
    """Whether paged_attention_qkv takes this launch shape (coopt_verify_attention_qkv)."""
    code = _lib.DT_I8 if kv_cache_dtype == "int8" else _lib.DT_BF16
    return bool(_lib.load().coopt_verify_attention_qkv_supported(
        code, batch, num_heads, num_kv_heads, head_dim, int(max_seqlen_q), int(max_seqlen_k)))


def paged_attention_qkv(qkv, positions, cos, sin, slot_mapping, k_cache, v_cache, cu_seqlens_q,
                        seq_lens, block_table, max_seqlen_q, max_seqlen_k, num_heads,
                        softmax_scale=None, kv_cache_dtype="auto", k_scale=None, v_scale=None,
                        out=None, workspace=None):
    """kv_cache.qkv_rope_and_cache followed by paged_attention in one launch (engine/model.py:
    238-247): the qkv projection's output (bf16 [T, (Hq + 2 Hkv) D] or its
    fused.LinearPartials), neox RoPE on q and k, k and v written to the paged cache, and the
    verification attention of q over it.  Same outputs and cache contents, bit for bit.
    Row j of sequence b must write key position seq_lens[b] - q_len_b + j (or slot -1), as a
    step's new tokens do; shapes where qkv_attention_supported() is False raise ValueError."""
    from .fused import LinearPartials

    _lib.require_cuda(positions, cos, sin, slot_mapping, k_cache, v_cache, cu_seqlens_q,
                      seq_lens, block_table)
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride() or \
            k_cache.dim() != 4 or k_cache.stride(-1) != 1:
        raise ValueError("k/v caches must be [num_blocks, block_size, Hkv, D] alike")
    NB, bs, Hkv, D = k_cache.shape
    Hq = int(num_heads)
    width = (Hq + 2 * Hkv) * D
    part = qkv if isinstance(qkv, LinearPartials) else None
    if part is not None:
        if part.n != width:
            raise ValueError(f"partials are {part.n} wide, expected {width}")
        T, dev, qkv_t = part.rows, part.device, None
    else:
        _lib.require_cuda(qkv)
        if qkv.dtype != torch.bfloat16 or qkv.dim() != 2 or qkv.shape[1] != width or qkv.stride(1) != 1:
            raise ValueError(f"qkv must be bf16 [T, {width}] with contiguous rows")
        T, dev, qkv_t = qkv.shape[0], qkv.device, qkv
    B = seq_lens.numel()
    if cu_seqlens_q.numel() != B + 1:
        raise ValueError("cu_seqlens_q must have batch + 1 entries")
    for name, t in (("cu_seqlens_q", cu_seqlens_q), ("seq_lens", seq_lens),
                    ("block_table", block_table)):
        if t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32")
    if block_table.dim() != 2 or block_table.shape[0] != B or block_table.stride(1) != 1:
        raise ValueError("block_table must be [batch, width] int32, row-major")
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != T:
        raise ValueError("slot_mapping must be int64 with one entry per row")
    if positions.dtype != torch.int64 or positions.numel() != T:
        raise ValueError("positions must be int64 with one entry per row")
    if cos.shape != sin.shape or cos.stride() != sin.stride() or cos.shape[1] < D // 2 or \
            cos.dtype != torch.bfloat16 or cos.stride(1) != 1:
        raise ValueError("cos/sin tables must be bf16 [max_pos, >= D/2] alike")
    if kv_cache_dtype == "auto":
        if k_cache.dtype != torch.bfloat16:
            raise ValueError("'auto' caches are bf16")
        code, ks, vs, sstr = _lib.DT_BF16, None, None, (0, 0, 0)
    elif kv_cache_dtype == "int8":
        if k_cache.dtype != torch.int8 or k_scale is None or v_scale is None or \
                k_scale.shape != (NB, bs, Hkv) or k_scale.dtype != torch.float16 or \
                v_scale.shape != k_scale.shape or v_scale.stride() != k_scale.stride():
            raise ValueError("'int8' caches need fp16 [num_blocks, block_size, Hkv] scale caches alike")
        _lib.require_cuda(k_scale, v_scale)
        code, ks, vs, sstr = _lib.DT_I8, k_scale, v_scale, k_scale.stride()
    else:
        raise ValueError(f"kv_cache_dtype must be 'auto' or 'int8', got {kv_cache_dtype!r}")
    if not qkv_attention_supported(kv_cache_dtype, B, Hq, Hkv, D, max_seqlen_q, max_seqlen_k):
        raise ValueError("shape not supported by the fused call; use qkv_rope_and_cache and "
                         "paged_attention")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty((T, Hq, D), dtype=torch.bfloat16, device=dev)
    elif out.shape != (T, Hq, D) or out.dtype != torch.bfloat16 or out.stride(-1) != 1:
        raise ValueError("out must be bf16 [T, Hq, D] with contiguous D")
    if B == 0 or T == 0:
        return out
    need = workspace_bytes(B, Hq, Hkv, D, int(max_seqlen_q), int(max_seqlen_k))
    if workspace is None:
        workspace = _WS.get(need, dev)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} "
                         f"bytes, {need} needed")
    positions, slot_mapping = positions.contiguous(), slot_mapping.contiguous()
    cu, sl = cu_seqlens_q.contiguous(), seq_lens.contiguous()
    cs = k_cache.stride()
    _lib.check(_lib.load().coopt_verify_attention_qkv(
        code, _lib.ptr(qkv_t), 0 if qkv_t is None else qkv_t.stride(0),
        None if part is None else _lib.ptr(part.buf), 0 if part is None else part.ks,
        0 if part is None else part.rows_padded * part.n,
        _lib.ptr(positions), _lib.ptr(cos), _lib.ptr(sin), cos.stride(0), cos.shape[0],
        _lib.ptr(slot_mapping), _lib.ptr(k_cache), _lib.ptr(v_cache), cs[0], cs[1], cs[2],
        _lib.ptr(ks), _lib.ptr(vs), sstr[0], sstr[1], sstr[2], _lib.ptr(block_table),
        block_table.stride(0), _lib.ptr(cu), _lib.ptr(sl), B, Hq, Hkv, D, bs, NB,
        int(max_seqlen_q), int(max_seqlen_k), float(softmax_scale), _lib.ptr(out),
        out.stride(0), out.stride(1), _lib.ptr(workspace),
        workspace.numel() * workspace.element_size(), _lib.stream_handle(dev)),
        "coopt_verify_attention_qkv")
    return out


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, max_seqlen_q, seqused_k, max_seqlen_k,
                           softmax_scale=None, causal=True, block_table=None, fa_version=2,
                           k_scale=None, v_scale=None, out=None, workspace=None):
    """Keyword-compatible with the vLLM call the reference makes (engine/model.py:244-247)."""
    if not causal:
        raise ValueError("only causal=True is supported (the reference always passes it)")
    if block_table is None:
        raise ValueError("block_table is required: this is the paged-KV path")
    del fa_version
    return paged_attention(q, k, v, cu_seqlens_q, seqused_k, block_table, max_seqlen_q,
                           max_seqlen_k, softmax_scale, k_scale, v_scale, out, workspace)
