"""Paged KV cache writes and the symmetric absmax INT8/INT4 codec, on gfx950 kernels.

Drop-in surfaces (reference paths under mohsinmubarak/iitj-llm-coopt):
  quantize(x, bits) / dequantize(q, scale, bits, dtype)   engine/kv_tier_manager.py:21-41
  reshape_and_cache_flash(k, v, k_cache, v_cache, slot_mapping, kv_cache_dtype, k_scale,
                          v_scale)                         engine/model.py:242-243 (vLLM op)
  qkv_rope_and_cache(qkv, positions, cos, sin, ...)        engine/model.py:238-243 in one launch

Cache layouts.  bf16 ("auto"): k_cache/v_cache [num_blocks, block_size, Hkv, D] bf16, possibly
a strided per-layer view of a block-major buffer (engine/elastic.py:74-77).  INT8 ("int8"):
int8 codes of the same shape plus fp16 scales [num_blocks, block_size, Hkv] passed as
k_scale/v_scale -- per (token, head) vector, exactly what quantize(cache[blocks], 8) produces
(engine/kv_tier_manager.py:99; SwappedKV shapes :46-49).
"""
import torch

from . import _lib

__all__ = ["quantize", "dequantize", "reshape_and_cache_flash", "allocate_kv_cache",
           "qkv_rope_and_cache"]


def quantize(x: torch.Tensor, bits: int):
    """x [..., D] -> (q, scale [...]) with symmetric absmax per last-dim vector.

    bits 16 returns (x.clone(), None) like the reference; bits 8 gives int8 codes; bits 4 packs
    two signed nibbles (+8 offset) per uint8, even element in the low nibble.
    """
    if bits == 16:
        return x.clone(), None
    if bits not in (8, 4):
        raise ValueError(f"bits must be 16, 8 or 4, got {bits}")
    _lib.require_cuda(x)
    D = x.shape[-1]
    xc = x.contiguous()
    rows = xc.numel() // D if D else 0
    if bits == 8:
        q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    else:
        if D % 2:
            raise ValueError("INT4 packing needs an even last dimension")
        q = torch.empty((*x.shape[:-1], D // 2), dtype=torch.uint8, device=x.device)
    scale = torch.empty(x.shape[:-1], dtype=torch.float16, device=x.device)
    lib = _lib.load()
    _lib.check(lib.coopt_quantize(bits, _lib.dt_code(x.dtype), _lib.ptr(xc), rows, D,
                                  _lib.ptr(q), _lib.ptr(scale), _lib.stream_handle(x.device)),
               "coopt_quantize")
    return q, scale


def dequantize(q: torch.Tensor, scale, bits: int, dtype=torch.bfloat16):
    """Inverse of quantize: dtype(float(code) * float(scale)) per element."""
    if bits == 16:
        return q
    if bits not in (8, 4):
        raise ValueError(f"bits must be 16, 8 or 4, got {bits}")
    _lib.require_cuda(q, scale)
    qc, sc = q.contiguous(), scale.contiguous()
    D = qc.shape[-1] * (2 if bits == 4 else 1)
    rows = sc.numel()
    out = torch.empty((*qc.shape[:-1], D), dtype=dtype, device=q.device)
    lib = _lib.load()
    _lib.check(lib.coopt_dequantize(bits, _lib.ptr(qc), _lib.ptr(sc), rows, D,
                                    _lib.dt_code(dtype), _lib.ptr(out),
                                    _lib.stream_handle(q.device)), "coopt_dequantize")
    return out


def allocate_kv_cache(num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int,
                      kv_cache_dtype: str = "auto", device="cuda", dtype=torch.bfloat16):
    """One layer's (k_cache, v_cache, k_scale, v_scale); the scales are None for "auto".

    Every tensor has the reference's logical shape -- caches [num_blocks, block_size, Hkv, D]
    (engine/model.py:148-155), INT8 scales [num_blocks, block_size, Hkv] -- as a view of
    head-major storage [num_blocks, Hkv, block_size, ...]: one head's tokens of a block are
    adjacent in HBM, so the verify-attention kernel reads each (block, head) as one contiguous
    run (16 tokens x D codes) instead of D-sized pieces strided by Hkv * D.  The kernels take
    any strides, so caches in the reference's token-major layout work too.
    """
    store = (num_blocks, num_kv_heads, block_size, head_dim)
    if kv_cache_dtype == "auto":
        return (torch.zeros(store, dtype=dtype, device=device).transpose(1, 2),
                torch.zeros(store, dtype=dtype, device=device).transpose(1, 2), None, None)
    if kv_cache_dtype == "int8":
        sstore = (num_blocks, num_kv_heads, block_size)
        return (torch.zeros(store, dtype=torch.int8, device=device).transpose(1, 2),
                torch.zeros(store, dtype=torch.int8, device=device).transpose(1, 2),
                torch.zeros(sstore, dtype=torch.float16, device=device).transpose(1, 2),
                torch.zeros(sstore, dtype=torch.float16, device=device).transpose(1, 2))
    raise ValueError(f"kv_cache_dtype must be 'auto' or 'int8', got {kv_cache_dtype!r}")


def _check_cache_pair(k_cache, v_cache):
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must have the same shape and strides")
    if k_cache.dim() != 4 or k_cache.stride(-1) != 1:
        raise ValueError("caches must be [num_blocks, block_size, Hkv, D] with contiguous D")


def reshape_and_cache_flash(k, v, k_cache, v_cache, slot_mapping, kv_cache_dtype="auto",
                            k_scale=None, v_scale=None):
    """k_cache[slot // bs, slot % bs] = k (and v), in place; slots < 0 are skipped.

    kv_cache_dtype "auto": bf16 caches, k_scale/v_scale ignored (the reference passes fp32
    ones, engine/model.py:129).  "int8": int8 code caches; k_scale/v_scale are the fp16
    [num_blocks, block_size, Hkv] scale caches and each written vector is quantised in the
    same kernel.
    """
    _lib.require_cuda(k, v, k_cache, v_cache, slot_mapping)
    _check_cache_pair(k_cache, v_cache)
    if k.shape != v.shape or k.dim() != 3 or k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("k and v must be [T, Hkv, D] with contiguous D")
    if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("k and v must be bf16")
    T, Hkv, D = k.shape
    NB, bs, cH, cD = k_cache.shape
    if (cH, cD) != (Hkv, D):
        raise ValueError(f"cache heads/dim {(cH, cD)} != k's {(Hkv, D)}")
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != T:
        raise ValueError("slot_mapping must be int64 with one entry per token")
    slot_mapping = slot_mapping.contiguous()
    if kv_cache_dtype == "auto":
        if k_cache.dtype != torch.bfloat16:
            raise ValueError("'auto' caches are bf16")
        code, ks, vs, sstr = _lib.DT_BF16, None, None, (0, 0, 0)
    elif kv_cache_dtype == "int8":
        if k_cache.dtype != torch.int8:
            raise ValueError("'int8' caches hold int8 codes")
        if k_scale is None or v_scale is None:
            raise ValueError("'int8' caches need k_scale and v_scale scale caches")
        if k_scale.shape != (NB, bs, Hkv) or k_scale.dtype != torch.float16 or \
                k_scale.stride() != v_scale.stride() or v_scale.shape != k_scale.shape:
            raise ValueError("scale caches must be fp16 [num_blocks, block_size, Hkv] alike")
        code, ks, vs, sstr = _lib.DT_I8, k_scale, v_scale, k_scale.stride()
    else:
        raise ValueError(f"kv_cache_dtype must be 'auto' or 'int8', got {kv_cache_dtype!r}")
    _lib.require_cuda(ks, vs)
    lib = _lib.load()
    cs = k_cache.stride()
    _lib.check(lib.coopt_kv_write(code, _lib.ptr(k), _lib.ptr(v), k.stride(0), k.stride(1),
                                  v.stride(0), v.stride(1), _lib.ptr(k_cache), _lib.ptr(v_cache), cs[0], cs[1], cs[2],
                                  _lib.ptr(ks), _lib.ptr(vs), sstr[0], sstr[1], sstr[2],
                                  _lib.ptr(slot_mapping), T, Hkv, D, bs, NB,
                                  _lib.stream_handle(k.device)), "coopt_kv_write")


def qkv_rope_and_cache(qkv, positions, cos, sin, k_cache, v_cache, slot_mapping, num_heads,
                       num_kv_heads, head_dim, kv_cache_dtype="auto", k_scale=None,
                       v_scale=None, q_out=None):
    """The chain after the qkv projection (engine/model.py:238-243) in one launch: split q/k/v,
    neox RoPE on q and k, k and v into the paged cache (as reshape_and_cache_flash), and
    return q [T, num_heads, head_dim].  `qkv` is the projection's bf16 output [T, (Hq + 2 Hkv)
    D] or its fused.LinearPartials (split-K partials, reduced here).  Bit for bit the same as
    rope_ + reshape_and_cache_flash on the reduced output."""
    from .fused import LinearPartials

    Hq, Hkv, D = int(num_heads), int(num_kv_heads), int(head_dim)
    width = (Hq + 2 * Hkv) * D
    part = qkv if isinstance(qkv, LinearPartials) else None
    if part is not None:
        if part.n != width:
            raise ValueError(f"partials are {part.n} wide, expected {width}")
        T, dev = part.rows, part.device
        qkv_t = None
    else:
        _lib.require_cuda(qkv)
        if qkv.dtype != torch.bfloat16 or qkv.dim() != 2 or qkv.shape[1] != width or qkv.stride(1) != 1:
            raise ValueError(f"qkv must be bf16 [T, {width}] with contiguous rows")
        T, dev, qkv_t = qkv.shape[0], qkv.device, qkv
    _lib.require_cuda(positions, cos, sin, k_cache, v_cache, slot_mapping)
    _check_cache_pair(k_cache, v_cache)
    NB, bs, cH, cD = k_cache.shape
    if (cH, cD) != (Hkv, D):
        raise ValueError(f"cache heads/dim {(cH, cD)} != ({Hkv}, {D})")
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != T:
        raise ValueError("slot_mapping must be int64 with one entry per token")
    if positions.dtype != torch.int64 or positions.numel() != T:
        raise ValueError("positions must be int64 with one entry per token")
    if cos.shape != sin.shape or cos.stride() != sin.stride() or cos.shape[1] < D // 2 or \
            cos.dtype != torch.bfloat16 or cos.stride(1) != 1:
        raise ValueError("cos/sin tables must be bf16 [max_pos, >= D/2] alike")
    if kv_cache_dtype == "auto":
        code, ks, vs, sstr = _lib.DT_BF16, None, None, (0, 0, 0)
    elif kv_cache_dtype == "int8":
        if k_scale is None or v_scale is None or k_scale.stride() != v_scale.stride():
            raise ValueError("'int8' caches need alike k_scale and v_scale scale caches")
        code, ks, vs, sstr = _lib.DT_I8, k_scale, v_scale, k_scale.stride()
    else:
        raise ValueError(f"kv_cache_dtype must be 'auto' or 'int8', got {kv_cache_dtype!r}")
    if q_out is None:
        q_out = torch.empty((T, Hq, D), dtype=torch.bfloat16, device=dev)
    positions, slot_mapping = positions.contiguous(), slot_mapping.contiguous()
    cs = k_cache.stride()
    _lib.check(_lib.load().coopt_qkv_epilogue(
        code, _lib.ptr(qkv_t), 0 if qkv_t is None else qkv_t.stride(0),
        None if part is None else _lib.ptr(part.buf), 0 if part is None else part.ks,
        0 if part is None else part.rows_padded * part.n,
        _lib.ptr(positions), _lib.ptr(cos), _lib.ptr(sin), cos.stride(0),
        cos.shape[0], _lib.ptr(q_out), q_out.stride(0), q_out.stride(1), _lib.ptr(k_cache),
        _lib.ptr(v_cache), cs[0], cs[1], cs[2], _lib.ptr(ks), _lib.ptr(vs), sstr[0], sstr[1],
        sstr[2], _lib.ptr(slot_mapping), T, Hq, Hkv, D, bs, NB,
        _lib.stream_handle(dev)), "coopt_qkv_epilogue")
    return q_out
