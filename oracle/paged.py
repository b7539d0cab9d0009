"""Paged KV addressing, KV write and paged causal GQA attention (numpy, CPU).

slot_mapping   engine/block_manager.py:216-220   slot = table[p // bs] * bs + p % bs
block_table    engine/block_manager.py:222-229   [B, W] int32, rows zero-padded
kv_write       engine/model.py:190, 201-203      k_cache[slot // bs, slot % bs] = k
               (the semantics tests/kv_write_check.py:26-30 pins for the fused vLLM op);
               INT8 caches store quantize(k, 8) (engine/kv_tier_manager.py:21-31) per vector
swap_out/in    engine/kv_tier_manager.py:99, 119  quantize(cache[blocks]) / cache[blocks] = dequantize
migrate        engine/block_manager.py:165-187   move in-use blocks out of a set, FIFO destinations
copy_blocks    engine/elastic.py:131              buf[dst] = buf[src] per migrated block
attention      engine/model.py:204-207, 244-247 (flash_attn_varlen_func, causal, paged):
               query j of a sequence with n new tokens and L keys sees keys [0, L - n + j]
               (causal mask aligned bottom-right, engine/model.py:8-10); head h reads KV head
               h // (Hq / Hkv); scale 1/sqrt(D) (engine/model.py:102).  INT8 KV is attention
               over dequantize(quantize(KV)) in bf16 (eval/quality.py:48-52).

The attention kernel is third-party (vLLM 0.31.0's FlashAttention-2) and absent here, so its
numerics are pinned only by the closed form: this module computes it in float64 over the
gathered pages.  Pinned further by tests/test_oracle_paged.py: the block-manager known-answer
test of tests/test_units.py:19-29, strided (block-major) views agreeing with contiguous ones
(tests/strided_kv_check.py), single-key and uniform-score closed forms, and a brute-force
per-(row, head) loop.
"""
import numpy as np

from . import codec


def slot_mapping(table, start: int, end: int, block_size: int):
    table = np.asarray(table, dtype=np.int64)
    pos = np.arange(start, end, dtype=np.int64)
    return table[pos // block_size] * block_size + pos % block_size


def block_table(tables, width=None):
    w = max((len(t) for t in tables), default=0) if width is None else width
    out = np.zeros((len(tables), w), dtype=np.int32)
    for i, t in enumerate(tables):
        out[i, :len(t)] = t
    return out


def kv_write(k_cache, v_cache, k, v, slots, block_size: int):
    """In-place index_put into [NB, bs, H, D] caches (numpy arrays or writable views)."""
    slots = np.asarray(slots, dtype=np.int64)
    ok = (slots >= 0) & (slots < k_cache.shape[0] * block_size)
    blk, off = slots[ok] // block_size, slots[ok] % block_size
    k_cache[blk, off] = np.asarray(k)[ok]
    v_cache[blk, off] = np.asarray(v)[ok]


def kv_write_int8(kq, vq, ks, vs, k, v, slots, block_size: int, mode: str = "device"):
    """INT8 caches: codes [NB, bs, H, D] int8 and fp16 scales [NB, bs, H]."""
    qk, sk = codec.quantize(k, 8, mode)
    qv, sv = codec.quantize(v, 8, mode)
    slots = np.asarray(slots, dtype=np.int64)
    ok = (slots >= 0) & (slots < kq.shape[0] * block_size)
    blk, off = slots[ok] // block_size, slots[ok] % block_size
    kq[blk, off], vq[blk, off] = qk[ok], qv[ok]
    ks[blk, off], vs[blk, off] = sk[ok], sv[ok]


def gather(cache, table_row, L: int, block_size: int):
    pos = np.arange(L)
    return cache[np.asarray(table_row)[pos // block_size], pos % block_size]


def attention_seq(q, K, V, scale=None):
    """One sequence: q [n, Hq, D] (its n new rows), K/V [L, Hkv, D] gathered keys/values.

    Query j sees keys [0, L - n + j]; returns [n, Hq, D] float64 (0 where nothing is visible).
    """
    q = np.asarray(q, dtype=np.float64)
    n, Hq, D = q.shape
    L, Hkv = K.shape[0], K.shape[1]
    G = Hq // Hkv
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    if n == 0 or L == 0:
        return np.zeros((n, Hq, D))
    Kh = np.ascontiguousarray(np.asarray(K, np.float64).transpose(1, 2, 0))  # [Hkv, D, L]
    Vh = np.ascontiguousarray(np.asarray(V, np.float64).transpose(1, 0, 2))  # [Hkv, L, D]
    Q = q.reshape(n, Hkv, G, D).transpose(1, 0, 2, 3).reshape(Hkv, n * G, D)
    s = np.matmul(Q, Kh) * scale                                              # [Hkv, n*G, L]
    lim = np.repeat(L - n + np.arange(n), G)                                  # row (j, g)
    s = np.where(np.arange(L)[None, None, :] > lim[None, :, None], -np.inf, s)
    m = s.max(-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(s - m)
    den = p.sum(-1, keepdims=True)
    p = np.divide(p, den, out=np.zeros_like(p), where=den > 0)
    o = np.matmul(p, Vh)                                                      # [Hkv, n*G, D]
    return o.reshape(Hkv, n, G, D).transpose(1, 0, 2, 3).reshape(n, Hq, D)


def attention(q, k_cache, v_cache, cu_seqlens_q, seq_lens, block_tables, block_size: int,
              scale=None):
    """float64 causal paged GQA attention; q [T, Hq, D]; caches hold K/V values [NB, bs, Hkv, D].

    Returns out [T, Hq, D] float64.  Rows whose visible range is empty are 0.
    """
    q = np.asarray(q, dtype=np.float64)
    out = np.zeros(q.shape, dtype=np.float64)
    cu = np.asarray(cu_seqlens_q)
    for b in range(len(seq_lens)):
        q0, n, L = int(cu[b]), int(cu[b + 1] - cu[b]), int(seq_lens[b])
        if n == 0 or L == 0:
            continue
        K = gather(k_cache, block_tables[b], L, block_size)
        V = gather(v_cache, block_tables[b], L, block_size)
        out[q0:q0 + n] = attention_seq(q[q0:q0 + n], K, V, scale)
    return out


def dequantized_cache(codes, scales):
    """INT8 cache -> the bf16 values dequantize(q, scale, 8, bf16) gives, as float32."""
    return codec.bf16_round(codec.dequantize(codes, scales, 8))


def swap_out(cache, blocks, bits: int, mode: str = "device"):
    """quantize(cache[blocks], bits) (engine/kv_tier_manager.py:99) on cache values [NB, bs,
    H, D]: -> (codes, fp16 scales), or (cache[blocks] copy, None) at 16 bits.  Ids outside the
    pool give zero vectors (the kernel's documented behaviour for them)."""
    cache = np.asarray(cache, dtype=np.float32)
    blocks = np.asarray(blocks, dtype=np.int64)
    ok = (blocks >= 0) & (blocks < cache.shape[0])
    x = np.zeros((len(blocks),) + cache.shape[1:], dtype=np.float32)
    x[ok] = cache[blocks[ok]]
    if bits == 16:
        return x, None
    return codec.quantize(x, bits, mode)


def swap_in(q, scale, bits: int):
    """dequantize(q, scale, bits, bf16) (engine/kv_tier_manager.py:119) as float32 values."""
    if bits == 16:
        return np.asarray(q, dtype=np.float32)
    return codec.bf16_round(codec.dequantize(q, scale, bits))


def migrate(tables, free, ids):
    """BlockManager.migrate_out_of (engine/block_manager.py:165-187) over plain lists, without
    prefix-cache state: -> (pairs [(src, dst)], tables, free) after the move, or None when
    fewer free blocks than in-use blocks of `ids` lie outside `ids` (nothing changes).  Sources
    are the in-use ids in ascending order; each takes the first free block outside `ids`
    (:202-208), every table entry holding it is rewritten, and it joins the end of the free
    list."""
    ids = set(ids)
    tables = {k: list(v) for k, v in tables.items()}
    free = list(free)
    used = sorted({b for t in tables.values() for b in t if b in ids})
    if sum(1 for b in free if b not in ids) < len(used):
        return None
    pairs = []
    for src in used:
        j = next(i for i, b in enumerate(free) if b not in ids)
        dst = free.pop(j)
        pairs.append((src, dst))
        for t in tables.values():
            for i, b in enumerate(t):
                if b == src:
                    t[i] = dst
        free.append(src)
    return pairs, tables, free


def copy_blocks(caches, pairs):
    """buf[dst] = buf[src] for each pair in order (engine/elastic.py:131), on numpy arrays
    whose dim 0 is the block id; returns new arrays."""
    out = [np.array(c, copy=True) for c in caches]
    for s, d in pairs:
        for c in out:
            c[d] = c[s]
    return out
