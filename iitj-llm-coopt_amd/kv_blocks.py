"""Block-major KV buffer and the block migration copy, on the coopt_kv_copy_blocks kernel.

Reference paths under mohsinmubarak/iitj-llm-coopt:
  allocate_block_major_kv   the elastic buffer [blocks, layers, K/V, bs, Hkv, D] and its
                            strided per-layer views (engine/elastic.py:74-77)
  copy_blocks               copy_fn(src, dst) = buf[dst].copy_(buf[src]) of
                            BlockManager.migrate_out_of (engine/elastic.py:131), batched: every
                            pair of a migration, in every cache, in one launch
  migrate_out_of            the unpark migration (engine/elastic.py:129-134): the block
                            manager's bookkeeping, then one copy_blocks launch

A "cache" here is any tensor whose dim 0 is the block id and whose blocks are dense: the whole
block-major buffer (a 2 MiB block per id for the 8B target), or per-layer K / V caches and
INT8 scale caches from allocate_kv_cache.
"""
import numpy as np
import torch

from . import _lib

__all__ = ["allocate_block_major_kv", "block_region", "copy_blocks", "migrate_out_of"]


def allocate_block_major_kv(num_blocks: int, num_layers: int, block_size: int, num_kv_heads: int,
                            head_dim: int, dtype=torch.bfloat16, device="cuda"):
    """-> (buf, k_caches, v_caches): buf [NB, L, 2, bs, Hkv, D] and its per-layer views
    buf[:, l, 0] / buf[:, l, 1], [NB, bs, Hkv, D] each (engine/elastic.py:74-77).  Block b of
    every layer is the contiguous chunk buf[b]; the attention and KV-write kernels take the
    strided views as they are."""
    buf = torch.empty((num_blocks, num_layers, 2, block_size, num_kv_heads, head_dim), dtype=dtype,
                      device=device)
    return buf, [buf[:, i, 0] for i in range(num_layers)], [buf[:, i, 1] for i in range(num_layers)]


def block_region(t: torch.Tensor):
    """(base address, bytes between block ids, bytes per block) of a tensor whose dim 0 is the
    block id; raises ValueError unless each block t[b] is one dense byte range."""
    if t.dim() < 1 or t.shape[0] == 0:
        raise ValueError("a cache needs a leading block dimension")
    dims = sorted((st, n) for n, st in zip(t.shape[1:], t.stride()[1:]) if n > 1)
    expect = 1
    for st, n in dims:
        if st != expect:
            raise ValueError(f"blocks of a {tuple(t.shape)} tensor with strides {t.stride()} "
                             "are not dense")
        expect *= n
    per = expect * t.element_size()
    stride = t.stride(0) * t.element_size()
    if stride < per:
        raise ValueError("blocks overlap (block stride smaller than a block)")
    return t.data_ptr(), stride, per


def _ids_on(dev, ids):
    if isinstance(ids, torch.Tensor):
        return ids.to(device=dev, dtype=torch.int64).contiguous()
    return torch.as_tensor(np.asarray(ids, dtype=np.int64)).to(dev)


def copy_blocks(caches, src, dst, num_blocks=None):
    """For every i: block dst[i] <- block src[i] in every cache, in one launch (one per 32
    caches).  `caches`: a tensor or a list of tensors on one device, all with the same number
    of blocks (or pass num_blocks).  `src` / `dst`: equal-length int sequences or tensors.
    Host-side ids are checked: in range, no dst repeated, no dst that is also a src (the
    kernel copies pairs in no particular order)."""
    if isinstance(caches, torch.Tensor):
        caches = [caches]
    caches = list(caches)
    if not caches:
        return
    _lib.require_cuda(*caches)
    dev = caches[0].device
    if any(c.device != dev for c in caches):
        raise ValueError("all caches must be on one device")
    nb = int(caches[0].shape[0]) if num_blocks is None else int(num_blocks)
    if num_blocks is None and any(int(c.shape[0]) != nb for c in caches):
        raise ValueError("caches hold different numbers of blocks; pass num_blocks")
    if any(int(c.shape[0]) < nb for c in caches):
        raise ValueError("num_blocks exceeds a cache's block count")
    host = not (isinstance(src, torch.Tensor) and src.is_cuda)
    if host:
        s = np.asarray(src.cpu() if isinstance(src, torch.Tensor) else src, dtype=np.int64).ravel()
        d = np.asarray(dst.cpu() if isinstance(dst, torch.Tensor) else dst, dtype=np.int64).ravel()
        if s.shape != d.shape:
            raise ValueError("src and dst must have the same length")
        if len(s) == 0:
            return
        if s.min() < 0 or d.min() < 0 or s.max() >= nb or d.max() >= nb:
            raise ValueError(f"block ids must lie in [0, {nb})")
        if len(np.unique(d)) != len(d) or np.intersect1d(s, d).size:
            raise ValueError("dst ids must be distinct and disjoint from the src ids")
        ids = torch.from_numpy(np.stack([s, d])).to(dev)
        s_t, d_t = ids[0], ids[1]
    else:
        s_t, d_t = _ids_on(dev, src), _ids_on(dev, dst)
        if s_t.shape != d_t.shape:
            raise ValueError("src and dst must have the same length")
        if s_t.numel() == 0:
            return
    regions = np.array([block_region(c) for c in caches], dtype=np.int64)
    _lib.check(_lib.load().coopt_kv_copy_blocks(
        regions.ctypes.data, len(caches), _lib.ptr(s_t), _lib.ptr(d_t), int(s_t.numel()), nb,
        _lib.stream_handle(dev)), "coopt_kv_copy_blocks")


def migrate_out_of(bm, ids, caches) -> int:
    """Move every in-use block in `ids` to a free block outside `ids` and copy its KV in every
    cache, as the elastic unpark does (engine/elastic.py:131), in one launch.  `bm` is a
    BlockManager with migrate_out_of(ids, copy_fn) (this package's or the reference's); the
    pairs it reports are disjoint (sources inside `ids`, destinations outside), so copying
    them together equals copying them one at a time.  Returns blocks moved, or -1 when there
    is not enough room outside `ids` (nothing moved)."""
    pairs = []
    moved = bm.migrate_out_of(ids, lambda s, d: pairs.append((s, d)))
    if moved > 0:
        copy_blocks(caches, [p[0] for p in pairs], [p[1] for p in pairs],
                    num_blocks=min(int(c.shape[0]) for c in
                                   ([caches] if isinstance(caches, torch.Tensor) else caches)))
    return moved
