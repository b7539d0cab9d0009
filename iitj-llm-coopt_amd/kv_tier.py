"""GPU -> CPU KV tiering with quantize-on-evict, on the fused swap codec.

Call surface of engine/kv_tier_manager.py (mohsinmubarak/iitj-llm-coopt): SwappedKV (:44-52),
KVTierManager(engine, cpu_gb, bits) with cpu_usage / hit_rate (:67-74), estimate_bytes
(:76-79), has (:81-82), swap_out (:84-107), swap_in (:109-123), drop (:125-128) and
note_recompute (:130-131).

The reference quantizes cache[blocks] per layer (a gather plus the codec's elementwise ops)
on a side stream and copies every per-layer tensor to pinned memory separately.  Here each
(layer, K/V) cache is one coopt_kv_swap_out launch that gathers and quantizes into a single
device staging buffer, and the whole sequence crosses PCIe in one copy per direction; swap_in
scatters with coopt_kv_swap_in.  Codes and scales are bit-identical to the reference's
quantize on the GPU.  A cache that already holds INT8 codes (allocate_kv_cache(..., "int8"))
is swapped code for code with its scales, i.e. losslessly, whatever `bits` is set to.

`engine` needs: engine.target.k_cache / v_cache (per-layer lists), engine.bm (BlockManager
with .tables), and optionally engine.target.k_scale / v_scale (per-layer lists, INT8 caches),
engine.target.cfg (num_hidden_layers, num_key_value_heads, head_dim) and engine.counters.
"""
from dataclasses import dataclass

import torch

from . import _lib

__all__ = ["SwappedKV", "KVTierManager", "swap_out_blocks", "swap_in_blocks", "swap_out_caches",
           "swap_in_caches"]


@dataclass
class SwappedKV:
    k: list              # per layer: swapped [nb, bs, Hkv, D(/2)] on pinned CPU
    v: list
    k_scale: list        # per layer fp16 [nb, bs, Hkv] (None at 16 bits)
    v_scale: list
    num_tokens: int
    bits: int
    nbytes: int


def _cache_code(cache):
    if cache.dtype == torch.bfloat16:
        return _lib.DT_BF16
    if cache.dtype == torch.int8:
        return _lib.DT_I8
    raise ValueError(f"caches must be bf16 or int8 codes, got {cache.dtype}")


def _check_cache(cache, scale):
    if cache.dim() != 4 or cache.stride(-1) != 1:
        raise ValueError("caches must be [num_blocks, block_size, Hkv, D] with contiguous D")
    if cache.dtype == torch.int8:
        if scale is None or scale.shape != cache.shape[:-1] or scale.dtype != torch.float16:
            raise ValueError("an INT8 cache needs its fp16 [num_blocks, block_size, Hkv] scales")


def _swap_shapes(cache, nb, bits):
    _, bs, H, D = cache.shape
    if bits == 16:
        return (nb, bs, H, D), cache.dtype, None
    return (nb, bs, H, D // 2 if bits == 4 else D), (torch.uint8 if bits == 4 else torch.int8), (nb, bs, H)


def swap_out_blocks(cache, block_ids, bits: int, cache_scale=None, out=None, out_scale=None):
    """quantize(cache[block_ids], bits) in one launch -> (q, scale) on the cache's device.

    bf16 caches: bits 16 / 8 / 4 as kv_tier_manager.quantize; INT8 caches: the codes and
    scales themselves (bits must be 8)."""
    _lib.require_cuda(cache, block_ids)
    _check_cache(cache, cache_scale)
    code = _cache_code(cache)
    if code == _lib.DT_I8 and bits != 8:
        raise ValueError("an INT8 cache swaps at 8 bits")
    ids = block_ids.to(torch.int64).contiguous()
    nb = ids.numel()
    qshape, qdtype, sshape = _swap_shapes(cache, nb, bits)
    q = torch.empty(qshape, dtype=qdtype, device=cache.device) if out is None else out
    s = None
    if sshape is not None:
        s = torch.empty(sshape, dtype=torch.float16, device=cache.device) if out_scale is None else out_scale
    if q.shape != qshape or not q.is_contiguous() or (s is not None and (s.shape != sshape or not s.is_contiguous())):
        raise ValueError("swap buffers must be contiguous and of the swapped shape")
    cs = cache.stride()
    ss = cache_scale.stride() if code == _lib.DT_I8 else (0, 0, 0)
    _, bs, H, D = cache.shape
    _lib.check(_lib.load().coopt_kv_swap_out(
        bits, code, _lib.ptr(cache), cs[0], cs[1], cs[2],
        _lib.ptr(cache_scale) if code == _lib.DT_I8 else None, ss[0], ss[1], ss[2],
        _lib.ptr(ids), nb, bs, H, D, cache.shape[0], _lib.ptr(q), _lib.ptr(s),
        _lib.stream_handle(cache.device)), "coopt_kv_swap_out")
    return q, s


def swap_in_blocks(q, scale, bits: int, block_ids, cache, cache_scale=None):
    """cache[block_ids] = dequantize(q, scale, bits, cache.dtype), in place, one launch."""
    _lib.require_cuda(q, cache, block_ids)
    _check_cache(cache, cache_scale)
    code = _cache_code(cache)
    if code == _lib.DT_I8 and bits != 8:
        raise ValueError("an INT8 cache swaps at 8 bits")
    ids = block_ids.to(torch.int64).contiguous()
    nb = ids.numel()
    qshape, qdtype, sshape = _swap_shapes(cache, nb, bits)
    if q.shape != qshape or q.dtype != qdtype or not q.is_contiguous():
        raise ValueError(f"q must be contiguous {qdtype} {qshape}")
    if sshape is not None and (scale is None or scale.shape != sshape or not scale.is_contiguous()):
        raise ValueError(f"scale must be contiguous fp16 {sshape}")
    cs = cache.stride()
    ss = cache_scale.stride() if code == _lib.DT_I8 else (0, 0, 0)
    _, bs, H, D = cache.shape
    _lib.check(_lib.load().coopt_kv_swap_in(
        bits, code, _lib.ptr(q), _lib.ptr(scale), _lib.ptr(ids), nb, bs, H, D, cache.shape[0],
        _lib.ptr(cache), cs[0], cs[1], cs[2],
        _lib.ptr(cache_scale) if code == _lib.DT_I8 else None, ss[0], ss[1], ss[2],
        _lib.stream_handle(cache.device)), "coopt_kv_swap_in")
    return cache


def _uniform_caches(caches, scales):
    """(dtype code, cache strides, scale strides) shared by every cache, or None."""
    c0 = caches[0]
    for c, sc in zip(caches, scales):
        _check_cache(c, sc)
        if c.shape != c0.shape or c.stride() != c0.stride() or c.dtype != c0.dtype or c.device != c0.device:
            return None
    code = _cache_code(c0)
    ss = (0, 0, 0)
    if code == _lib.DT_I8:
        s0 = scales[0]
        if any(sc.stride() != s0.stride() for sc in scales):
            return None
        ss = s0.stride()
    return code, c0.stride(), ss


def _pointer_array(ts):
    import ctypes
    arr = (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])
    return arr, ctypes.addressof(arr)


def swap_out_caches(caches, block_ids, bits: int, scales=None, out=None, out_scale=None):
    """swap_out_blocks over a list of caches of one shape, dtype and strides (the K and V caches
    of every layer) in one launch -> (q [n, ...], scale [n, ...]); cache i's rows are q[i] and
    scale[i], bit-identical to swap_out_blocks(caches[i], ...).  Caches that differ in layout
    are swapped one launch each."""
    n = len(caches)
    scales = list(scales) if scales is not None else [None] * n
    _lib.require_cuda(caches[0], block_ids)
    ids = block_ids.to(torch.int64).contiguous()
    nb = ids.numel()
    qshape, qdtype, sshape = _swap_shapes(caches[0], nb, bits)
    dev = caches[0].device
    q = torch.empty((n, *qshape), dtype=qdtype, device=dev) if out is None else out
    s = None
    if sshape is not None:
        s = torch.empty((n, *sshape), dtype=torch.float16, device=dev) if out_scale is None else out_scale
    if q.shape != (n, *qshape) or not q.is_contiguous() or (s is not None and (s.shape != (n, *sshape) or not s.is_contiguous())):
        raise ValueError("swap buffers must be contiguous [n, ...] of the swapped shape")
    uni = _uniform_caches(caches, scales)
    if uni is None:
        for i, (c, sc) in enumerate(zip(caches, scales)):
            swap_out_blocks(c, ids, bits, sc, out=q[i], out_scale=None if s is None else s[i])
        return q, s
    code, cs, ss = uni
    if code == _lib.DT_I8 and bits != 8:
        raise ValueError("an INT8 cache swaps at 8 bits")
    carr, cptr = _pointer_array(caches)
    sarr, sptr = _pointer_array(scales) if code == _lib.DT_I8 else (None, None)
    _, bs, H, D = caches[0].shape
    _lib.check(_lib.load().coopt_kv_swap_out_caches(
        bits, code, n, cptr, sptr, cs[0], cs[1], cs[2], ss[0], ss[1], ss[2], _lib.ptr(ids), nb, bs,
        H, D, caches[0].shape[0], _lib.ptr(q), _lib.ptr(s), _lib.stream_handle(dev)),
        "coopt_kv_swap_out_caches")
    del carr, sarr
    return q, s


def swap_in_caches(q, scale, bits: int, block_ids, caches, scales=None):
    """swap_in_blocks(q[i], scale[i], ..., caches[i]) for every i, in one launch when the
    caches share shape, dtype and strides."""
    n = len(caches)
    scales = list(scales) if scales is not None else [None] * n
    _lib.require_cuda(q, caches[0], block_ids)
    ids = block_ids.to(torch.int64).contiguous()
    nb = ids.numel()
    qshape, qdtype, sshape = _swap_shapes(caches[0], nb, bits)
    if q.shape != (n, *qshape) or q.dtype != qdtype or not q.is_contiguous():
        raise ValueError(f"q must be contiguous {qdtype} {(n, *qshape)}")
    if sshape is not None and (scale is None or scale.shape != (n, *sshape) or not scale.is_contiguous()):
        raise ValueError(f"scale must be contiguous fp16 {(n, *sshape)}")
    uni = _uniform_caches(caches, scales)
    if uni is None:
        for i, (c, sc) in enumerate(zip(caches, scales)):
            swap_in_blocks(q[i], None if scale is None else scale[i], bits, ids, c, sc)
        return caches
    code, cs, ss = uni
    if code == _lib.DT_I8 and bits != 8:
        raise ValueError("an INT8 cache swaps at 8 bits")
    carr, cptr = _pointer_array(caches)
    sarr, sptr = _pointer_array(scales) if code == _lib.DT_I8 else (None, None)
    _, bs, H, D = caches[0].shape
    _lib.check(_lib.load().coopt_kv_swap_in_caches(
        bits, code, n, _lib.ptr(q), _lib.ptr(scale), _lib.ptr(ids), nb, bs, H, D,
        caches[0].shape[0], cptr, sptr, cs[0], cs[1], cs[2], ss[0], ss[1], ss[2],
        _lib.stream_handle(caches[0].device)), "coopt_kv_swap_in_caches")
    del carr, sarr
    return caches


class KVTierManager:
    def __init__(self, engine, cpu_gb: float = 32.0, bits: int = 8):
        if bits not in (16, 8, 4):
            raise ValueError("bits must be 16, 8 or 4")
        self.e = engine
        self.capacity = int(cpu_gb * 2**30)
        self.bits = bits                 # codec width of the next swap_out (a policy may change it)
        self.store: dict = {}
        self.used = 0
        self._stream = None              # side stream for swap_out, created on first use
        self.restores = self.recomputes = 0
        self.bytes_out = self.bytes_in = 0
        engine.kv_tiers = self

    # ---- the reference's accounting (engine/kv_tier_manager.py:67-82) ---------------------
    @property
    def cpu_usage(self):
        return self.used / self.capacity

    @property
    def hit_rate(self):
        total = self.restores + self.recomputes
        return self.restores / total if total else 0.0

    def _geometry(self):
        cfg = getattr(self.e.target, "cfg", None)
        if cfg is not None:
            return cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
        kc = self.e.target.k_cache[0]
        return len(self.e.target.k_cache), kc.shape[2], kc.shape[3]

    def estimate_bytes(self, num_tokens: int, bits: int) -> int:
        layers, hkv, d = self._geometry()
        per_token = 2 * layers * hkv * d * bits / 8
        return int(per_token * num_tokens * (1 + (2 / d if bits < 16 else 0)))

    def has(self, seq_id):
        return seq_id in self.store

    def _bits_for_cache(self):
        kc = self.e.target.k_cache
        return 8 if len(kc) and kc[0].dtype == torch.int8 else self.bits

    def _scales(self):
        t = self.e.target
        L = len(t.k_cache)
        return (getattr(t, "k_scale", None) or [None] * L, getattr(t, "v_scale", None) or [None] * L)

    # ---- swap out / in ---------------------------------------------------------------------
    def swap_out(self, seq) -> bool:
        """Moves the target KV of seq's first num_computed tokens to host memory (quantised to
        self.bits); returns False, moving nothing, when the tier lacks the room."""
        n = seq.num_computed
        if n == 0:
            return False
        bits = self._bits_for_cache()
        need = self.estimate_bytes(n, bits)
        if self.used + need > self.capacity:
            return False
        e, bm = self.e, self.e.bm
        kcs, vcs = e.target.k_cache, e.target.v_cache
        kss, vss = self._scales()
        dev = kcs[0].device
        blocks = torch.tensor(bm.tables[seq.seq_id][: bm.blocks_for(n)], device=dev, dtype=torch.int64)
        L, nb = len(kcs), blocks.numel()
        qshape, qdtype, sshape = _swap_shapes(kcs[0], nb, bits)
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=dev)
        self._stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self._stream):
            # one staging buffer for the whole sequence, one PCIe copy each for codes and scales
            q = torch.empty((L, 2, *qshape), dtype=qdtype, device=dev)
            s = torch.empty((L, 2, *sshape), dtype=torch.float16, device=dev) if sshape else None
            # every layer's K and V cache in one launch: cache 2 li + j is q[li, j]
            caches = [c for li in range(L) for c in (kcs[li], vcs[li])]
            cscales = [c for li in range(L) for c in (kss[li], vss[li])]
            swap_out_caches(caches, blocks, bits, cscales, out=q.view(2 * L, *qshape),
                            out_scale=None if s is None else s.view(2 * L, *sshape))
            hq = torch.empty(q.shape, dtype=q.dtype, pin_memory=True)
            hq.copy_(q, non_blocking=True)
            hs = None
            if s is not None:
                hs = torch.empty(s.shape, dtype=s.dtype, pin_memory=True)
                hs.copy_(s, non_blocking=True)
        self._stream.synchronize()
        out = SwappedKV([hq[li, 0] for li in range(L)], [hq[li, 1] for li in range(L)],
                        [None if hs is None else hs[li, 0] for li in range(L)],
                        [None if hs is None else hs[li, 1] for li in range(L)], n, bits, need)
        self.store[seq.seq_id] = out
        self.used += need
        self.bytes_out += need
        counters = getattr(e, "counters", None)
        if counters is not None:
            counters["kv_evictions_total"] = counters.get("kv_evictions_total", 0) + 1
        return True

    def swap_in(self, seq) -> None:
        """Brings seq's swapped KV back into blocks ensure() hands out now (the caller has
        made sure they are available), dequantised into the caches."""
        sw = self.store.pop(seq.seq_id)
        e, bm = self.e, self.e.bm
        kcs, vcs = e.target.k_cache, e.target.v_cache
        kss, vss = self._scales()
        dev = kcs[0].device
        bm.ensure(seq.seq_id, sw.num_tokens)
        blocks = torch.tensor(bm.tables[seq.seq_id][: bm.blocks_for(sw.num_tokens)], device=dev,
                              dtype=torch.int64)
        L = len(kcs)
        # the per-layer entries are views of one pinned buffer: one copy per direction
        base_q = sw.k[0]._base if sw.k[0]._base is not None else None
        if base_q is not None and base_q.shape[:2] == (L, 2):
            q = base_q.to(dev, non_blocking=True)
            qs = [(q[li, 0], q[li, 1]) for li in range(L)]
            qall = q
        else:
            qs = [(sw.k[li].to(dev, non_blocking=True), sw.v[li].to(dev, non_blocking=True)) for li in range(L)]
            qall = None
        sall = None
        if sw.bits == 16:
            ss = [(None, None)] * L
        else:
            base_s = sw.k_scale[0]._base
            if base_s is not None and base_s.shape[:2] == (L, 2):
                s = base_s.to(dev, non_blocking=True)
                ss = [(s[li, 0], s[li, 1]) for li in range(L)]
                sall = s
            else:
                ss = [(sw.k_scale[li].to(dev, non_blocking=True), sw.v_scale[li].to(dev, non_blocking=True))
                      for li in range(L)]
        if qall is not None and (sw.bits == 16 or sall is not None):
            # every layer's K and V cache in one launch
            caches = [c for li in range(L) for c in (kcs[li], vcs[li])]
            cscales = [c for li in range(L) for c in (kss[li], vss[li])]
            swap_in_caches(qall.view(2 * L, *qall.shape[2:]),
                           None if sw.bits == 16 else sall.view(2 * L, *sall.shape[2:]),
                           sw.bits, blocks, caches, cscales)
        else:
            for li in range(L):
                swap_in_blocks(qs[li][0], ss[li][0], sw.bits, blocks, kcs[li], kss[li])
                swap_in_blocks(qs[li][1], ss[li][1], sw.bits, blocks, vcs[li], vss[li])
        self.used -= sw.nbytes
        self.bytes_in += sw.nbytes
        self.restores += 1
        counters = getattr(e, "counters", None)
        if counters is not None:
            counters["kv_restores_total"] = counters.get("kv_restores_total", 0) + 1

    def drop(self, seq_id):
        sw = self.store.pop(seq_id, None)
        if sw:
            self.used -= sw.nbytes

    def note_recompute(self):
        self.recomputes += 1
