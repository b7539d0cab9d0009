"""GPU parity: the KV tier swap codec (coopt_kv_swap_out / coopt_kv_swap_in) and KVTierManager.

Bar: codes and fp16 scales bit-exact against the reference's swap lines executed by torch on
the same GPU (q, s = quantize(cache[blocks], bits), engine/kv_tier_manager.py:21-31 and :99)
and against oracle.paged.swap_out; restored caches bit-exact against
dequantize(q, s, bits, bf16) (:34-41, :119); INT8 caches round-trip losslessly.
"""
import types

import numpy as np
import pytest
import torch

import iitj_llm_coopt_amd as M
from oracle import paged as OP

pytestmark = pytest.mark.gpu


def ref_quantize(x, bits):
    """engine/kv_tier_manager.py:21-31, run by torch on the GPU."""
    if bits == 16:
        return x.clone(), None
    qmax = 127 if bits == 8 else 7
    scale = x.abs().amax(-1, keepdim=True).float().clamp_min(1e-8) / qmax
    q = torch.round(x.float() / scale).clamp(-qmax, qmax).to(torch.int8)
    if bits == 4:
        q = q + 8
        q = (q[..., 0::2] | (q[..., 1::2] << 4)).to(torch.uint8)
    return q, scale.squeeze(-1).to(torch.float16)


def ref_dequantize(q, scale, bits, dtype=torch.bfloat16):
    """engine/kv_tier_manager.py:34-41, run by torch on the GPU."""
    if bits == 16:
        return q
    if bits == 4:
        lo = (q & 0x0F).to(torch.int8) - 8
        hi = (q >> 4).to(torch.int8) - 8
        q = torch.stack((lo, hi), dim=-1).flatten(-2)
    return (q.float() * scale.float().unsqueeze(-1)).to(dtype)


def kv_values(shape, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(shape, generator=g, device=dev)
    x = torch.where(torch.rand(shape, generator=g, device=dev) < 0.01, x * 20, x)
    x[0, 0, 0] = 0  # an all-zero vector
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("head_major", [False, True])
@pytest.mark.parametrize("bits", [16, 8, 4])
def test_swap_out_matches_reference_lines(dev, bits, head_major):
    NB, bs, H, D = 96, 16, 8, 128
    if head_major:
        cache, _, _, _ = M.allocate_kv_cache(NB, bs, H, D, "auto", device=dev)
        cache.copy_(kv_values((NB, bs, H, D), dev, bits))
    else:
        cache = kv_values((NB, bs, H, D), dev, bits)
    blocks = torch.tensor([5, 90, 0, 17, 33, 64, 2], device=dev)
    q, s = M.swap_out_blocks(cache, blocks, bits)
    rq, rs = ref_quantize(cache[blocks], bits)
    assert torch.equal(q.view(rq.dtype) if bits == 16 else q.view(rq.dtype), rq)
    if bits != 16:
        assert torch.equal(s, rs)
    oq, osc = OP.swap_out(cache.float().cpu().numpy(), blocks.cpu().numpy(), bits)
    if bits == 16:
        assert np.array_equal(q.float().cpu().numpy(), oq)
    else:
        assert np.array_equal(q.cpu().numpy(), oq) and np.array_equal(s.cpu().numpy(), osc)


def test_swap_out_out_of_pool_ids_read_as_zero(dev):
    cache = kv_values((8, 16, 8, 128), dev, 1)
    q, s = M.swap_out_blocks(cache, torch.tensor([3, -1, 8], device=dev), 8)
    assert bool((q[1] == 0).all()) and bool((s[1] == 0).all())
    assert torch.equal(q[0], ref_quantize(cache[3], 8)[0])


@pytest.mark.parametrize("bits", [16, 8, 4])
def test_swap_in_matches_reference_dequantize(dev, bits):
    NB, bs, H, D = 64, 16, 8, 128
    src = kv_values((NB, bs, H, D), dev, 7)
    q, s = ref_quantize(src[:9], bits)
    cache, _, _, _ = M.allocate_kv_cache(NB, bs, H, D, "auto", device=dev)
    before = cache.clone()
    blocks = torch.tensor([40, 3, 11, 63, 0, 21, 22, 50, 9], device=dev)
    M.swap_in_blocks(q.contiguous(), None if s is None else s.contiguous(), bits, blocks, cache)
    want = before.clone()
    want[blocks] = ref_dequantize(q, s, bits, torch.bfloat16)
    assert torch.equal(cache, want)  # restored blocks exact, every other block untouched


class _Seq:
    def __init__(self, seq_id, n):
        self.seq_id, self.num_computed = seq_id, n


def _engine(dev, L, NB, bs, H, D, kv, seed):
    kc, vc, ks, vs = [], [], [], []
    for li in range(L):
        a, b, c, d = M.allocate_kv_cache(NB, bs, H, D, kv, device=dev)
        if kv == "auto":
            a.copy_(kv_values(a.shape, dev, seed + 2 * li))
            b.copy_(kv_values(b.shape, dev, seed + 2 * li + 1))
        else:
            slots = torch.arange(NB * bs, device=dev)
            M.reshape_and_cache_flash(kv_values((NB * bs, H, D), dev, seed + 2 * li),
                                      kv_values((NB * bs, H, D), dev, seed + 2 * li + 1),
                                      a, b, slots, "int8", c, d)
        kc.append(a); vc.append(b); ks.append(c); vs.append(d)
    target = types.SimpleNamespace(k_cache=kc, v_cache=vc,
                                   k_scale=ks if kv == "int8" else None, v_scale=vs if kv == "int8" else None,
                                   cfg=types.SimpleNamespace(num_hidden_layers=L, num_key_value_heads=H, head_dim=D))
    rng = np.random.default_rng(seed)
    return types.SimpleNamespace(target=target, bm=M.BlockManager(NB, bs, free_order=rng.permutation(NB)),
                                 counters={})


@pytest.mark.parametrize("kv,bits", [("auto", 8), ("auto", 4), ("auto", 16), ("int8", 8)])
def test_tier_manager_round_trip(dev, kv, bits):
    """swap_out -> free the blocks -> another sequence overwrites them -> swap_in into new
    blocks: the restored KV is dequantize(quantize(original)) (bf16 caches) or the original
    codes and scales (INT8 caches), bit for bit."""
    L, NB, bs, H, D = 3, 64, 16, 8, 128
    e = _engine(dev, L, NB, bs, H, D, kv, seed=11)
    tm = M.KVTierManager(e, cpu_gb=1.0, bits=bits)
    seq = _Seq(1, 37)
    e.bm.ensure(1, 37)
    blocks = torch.tensor(e.bm.tables[1], device=dev)
    orig = [(e.target.k_cache[li][blocks].clone(), e.target.v_cache[li][blocks].clone()) for li in range(L)]
    orig_s = ([(e.target.k_scale[li][blocks].clone(), e.target.v_scale[li][blocks].clone()) for li in range(L)]
              if kv == "int8" else None)
    assert tm.swap_out(seq) and tm.has(1)
    assert tm.used == tm.estimate_bytes(37, 8 if kv == "int8" else bits)
    e.bm.free(1)
    e.bm.ensure(2, NB * bs // 2)  # reuse (and scribble over) the freed blocks
    for li in range(L):
        b2 = torch.tensor(e.bm.tables[2], device=dev)
        e.target.k_cache[li][b2] = 0
        e.target.v_cache[li][b2] = 0
    tm.swap_in(seq)
    assert not tm.has(1) and tm.used == 0 and tm.restores == 1
    assert e.counters == {"kv_evictions_total": 1, "kv_restores_total": 1}
    nb = torch.tensor(e.bm.tables[1], device=dev)
    for li in range(L):
        for j, (cache, o) in enumerate(((e.target.k_cache[li], orig[li][0]), (e.target.v_cache[li], orig[li][1]))):
            got = cache[nb]
            if kv == "int8":
                assert torch.equal(got, o)
                sc = (e.target.k_scale if j == 0 else e.target.v_scale)[li][nb]
                assert torch.equal(sc, orig_s[li][j])
            else:
                q, s = ref_quantize(o, bits)
                assert torch.equal(got, ref_dequantize(q, s, bits))


def test_tier_manager_refuses_when_full_and_drops(dev):
    e = _engine(dev, 2, 32, 16, 8, 128, "auto", seed=3)
    tm = M.KVTierManager(e, cpu_gb=1e-4, bits=8)   # ~100 KB
    e.bm.ensure(5, 200)
    assert not tm.swap_out(_Seq(5, 200))           # does not fit
    tm.capacity = 1 << 30
    assert tm.swap_out(_Seq(5, 200))
    tm.drop(5)
    assert tm.used == 0 and not tm.has(5)


@pytest.mark.parametrize("kv,bits", [("auto", 16), ("auto", 8), ("auto", 4), ("int8", 8)])
@pytest.mark.parametrize("n", [2, 70])   # 70 caches take two launches (64 per launch)
def test_multi_cache_swap_equals_per_cache_swaps(dev, kv, bits, n):
    """swap_out_caches / swap_in_caches over n caches of one layout == n single-cache calls,
    bit for bit, both directions; ids outside the pool read as zero and are skipped."""
    NB, BS, H, D = 24, 16, 4, 64
    caches, scales = [], []
    for i in range(n):
        kc, _, ks, _ = M.allocate_kv_cache(NB, BS, H, D, kv, device=dev)
        x = kv_values((NB * BS, H, D), dev, seed=100 + i)
        M.reshape_and_cache_flash(x, x, kc, kc.clone(), torch.arange(NB * BS, device=dev), kv, ks,
                                  None if ks is None else ks.clone())
        caches.append(kc)
        scales.append(ks)
    ids = torch.tensor([5, 0, 23, -1, 7, 40], device=dev)
    q, s = M.swap_out_caches(caches, ids, bits, scales)
    for i in range(n):
        qi, si = M.swap_out_blocks(caches[i], ids, bits, scales[i])
        assert torch.equal(q[i], qi), i
        if si is not None:
            assert torch.equal(s[i], si), i
    # restore into fresh caches, then compare with single-cache restores
    fresh = [M.allocate_kv_cache(NB, BS, H, D, kv, device=dev) for _ in range(n)]
    tgt = [f[0] for f in fresh]
    tsc = [f[2] for f in fresh]
    dst = torch.tensor([1, 2, 3, -1, 4, 99], device=dev)
    M.swap_in_caches(q, s, bits, dst, tgt, tsc)
    for i in range(n):
        one, _, one_s, _ = M.allocate_kv_cache(NB, BS, H, D, kv, device=dev)
        M.swap_in_blocks(q[i], None if s is None else s[i], bits, dst, one, one_s)
        assert torch.equal(tgt[i].view(torch.uint8), one.view(torch.uint8)), i
        if one_s is not None:
            assert torch.equal(tsc[i], one_s), i


def test_multi_cache_swap_falls_back_on_mixed_layouts(dev):
    """A token-major cache among head-major ones: one launch per cache, same results."""
    NB, BS, H, D = 8, 16, 2, 64
    a, _, _, _ = M.allocate_kv_cache(NB, BS, H, D, "auto", device=dev)
    b = torch.zeros(NB, BS, H, D, dtype=torch.bfloat16, device=dev)   # token-major
    for i, c in enumerate((a, b)):
        c.copy_(kv_values((NB, BS, H, D), dev, seed=7 + i))
    ids = torch.tensor([3, 1], device=dev)
    q, s = M.swap_out_caches([a, b], ids, 8)
    for i, c in enumerate((a, b)):
        qi, si = M.swap_out_blocks(c, ids, 8)
        assert torch.equal(q[i], qi) and torch.equal(s[i], si)


@pytest.mark.parametrize("kv,bits", [("auto", 16), ("auto", 8), ("auto", 4), ("int8", 8)])
@pytest.mark.parametrize("H,D", [(8, 128), (4, 64), (3, 128)])
def test_wide_swap_matches_reference_lines(dev, kv, bits, H, D):
    """A swap wide enough for the several-chunks-per-thread kernels (64 caches x 40 ids; one
    cache alone takes the one-chunk form): codes and scales equal to the reference lines and
    to per-cache calls; restored caches equal to dequantize and to per-cache restores.  The
    (4, 64) and (3, 128) geometries leave lanes past a block's end, which must not write."""
    NB, BS, n = 48, 16, 64
    rng = np.random.default_rng(H * D + bits)
    ids_np = rng.permutation(NB)[:40].astype(np.int64)
    ids_np[[3, 17]] = [-1, NB + 5]          # out of the pool: zeros out, skipped in
    ids = torch.from_numpy(ids_np).to(dev)
    valid = torch.from_numpy((ids_np >= 0) & (ids_np < NB)).to(dev)
    caches, scales = [], []
    for i in range(n):
        kc, _, ks, _ = M.allocate_kv_cache(NB, BS, H, D, kv, device=dev)
        x = kv_values((NB * BS, H, D), dev, seed=300 + i)
        M.reshape_and_cache_flash(x, x, kc, kc.clone(), torch.arange(NB * BS, device=dev), kv, ks,
                                  None if ks is None else ks.clone())
        caches.append(kc)
        scales.append(ks)
    q, s = M.swap_out_caches(caches, ids, bits, scales)
    vid = ids[valid]
    for i in (0, 1, 31, 63):
        if kv == "int8":
            rq, rs = caches[i][vid], scales[i][vid]          # INT8 caches move as they are
        else:
            rq, rs = ref_quantize(caches[i][vid], bits)
        assert torch.equal(q[i][valid].view(rq.dtype), rq), i
        assert bool((q[i][~valid].view(torch.uint8) == 0).all()), i
        if rs is not None:
            assert torch.equal(s[i][valid], rs), i
            assert bool((s[i][~valid] == 0).all()), i
        qi, si = M.swap_out_blocks(caches[i], ids, bits, scales[i])
        assert torch.equal(q[i], qi), i
        if si is not None:
            assert torch.equal(s[i], si), i
    # restore into fresh caches: the swapped rows dequantised, every other block untouched
    fresh = [M.allocate_kv_cache(NB, BS, H, D, kv, device=dev) for _ in range(n)]
    tgt, tsc = [f[0] for f in fresh], [f[2] for f in fresh]
    M.swap_in_caches(q, s, bits, ids, tgt, tsc)
    for i in (0, 1, 31, 63):
        want = torch.zeros_like(tgt[i])
        if kv == "int8":
            want[vid] = caches[i][vid]
            want_s = torch.zeros_like(tsc[i])
            want_s[vid] = scales[i][vid]
            assert torch.equal(tsc[i], want_s), i
        else:
            want[vid] = ref_dequantize(q[i][valid], None if s is None else s[i][valid], bits)
        assert torch.equal(tgt[i].view(torch.uint8), want.view(torch.uint8)), i
        one, _, one_s, _ = M.allocate_kv_cache(NB, BS, H, D, kv, device=dev)
        M.swap_in_blocks(q[i], None if s is None else s[i], bits, ids, one, one_s)
        assert torch.equal(tgt[i].view(torch.uint8), one.view(torch.uint8)), i


@pytest.mark.parametrize("H,D", [(8, 128), (3, 128)])
def test_wide_swap_out_into_8_byte_aligned_rows(dev, H, D):
    """bf16 caches out at 8 bits into a buffer 8 bytes off 16-byte alignment (the C-ABI allows
    8): the one-chunk-a-lane kernel, equal to the two-chunks-a-lane form an aligned buffer
    gets (16-byte code stores), which the reference-line test above checks."""
    NB, BS, n = 48, 16, 64
    ids = torch.from_numpy(np.random.default_rng(D + H).permutation(NB)[:40].astype(np.int64)).to(dev)
    ids[5] = -1
    caches = []
    for i in range(n):
        kc, _, _, _ = M.allocate_kv_cache(NB, BS, H, D, "auto", device=dev)
        kc.copy_(kv_values((NB, BS, H, D), dev, seed=500 + i))
        caches.append(kc)
    q, s = M.swap_out_caches(caches, ids, 8)
    buf = torch.zeros(q.numel() + 16, dtype=torch.int8, device=dev)
    assert buf.data_ptr() % 16 == 0
    q8 = buf[8:8 + q.numel()].view(q.shape)
    q2, s2 = M.swap_out_caches(caches, ids, 8, out=q8)
    assert q2.data_ptr() % 16 == 8
    assert torch.equal(q2, q) and torch.equal(s2, s)
    assert not buf[:8].any() and not buf[8 + q.numel():].any()
