"""GPU: the fused qkv epilogue (coopt_qkv_epilogue: split, neox RoPE, q out, K/V into the
paged cache; engine/model.py:238-243) against the unfused kernels it replaces.

Bar: bit-exact -- q, every cache byte (codes, scales, bf16 values) -- against
coopt_linear + coopt_rope + coopt_kv_write, from the bf16 projection output and from its
split-K partials, with bf16 and INT8 caches; rows with slot -1 write no cache entry.
"""
import numpy as np
import pytest
import torch

import iitj_llm_coopt_amd as M
from iitj_llm_coopt_amd import fused

pytestmark = pytest.mark.gpu


def tables(D, max_pos, dev):
    inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    f = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv)
    emb = torch.cat((f, f), -1)
    return emb.cos().to(dev, torch.bfloat16), emb.sin().to(dev, torch.bfloat16)


@pytest.mark.parametrize("kv", ["auto", "int8"])
@pytest.mark.parametrize("T,Hq,Hkv,D,K", [(160, 32, 8, 128, 4096), (32, 32, 8, 64, 2048),
                                          (7, 4, 2, 128, 256),
                                          (160, 8, 2, 64, 4352)])   # K split 7 ways
@pytest.mark.parametrize("deferred", [False, True])
def test_epilogue_equals_unfused_chain(dev, kv, T, Hq, Hkv, D, K, deferred):
    g = torch.Generator(device=dev).manual_seed(T + D + K)
    rng = np.random.default_rng(T + D)
    N = (Hq + 2 * Hkv) * D
    h = torch.randn(T, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.03).to(torch.bfloat16)
    max_pos = 4096
    cos, sin = tables(D, max_pos, dev)
    pos = torch.from_numpy(rng.integers(0, max_pos + 50, T)).to(dev)        # some clamped
    NB, bs = -(-T // 16) * 4 + 3, 16
    slots = torch.from_numpy(rng.permutation(NB * bs)[:T].astype(np.int64)).to(dev)
    slots[::5] = -1                                                         # padding rows
    caches = [M.allocate_kv_cache(NB, bs, Hkv, D, kv, device=dev) for _ in range(2)]
    for c in caches:
        for t in c:
            if t is not None:
                t.zero_()
    # unfused: projection, RoPE in place on the views, KV write
    qkv = fused.linear(h, w)
    q_ref = qkv[:, : Hq * D].reshape(T, Hq, D).clone()
    k_ref = qkv[:, Hq * D: (Hq + Hkv) * D].reshape(T, Hkv, D).clone()
    v_ref = qkv[:, (Hq + Hkv) * D:].reshape(T, Hkv, D)
    fused.rope_(q_ref, k_ref, pos, cos, sin)
    kc, vc, ks, vs = caches[0]
    M.reshape_and_cache_flash(k_ref, v_ref.contiguous(), kc, vc, slots, kv, ks, vs)
    # fused
    kc2, vc2, ks2, vs2 = caches[1]
    src = fused.linear(h, w, defer_reduce=True) if deferred else qkv
    if deferred:
        assert isinstance(src, fused.LinearPartials)
        print(f"[qkv epilogue] T={T} D={D} {kv}: {src.ks} slice(s)", flush=True)
    q = M.qkv_rope_and_cache(src, pos, cos, sin, kc2, vc2, slots, Hq, Hkv, D, kv, ks2, vs2)
    assert torch.equal(q, q_ref)
    assert torch.equal(kc2, kc) and torch.equal(vc2, vc)
    if kv == "int8":
        assert torch.equal(ks2, ks) and torch.equal(vs2, vs)
