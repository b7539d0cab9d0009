"""GPU: coopt_verify_attention_qkv (the qkv epilogue inside the attention launch) against the
two launches it replaces -- coopt_qkv_epilogue then coopt_verify_attention -- from identical
caches.  Bar: the attention output and every cache entry (codes, scales, bf16 values)
bit-identical.  Those two launches are pinned against the oracle by test_gpu_qkv_epilogue.py
and test_gpu_attention.py.

Layout as the speculative step builds it (engine/cuda_graphs.py:76-104): every sequence owns
S rows, its first n_real rows are real (key positions ctx + j), the rest are padding (slot -1),
and seq_len = ctx + S.
"""
import math

import numpy as np
import pytest
import torch

import iitj_llm_coopt_amd as M
from iitj_llm_coopt_amd.fused import linear

pytestmark = pytest.mark.gpu


def report(msg):
    print(msg, flush=True)


def rope_tables(max_pos, D, dev, theta=500000.0):
    inv = theta ** (-torch.arange(0, D // 2, dtype=torch.float64) * 2 / D)
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None, :]
    return ang.cos().to(torch.bfloat16).to(dev), ang.sin().to(torch.bfloat16).to(dev)


def build(dev, B, Hq, Hkv, D, S, ctx, n_real, kv, qkv_kind, seed, bs=16, pos_shift=None,
          token_major=False):
    gen = torch.Generator(device=dev).manual_seed(seed)
    rng = np.random.default_rng(seed)
    W = [-(-(c + S) // bs) for c in ctx]
    NB = sum(W) + 4
    perm = rng.permutation(NB)
    table = np.zeros((B, max(W)), np.int32)
    o = 0
    for b in range(B):
        table[b, :W[b]] = perm[o:o + W[b]]
        o += W[b]
    if token_major:
        # the reference's own layout: token-major caches and scales (scale token stride Hkv)
        cdt = torch.int8 if kv == "int8" else torch.bfloat16
        kc = torch.zeros(NB, bs, Hkv, D, dtype=cdt, device=dev)
        vc = torch.zeros_like(kc)
        ks = torch.zeros(NB, bs, Hkv, dtype=torch.float16, device=dev) if kv == "int8" else None
        vs = None if ks is None else torch.zeros_like(ks)
    else:
        kc, vc, ks, vs = M.allocate_kv_cache(NB, bs, Hkv, D, kv, device=dev)
    # the cached context, written through the KV write
    ctx_slots = np.concatenate([table[b][np.arange(ctx[b]) // bs] * bs + np.arange(ctx[b]) % bs
                                for b in range(B)]).astype(np.int64)
    Tc = ctx_slots.size
    k0 = torch.randn(Tc, Hkv, D, generator=gen, device=dev).to(torch.bfloat16)
    v0 = torch.randn(Tc, Hkv, D, generator=gen, device=dev).to(torch.bfloat16)
    M.reshape_and_cache_flash(k0, v0, kc, vc, torch.from_numpy(ctx_slots).to(dev), kv, ks, vs)
    pos, slots = [], []
    for b in range(B):
        for j in range(S):
            p = ctx[b] + j
            pos.append(p + (pos_shift(b, j) if pos_shift else 0))
            slots.append(int(table[b][p // bs]) * bs + p % bs if j < n_real[b] else -1)
    T = B * S
    hidden = 4096 if D == 128 else 2048     # the target's and the draft's hidden sizes
    h = (torch.randn(T, hidden, generator=gen, device=dev) * 0.5).to(torch.bfloat16)
    w = (torch.randn((Hq + 2 * Hkv) * D, hidden, generator=gen, device=dev) * 0.05).to(torch.bfloat16)
    qkv = linear(h, w, defer_reduce=(qkv_kind == "partials"))
    if qkv_kind == "partials":
        assert isinstance(qkv, M.fused.LinearPartials), "expected the split-K kernel path"
        assert 1 <= qkv.ks <= 4, qkv.ks
        report(f"[fused qkv] B={B} S={S} D={D}: {qkv.ks} K slice(s)")
    cos, sin = rope_tables(max(max(pos), max(c + S for c in ctx)) + 8, D, dev)
    meta = dict(pos=torch.tensor(pos, dtype=torch.int64, device=dev),
                slots=torch.tensor(slots, dtype=torch.int64, device=dev),
                cu=(torch.arange(B + 1, dtype=torch.int32, device=dev) * S),
                seq=torch.tensor([c + S for c in ctx], dtype=torch.int32, device=dev),
                table=torch.from_numpy(table).to(dev), S=S, max_k=max(c + S for c in ctx),
                cos=cos, sin=sin)
    return (kc, vc, ks, vs), qkv, meta


def run_both(caches, qkv, m, Hq, Hkv, D, kv):
    kc, vc, ks, vs = caches
    copy = [None if x is None else x.clone() for x in caches]
    scale = 1.0 / math.sqrt(D)
    # two launches on the original caches
    q = M.qkv_rope_and_cache(qkv, m["pos"], m["cos"], m["sin"], kc, vc, m["slots"], Hq, Hkv, D,
                             kv, ks, vs)
    ref = M.paged_attention(q, kc, vc, m["cu"], m["seq"], m["table"], m["S"], m["max_k"], scale,
                            ks, vs)
    # one launch on the copy
    got = M.paged_attention_qkv(qkv, m["pos"], m["cos"], m["sin"], m["slots"], copy[0], copy[1],
                                m["cu"], m["seq"], m["table"], m["S"], m["max_k"], Hq, scale, kv,
                                copy[2], copy[3])
    torch.cuda.synchronize()
    return ref, got, caches, copy


CASES = [
    # (label, kv, D, B, S, qkv input) -- the step's target verify, its draft proposal and
    # catch-up, a bf16 head_dim-128 verify at 4 rows per sequence
    ("int8 D128 S5 partials", "int8", 128, 32, 5, "partials"),
    ("int8 D128 S5 bf16 rows", "int8", 128, 32, 5, "bf16"),
    ("bf16 D64 S1 partials", "auto", 64, 32, 1, "partials"),
    ("bf16 D64 S2 partials", "auto", 64, 32, 2, "partials"),
    ("bf16 D128 S4 bf16 rows", "auto", 128, 32, 4, "bf16"),
    ("int8 D128 S8, 64 sequences (ordered grid)", "int8", 128, 64, 8, "bf16"),
    # the other instantiations the call can reach: INT8 at head_dim 64, bf16 head_dim 128
    # from partials at one row tile, and INT8 over the reference's token-major scale caches
    ("int8 D64 S2 partials", "int8", 64, 32, 2, "partials"),
    ("int8 D64 S5 bf16 rows", "int8", 64, 32, 5, "bf16"),
    ("bf16 D128 S2 partials", "auto", 128, 32, 2, "partials"),
    ("int8 D128 S5 partials, token-major scales", "int8", 128, 32, 5, "partials-tm"),
    ("int8 D128 S2 bf16 rows, token-major scales", "int8", 128, 32, 2, "bf16-tm"),
]


@pytest.mark.parametrize("label,kv,D,B,S,kind", CASES)
def test_fused_equals_epilogue_then_attention(dev, label, kv, D, B, S, kind):
    Hq, Hkv = 32, 8
    rng = np.random.default_rng(B * 10 + S)
    ctx = rng.integers(30, 1200, B).tolist()
    ctx[0] = 0                                   # a sequence whose only keys are its new ones
    n_real = rng.integers(1, S + 1, B).tolist()  # ragged real rows, the rest padding
    n_real[1] = S
    assert M.qkv_attention_supported(kv, B, Hq, Hkv, D, S, max(c + S for c in ctx)), label
    tm = kind.endswith("-tm")
    caches, qkv, m = build(dev, B, Hq, Hkv, D, S, ctx, n_real, kv, kind.removesuffix("-tm"),
                           seed=B + S, token_major=tm)
    ref, got, ca, cb = run_both(caches, qkv, m, Hq, Hkv, D, kv)
    report(f"[fused qkv] {label}: max |diff| {float((ref.float() - got.float()).abs().max()):.3g}")
    assert torch.equal(ref, got), label
    for x, y in zip(ca, cb):
        if x is not None:
            assert torch.equal(x, y), f"{label}: caches differ"


def test_positions_other_than_key_positions(dev):
    """RoPE positions that differ from the rows' key positions (the kernel loads the table rows
    of the key position first and reloads on a mismatch), including one past the table."""
    B, S, D, Hq, Hkv, kv = 32, 5, 128, 32, 8, "int8"
    rng = np.random.default_rng(5)
    ctx = rng.integers(30, 900, B).tolist()
    n_real = [S] * B

    def shift(b, j):
        return 0 if b % 3 == 0 else (3 * b + j if b % 3 == 1 else -(ctx[b] + j) - 5 + 4 * j)

    caches, qkv, m = build(dev, B, Hq, Hkv, D, S, ctx, n_real, kv, "partials", seed=11,
                           pos_shift=shift)
    # a table that ends before the largest position: that row reads the last table row
    m["cos"], m["sin"] = m["cos"][:-9], m["sin"][:-9]
    ref, got, ca, cb = run_both(caches, qkv, m, Hq, Hkv, D, kv)
    report(f"[fused qkv] shifted positions: max |diff| {float((ref.float() - got.float()).abs().max()):.3g}")
    assert torch.equal(ref, got)
    for x, y in zip(ca, cb):
        if x is not None:
            assert torch.equal(x, y), "caches differ"


def test_unsupported_shapes_are_refused(dev):
    # 36 rows per KV head (q_len 9 at 4 query heads per KV head), and a batch whose long
    # contexts are split across blocks
    assert not M.qkv_attention_supported("int8", 32, 32, 8, 128, 9, 1200)
    assert not M.qkv_attention_supported("int8", 2, 32, 8, 128, 5, 4000)
    assert not M.qkv_attention_supported("auto", 32, 32, 8, 128, 8, 1200)  # bf16 D128, 32 rows
    caches, qkv, m = build(dev, 2, 32, 8, 128, 5, [3000, 3900], [5, 5], "int8", "partials", 1)
    kc, vc, ks, vs = caches
    with pytest.raises(ValueError, match="not supported"):
        M.paged_attention_qkv(qkv, m["pos"], m["cos"], m["sin"], m["slots"], kc, vc, m["cu"],
                              m["seq"], m["table"], m["S"], m["max_k"], 32, None, "int8", ks, vs)
