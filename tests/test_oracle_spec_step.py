"""CPU: pins oracle.spec_step (the step the GPU step is checked against).

* Stages reduce to pinned oracle functions: attention == oracle.paged.attention (float64
  closed form), cache slots == oracle.paged.slot_mapping, the INT8 write ==
  oracle.paged.kv_write_int8 (oracle.codec).
* Closed forms: RMSNorm of special vectors, RoPE as a rotation by pos * theta^(-2i/D) (the
  identity at position 0, pair norms kept), the RoPE tables of engine/model.py:120-124.
* Invariant: a prompt forwarded in one item equals the same prompt forwarded one token at a
  time through the paged cache (write-then-attend and the bottom-right causal mask).
* Hand-worked steps (logits injected through the hook, greedy and sampled): the proposal
  loop, accept / bonus rules, the reference's known answer (tests/test_units.py:47-52), lag 2
  after an all-accepted step, a lagging sequence's catch-up with gamma forced to 0, gamma 0,
  and the rollback of engine/engine.py:463-470.
"""
import math

import numpy as np
import pytest
import torch

from oracle import accept as OA
from oracle import paged as OP
from oracle import spec_step as OS

SHAPE = OS.Shape(hidden=64, heads=4, kv_heads=2, head_dim=16, vocab=40)


def tiny_weights(seed=0, shape=SHAPE, ffn=96, layers=2, std=0.2):
    g = torch.Generator().manual_seed(seed)
    w = lambda *s: (torch.randn(*s, generator=g) * std).to(torch.bfloat16)
    H, Hkv, D = shape.heads, shape.kv_heads, shape.head_dim
    return {"embed": w(shape.vocab, shape.hidden), "lm_head": w(shape.vocab, shape.hidden),
            "norm": torch.ones(shape.hidden, dtype=torch.bfloat16),
            "layers": [{"ln1": torch.ones(shape.hidden, dtype=torch.bfloat16),
                        "ln2": torch.ones(shape.hidden, dtype=torch.bfloat16),
                        "qkv": w((H + 2 * Hkv) * D, shape.hidden), "o": w(shape.hidden, H * D),
                        "gate_up": w(2 * ffn, shape.hidden), "down": w(shape.hidden, ffn)}
                       for _ in range(layers)]}


def make_cache(nslots, width, kv_dtype, shape=SHAPE, layers=2, bs=16, seed=0):
    rng = np.random.default_rng(seed)
    NB = nslots * width + 1
    table = rng.permutation(NB)[: nslots * width].reshape(nslots, width)
    Hkv, D = shape.kv_heads, shape.head_dim
    L = []
    for _ in range(layers):
        if kv_dtype == "int8":
            L.append((torch.zeros(NB, bs, Hkv, D, dtype=torch.int8), torch.zeros(NB, bs, Hkv, D, dtype=torch.int8),
                      torch.zeros(NB, bs, Hkv, dtype=torch.float16), torch.zeros(NB, bs, Hkv, dtype=torch.float16)))
        else:
            L.append((torch.zeros(NB, bs, Hkv, D, dtype=torch.bfloat16),
                      torch.zeros(NB, bs, Hkv, D, dtype=torch.bfloat16), None, None))
    return OS.PagedCache(L, table, bs, kv_dtype)


# ---- stages against pinned oracle functions -----------------------------------------------------
@pytest.mark.parametrize("kv", ["auto", "int8"])
def test_attend_and_write_reduce_to_oracle_paged(kv):
    g = torch.Generator().manual_seed(1)
    cache = make_cache(3, 8, kv, layers=1)
    items = [(0, [1] * 5, 37), (1, [1] * 1, 100), (2, [1] * 3, 0)]
    # fill every position each item attends to through the cache's own write
    for slot, toks, st in items:
        L = st + len(toks)
        k = torch.randn(L, 2, 16, generator=g).to(torch.bfloat16) * 3
        v = torch.randn(L, 2, 16, generator=g).to(torch.bfloat16) * 3
        cache.write(0, k, v, cache.slots(slot, 0, L))
    T = sum(len(t) for _, t, _ in items)
    q = torch.randn(T, 4, 16, generator=g).to(torch.bfloat16)
    got = OS.attend(q, cache, 0, items, 0.25).float().numpy()
    kc, vc, ks, vs = cache.layers[0]
    if kv == "int8":
        K = OP.dequantized_cache(kc.numpy(), ks.numpy())
        Vv = OP.dequantized_cache(vc.numpy(), vs.numpy())
    else:
        K, Vv = kc.float().numpy(), vc.float().numpy()
    cu = np.cumsum([0] + [len(t) for _, t, _ in items]).astype(np.int32)
    lens = np.array([st + len(t) for _, t, st in items], np.int32)
    ref = OP.attention(q.float().numpy(), K, Vv, cu, lens, cache.block_table, 16, 0.25)
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-3).all()
    # the write is oracle.paged's
    slots = np.concatenate([cache.slots(s, 0, st + len(t)) for s, t, st in items])
    for s, t, st in items:
        assert np.array_equal(cache.slots(s, st, st + len(t)),
                              OP.slot_mapping(cache.block_table[s], st, st + len(t), 16))
    if kv == "int8":
        k = torch.randn(4, 2, 16, generator=g).to(torch.bfloat16) * 20
        c2 = make_cache(3, 8, kv, layers=1)
        c2.write(0, k, k, slots[:4])
        kq = np.zeros_like(c2.layers[0][0].numpy())
        ksn = np.zeros_like(c2.layers[0][2].numpy())
        OP.kv_write_int8(kq, kq.copy(), ksn, ksn.copy(), k.float().numpy(), k.float().numpy(),
                         slots[:4], 16)
        assert np.array_equal(c2.layers[0][0].numpy(), kq)
        assert np.array_equal(c2.layers[0][2].numpy(), ksn)


# ---- closed forms ------------------------------------------------------------------------------
def test_rms_norm_closed_forms():
    w = torch.full((8,), 2.0, dtype=torch.bfloat16)
    # constant vector c: c / sqrt(c^2 + eps) ~= sign(c)
    for c in (0.5, -3.0, 100.0):
        x = torch.full((1, 8), c, dtype=torch.bfloat16)
        want = 2.0 * c / math.sqrt(c * c + 1e-5)
        assert torch.allclose(OS.rms_norm(x, w, 1e-5).float(), torch.full((1, 8), want), rtol=8e-3)
    # [3, 4, 0 ...]: rms = 5 / sqrt(8)
    x = torch.tensor([[3.0, 4.0, 0, 0, 0, 0, 0, 0]], dtype=torch.bfloat16)
    r = 5.0 / math.sqrt(8)
    want = torch.tensor([[3 / r, 4 / r, 0, 0, 0, 0, 0, 0]]) * 2
    assert torch.allclose(OS.rms_norm(x, w, 0.0).float(), want, rtol=8e-3)


def test_rope_is_a_rotation_by_position_times_frequency():
    D, theta = 16, 500000.0
    cos, sin = OS.rope_tables(theta, D, 4096, dtype=torch.float32)
    for p in (0, 1, 7, 1000, 4095):
        for i in range(D // 2):
            e = torch.zeros(1, 1, D)
            e[0, 0, i] = 1.0
            ang = p * theta ** (-2 * i / D)
            want = torch.zeros(D)
            want[i], want[i + D // 2] = math.cos(ang), math.sin(ang)
            # the oracle Llama's form: q * cos + rotate_half(q) * sin
            r = e * cos[p] + OS.rotate_half(e) * sin[p]
            assert torch.allclose(r[0, 0], want, atol=1e-4)
    c16, s16 = OS.rope_tables(theta, D, 8)
    assert c16.dtype == torch.bfloat16 and torch.equal(c16[0], torch.ones(D, dtype=torch.bfloat16))


# ---- the forward's invariant -------------------------------------------------------------------
@pytest.mark.parametrize("kv", ["auto", "int8"])
def test_prompt_in_one_item_equals_token_by_token(kv):
    w = tiny_weights(4)
    m = OS.OracleLlama(SHAPE, w, 256)
    toks = [3, 17, 5, 5, 39, 0, 12, 8, 30, 21, 2, 9, 14, 33, 1, 7, 26, 11, 4, 19]
    a = make_cache(1, 4, kv)
    full = m.forward(a, [(0, toks, 0)], [True])
    b = make_cache(1, 4, kv)
    rows = [m.forward(b, [(0, [t], i)], [False]) for i, t in enumerate(toks)]
    inc = torch.cat(rows)
    assert full.shape == (len(toks), SHAPE.vocab)
    err = float((full - inc).abs().max() / full.abs().max())
    assert err <= 3e-2, err
    assert (full.argmax(-1) == inc.argmax(-1)).float().mean() >= 0.9


# ---- hand-worked steps (logits injected through the hook) --------------------------------------
def onehot(ids, V=SHAPE.vocab):
    x = torch.full((len(ids), V), -30.0)
    x[torch.arange(len(ids)), torch.tensor(ids)] = 30.0
    return x


def run_step(seqs, T, target_argmax, draft_argmax, u=None, cap=None):
    """Greedy or sampled step where the draft's round-i logits favour draft_argmax[b][i] and
    the target's verify rows favour target_argmax[b][j]."""
    w = tiny_weights(5)
    tm, dm = OS.OracleLlama(SHAPE, w, 256), OS.OracleLlama(SHAPE, w, 256)
    tc, dcache = make_cache(len(seqs), 8, "int8"), make_cache(len(seqs), 8, "auto", seed=1)
    seen = []

    def hook(stage, i, slots, mine):
        seen.append((stage, i, list(slots), mine.shape[0]))
        if stage == "draft":
            return onehot([draft_argmax[b][i] for b in slots])
        rows = []
        for b in slots:
            n = sum(1 for s, _, sl, _ in seen if s == "draft" and b in sl) + 1
            rows += target_argmax[b][:n]
        return onehot(rows)

    B = len(seqs)
    gmax = max(s.gamma for s in seqs) or 1
    u_draft = np.full((gmax, B), 0.5, np.float32) if u is None else u[0]
    u_acc = np.full((B, gmax), 0.5, np.float32) if u is None else u[1]
    u_res = np.full(B, 0.5, np.float32) if u is None else u[2]
    rec, own = OS.step(seqs, tm, dm, tc, dcache, T, u_draft, u_acc, u_res, catchup_cap=cap,
                       logits_hook=hook)
    return rec, seen, tc, dcache


def test_hand_worked_greedy_step():
    # seq 0: lag 1, gamma 3, drafts [3, 5, 1] vs target argmax [3, 5, 7, 9] -> [3, 5, 7]
    #        (tests/test_units.py:47-52)
    # seq 1: lag 2 (previous step accepted everything), gamma 3, all accepted -> + bonus
    # seq 2: gamma 0: one target token, the draft untouched
    # seq 3: lagging (lag 6), gamma 2: catch-up over 5 tokens, gamma forced to 0
    seqs = [OS.Seq(list(range(10)), 9, 9, 3),
            OS.Seq(list(range(12)), 11, 10, 3),
            OS.Seq(list(range(8)), 7, 3, 0),
            OS.Seq(list(range(20)), 19, 14, 2)]
    tgt = {0: [3, 5, 7, 9], 1: [4, 6, 8, 2], 2: [11], 3: [13]}
    drf = {0: [3, 5, 1], 1: [4, 6, 8]}
    rec, seen, tc, dcache = run_step(seqs, 0.0, tgt, drf)
    assert [r.drafts for r in rec] == [[3, 5, 1], [4, 6, 8], [], []]
    assert [r.new for r in rec] == [[3, 5, 7], [4, 6, 8, 2], [11], [13]]
    assert [r.k for r in rec] == [2, 3, 0, 0]
    assert [r.catchup for r in rec] == [1, 2, 0, 5]
    # rounds: 0 from the catch-up logits of seqs 0 and 1, then two single-token rounds
    assert [(s, i, sl) for s, i, sl, _ in seen if s == "draft"] == \
        [("draft", 0, [0, 1]), ("draft", 1, [0, 1]), ("draft", 2, [0, 1])]
    assert seen[-1][:3] == ("target", 0, [0, 1, 2, 3]) and seen[-1][3] == 4 + 4 + 1 + 1
    # rollback: num_computed = len - 1; draft_computed = min(after drafting, len - 1)
    assert [len(s.tokens) for s in seqs] == [13, 16, 9, 21]
    assert [s.num_computed for s in seqs] == [12, 15, 8, 20]
    # seq 0 drafted to 10 + 2 = 12; seq 1 to 12 + 2 = 14 < 15; seq 2 untouched; seq 3 to 19
    assert [s.draft_computed for s in seqs] == [12, 14, 3, 19]
    assert [s.gamma for s in seqs] == [3, 3, 0, 0]
    # the target wrote positions num_computed .. num_computed + gamma of each sequence
    want = np.concatenate([tc.slots(0, 9, 13), tc.slots(1, 11, 15), tc.slots(2, 7, 8),
                           tc.slots(3, 19, 20)])
    assert sorted(tc.written) == sorted(want.tolist())
    wd = np.concatenate([dcache.slots(0, 9, 12), dcache.slots(1, 10, 14), dcache.slots(3, 14, 19)])
    assert sorted(dcache.written) == sorted(wd.tolist())


def test_capped_catch_up_spans_steps():
    seqs = [OS.Seq(list(range(30)), 29, 10, 2)]
    rec, *_ = run_step(seqs, 0.0, {0: [1]}, {}, cap=8)
    assert rec[0].catchup == 8 and rec[0].drafts == [] and seqs[0].draft_computed == 18
    assert len(seqs[0].tokens) == 31


def test_sampled_step_uses_the_uniforms_as_verify_does():
    # one sequence, gamma 2; the hook's logits make p and q explicit
    V = SHAPE.vocab
    seqs = [OS.Seq(list(range(10)), 9, 9, 2)]
    g = torch.Generator().manual_seed(9)
    dl = torch.randn(2, V, generator=g) * 2
    tl = torch.randn(3, V, generator=g) * 2
    u_draft = np.array([[0.3], [0.8]], np.float32)
    u_acc = np.array([[0.2, 0.9]], np.float32)
    u_res = np.array([0.6], np.float32)
    w = tiny_weights(6)
    tm, dm = OS.OracleLlama(SHAPE, w, 256), OS.OracleLlama(SHAPE, w, 256)

    def hook(stage, i, slots, mine):
        return dl[i:i + 1] if stage == "draft" else tl

    rec, _ = OS.step(seqs, tm, dm, make_cache(1, 8, "int8"), make_cache(1, 8, "auto"), 1.0,
                     u_draft, u_acc, u_res, logits_hook=hook)
    q = OA.softmax32(dl.numpy())
    d = [OA.inverse_cdf(q[0], 0.3)[0], OA.inverse_cdf(q[1], 0.8)[0]]
    want, k, _ = OA.verify(tl.numpy(), d, dl.numpy(), 1.0, u_acc[0], u_res[0])
    assert rec[0].drafts == d and rec[0].new == want and rec[0].k == k
    assert seqs[0].tokens == list(range(10)) + want
