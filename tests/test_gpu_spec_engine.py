"""GPU: the full speculative step (draft proposals -> paged verify -> fused accept -> rollback)
on tiny Llama-shaped models.

Checks the bookkeeping of engine/engine.py:463-470, greedy losslessness (speculative greedy
decoding reproduces plain greedy decoding of the target -- the reference's q2 check,
eval/quality.py:87-116), an identical draft being accepted, and HIP-graph replays of a whole
step against eager steps (several replays with eager work in between).
"""
import numpy as np
import pytest
import torch

from iitj_llm_coopt_amd.spec_engine import HipOps, LlamaShape, PagedKV, RandomLlama, SpecDecoder

pytestmark = pytest.mark.gpu

TINY_T = LlamaShape(hidden=256, ffn=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000)
TINY_D = LlamaShape(hidden=128, ffn=256, layers=1, heads=4, kv_heads=2, head_dim=64, vocab=1000,
                    tie_embeddings=True)


def report(msg):
    print(msg, flush=True)


def make(dev, B=4, gamma=3, P=24, steps=8, T=1.0, draft_same=False, target_kv="int8", seed=0,
         std=0.2):
    t = RandomLlama(TINY_T, dev, seed=seed + 1, std=std)
    d = t if draft_same else RandomLlama(TINY_D, dev, seed=seed + 2, std=std,
                                         packed=("qkv", "o", "gate_up", "down", "lm_head"))
    dec = SpecDecoder(t, d, B, gamma, P, steps, target_kv=target_kv,
                      draft_kv=target_kv if draft_same else "auto", temperature=T, seed=seed)
    g = torch.Generator(device=dev).manual_seed(seed + 3)
    prompts = torch.randint(0, TINY_T.vocab, (B, P), generator=g, device=dev)
    dec.prefill(prompts, torch.rand(B, generator=g, device=dev))
    return dec


def test_step_bookkeeping(dev):
    dec = make(dev, T=1.0)
    B, g = dec.B, dec.g
    for _ in range(6):
        n0 = dec.n.clone()
        e0 = int(dec.emitted)
        dec.step()
        n1 = dec.n
        acc = dec.res.accepted_len.long()
        assert torch.equal(n1, n0 + acc + 1)
        assert torch.equal(dec.dc, torch.minimum(n0 + g - 1, n1 - 1))
        assert int(dec.emitted) - e0 == int((n1 - n0).sum())
        assert bool(((acc >= 0) & (acc <= g)).all())
        for b in range(B):
            toks = dec.hist[b, : int(n1[b])]
            assert bool(((toks >= 0) & (toks < TINY_T.vocab)).all())
            # the accepted prefix is the drafts, then the kernel's token
            k = int(acc[b])
            assert dec.hist[b, int(n0[b]): int(n0[b]) + k].tolist() == dec.draft_tok[b, :k].tolist()
            assert int(dec.hist[b, int(n0[b]) + k]) == int(dec.res.tokens[b, k])


def plain_greedy(dec, new_tokens):
    """Autoregressive greedy decoding of the target alone (q_len 1 per step) from the state
    right after prefill: the reference's no-speculation path."""
    t, B, dev = dec.t, dec.B, dec.hist.device
    kv = dec.tkv
    ops = HipOps(dev)
    n = dec.n.clone()
    hist = dec.hist.clone()
    cu = torch.arange(B + 1, dtype=torch.int32, device=dev)
    for _ in range(new_tokens):
        pos = (n - 1).unsqueeze(1)
        slots = kv.slots(pos)
        meta = (cu, n.to(torch.int32), 1, dec.max_len)
        logits = t.forward(ops, kv, hist.gather(1, pos).reshape(-1), pos.reshape(-1), slots, meta)
        nxt = logits.float().argmax(-1)
        hist.scatter_(1, n.unsqueeze(1), nxt.unsqueeze(1))
        n = n + 1
    return hist, n


def test_greedy_speculation_reproduces_target_greedy(dev):
    """With temperature 0 the output must be the target's greedy continuation whatever the
    draft proposes (up to argmax flips from bf16 GEMM shapes, which are counted)."""
    dec = make(dev, B=4, gamma=4, P=24, steps=12, T=0.0, target_kv="auto")
    P1 = int(dec.n[0])
    ref_hist, _ = plain_greedy(make(dev, B=4, gamma=4, P=24, steps=12, T=0.0, target_kv="auto"), 16)
    for _ in range(8):
        dec.step()
    n = int(dec.n.min())
    got = dec.hist[:, P1:n].cpu().numpy()
    ref = ref_hist[:, P1:n].cpu().numpy()
    # position of the first divergence per sequence (a flip changes everything after it)
    first = [int(np.argmax(g != r)) if (g != r).any() else g.size for g, r in zip(got, ref)]
    report(f"[spec-greedy] generated {n - P1} tokens/seq; first divergence {first}")
    assert sum(f >= min(8, n - P1) for f in first) >= 3


def test_identical_draft_is_accepted(dev):
    """draft == target (same weights, same KV format), greedy: every draft matches the
    target's argmax except for rare bf16 flips between the q_len 1/2 and q_len 5 forwards."""
    dec = make(dev, B=4, gamma=4, P=24, steps=8, T=0.0, draft_same=True, target_kv="auto")
    for _ in range(6):
        dec.step()
    rate = int(dec.accepted) / int(dec.drafted)
    report(f"[identical draft] acceptance {rate:.3f}")
    assert rate >= 0.9


def test_graph_replays_match_eager_steps(dev):
    """Greedy, so the step is deterministic: replays of a captured step must equal eager
    steps from the same start, with eager work and syncs between replays."""
    a = make(dev, B=4, gamma=3, P=24, steps=12, T=0.0, seed=7)
    b = make(dev, B=4, gamma=3, P=24, steps=12, T=0.0, seed=7)
    assert torch.equal(a.hist, b.hist)
    a.step()
    b.step()
    b.capture()      # records the next step's bucket; leaves the state as it was
    assert torch.equal(a.hist, b.hist) and torch.equal(a.n, b.n)
    for i in range(4):
        b.replay()
        a.step()
        torch.cuda.synchronize(dev)
        _ = torch.randn(1000, device=dev).sum().item()  # unrelated eager work between replays
        assert torch.equal(a.n, b.n), i
        assert torch.equal(a.hist, b.hist), i
