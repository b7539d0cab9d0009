"""CPU: the oracle Llama's layer wiring against transformers' LlamaForCausalLM.

oracle.spec_step.OracleLlama restates the reference's forward (engine/model.py:181-218) stage
by stage, and tests/test_oracle_spec_step.py pins each stage on its own.  This test pins the
wiring of the stages -- residual adds, which norm feeds which projection, the q/k/v and
gate/up splits, RoPE on q and k, GQA head grouping, the final norm and lm_head -- against an
independent implementation: transformers' Llama (random init from a config, no download;
eager attention), in float32 so that both sides compute the same function up to summation
order.  Cases: a prompt written to the paged cache in one item (prefill), then verify items of
5 rows appended at the prompt's end that read the prompt back from the cache (the
bottom-right causal mask and the cache addressing), for an untied and a tied-embedding model
at RoPE theta 500000.
"""
import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")

from oracle import spec_step as OS  # noqa: E402

V, HID, FFN, LAYERS, HEADS, KV, D, THETA = 384, 128, 256, 3, 4, 2, 32, 500000.0
BS, NB, MAXPOS = 16, 32, 128


def hf_and_oracle(tie, seed):
    cfg = transformers.LlamaConfig(
        vocab_size=V, hidden_size=HID, intermediate_size=FFN, num_hidden_layers=LAYERS,
        num_attention_heads=HEADS, num_key_value_heads=KV, head_dim=D, rope_theta=THETA,
        rms_norm_eps=1e-5, max_position_embeddings=MAXPOS, tie_word_embeddings=tie,
        attention_bias=False, mlp_bias=False)
    cfg._attn_implementation = "eager"
    hf = transformers.LlamaForCausalLM(cfg).eval()
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in hf.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_(torch.rand(p.shape, generator=g) + 0.5)     # norms that matter
            else:
                p.copy_(torch.randn(p.shape, generator=g) * 0.08)
    m = hf.model
    layers = []
    for L in m.layers:
        a, f = L.self_attn, L.mlp
        layers.append({
            "ln1": L.input_layernorm.weight.detach().clone(),
            "ln2": L.post_attention_layernorm.weight.detach().clone(),
            "qkv": torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]).detach().clone(),
            "o": a.o_proj.weight.detach().clone(),
            "gate_up": torch.cat([f.gate_proj.weight, f.up_proj.weight]).detach().clone(),
            "down": f.down_proj.weight.detach().clone(),
        })
    w = {"embed": m.embed_tokens.weight.detach().clone(),
         "lm_head": hf.lm_head.weight.detach().clone(),
         "norm": m.norm.weight.detach().clone(), "layers": layers}
    if tie:
        assert torch.equal(w["lm_head"], w["embed"])
    oracle = OS.OracleLlama(OS.Shape(HID, HEADS, KV, D, V, 1e-5, THETA), w, MAXPOS,
                            dtype=torch.float32)
    return hf, oracle


def fp32_cache(B, seed):
    layers = [(torch.zeros(NB, BS, KV, D), torch.zeros(NB, BS, KV, D), None, None)
              for _ in range(LAYERS)]
    perm = np.random.default_rng(seed).permutation(NB)[: B * (NB // B)]
    return OS.PagedCache(layers, perm.reshape(B, NB // B), BS, "auto", torch.float32)


@pytest.mark.parametrize("tie", [False, True])
def test_oracle_llama_matches_transformers_llama(tie):
    hf, oracle = hf_and_oracle(tie, seed=7 + tie)
    g = torch.Generator().manual_seed(3)
    lens = [37, 21]
    seqs = [torch.randint(0, V, (n + 5,), generator=g) for n in lens]
    with torch.no_grad():
        ref = [hf(s[None]).logits[0].float() for s in seqs]
    cache = fp32_cache(2, seed=5)
    # prefill: each prompt in one item, every row's logits
    pre = oracle.forward(cache, [(b, seqs[b][:n].tolist(), 0) for b, n in enumerate(lens)],
                         [True, True])
    # verify items: 5 rows at the prompt's end, reading the prompt's K/V back from the cache
    ver = oracle.forward(cache, [(b, seqs[b][n:].tolist(), n) for b, n in enumerate(lens)],
                         [True, True])
    got = [torch.cat([pre[:lens[0]], ver[:5]]), torch.cat([pre[lens[0]:], ver[5:]])]
    for b in range(2):
        scale = float(ref[b].abs().max())
        err = float((got[b] - ref[b]).abs().max()) / scale
        print(f"[hf llama tie={tie}] sequence {b}: max |logit diff| / max |logit| = {err:.2e} "
              f"(max |logit| {scale:.3g})", flush=True)
        assert err <= 2e-5, (b, err)
        assert torch.equal(got[b].argmax(-1), ref[b].argmax(-1))


def test_a_wiring_slip_is_caught():
    """The bar is tight enough to see a plausible slip: the oracle with its post-attention
    norm weight swapped for the input norm's differs from transformers by far more than 2e-5."""
    hf, oracle = hf_and_oracle(False, seed=11)
    for L in oracle.w["layers"]:
        L["ln2"] = L["ln1"]
    s = torch.randint(0, V, (20,), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        ref = hf(s[None]).logits[0].float()
    got = oracle.forward(fp32_cache(1, seed=1), [(0, s.tolist(), 0)], [True])
    assert float((got - ref).abs().max()) / float(ref.abs().max()) > 1e-2
