"""CPU: the golden fixtures under tests/golden/ (written by tests/golden/make_golden.py from the
oracle) hold the closed forms of their special cases, and the oracle still reproduces them.

Checks that do not go through the oracle:
  codec      zero vectors -> scale 0 and codes 0; |x| = amax -> +-127; exact .5 ties round
             to even; constant vectors -> all +-127; rows where torch-GPU's "tensor * fl(1/127)"
             and torch-CPU's true division disagree (63.5 +- 1 ulp -> 64 vs 63); every code
             within 1/2 of x / scale (engine/kv_tier_manager.py:21-31).
  accept     a float64 restatement of engine/spec_decode.py:37-49 (softmax, ratio,
             first rejection, residual, inverse CDF) agrees wherever the recorded margin is
             above 1e-5; p = q accepts everything; q[d] = 0 accepts; a uniform on its ratio
             rejects (the reference's `u >= ratio`); zero residual draws from p_k; greedy is
             the argmax prefix rule (tests/test_units.py:47-52).
  attention  a row that sees exactly one key returns that key's value; a per-(row, head)
             float64 loop reproduces the stored outputs.
"""
import os

import numpy as np
import pytest

from oracle import accept as OA
from oracle import codec as OC
from oracle import paged as OP

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def bf16(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16)


# ----------------------------------------------------------------------------- codec
def test_codec_fixture_special_cases():
    z = load("codec_int8.npz")
    x = bf16(z["x_bf16"])
    q, s = z["q8_device"], f16(z["s8_device"]).astype(np.float32)
    # zero vectors: scale 1e-8 / 127 underflows fp16 to 0, every code 0
    assert np.all(s[:2] == 0) and np.all(q[:2] == 0)
    # |x| = amax -> +-127 on every row with a non-zero amax that fp16 can represent
    clamped = 0
    for r in range(len(x)):
        a = np.abs(x[r]).max()
        if a == 0:
            continue
        i = int(np.abs(x[r]).argmax())
        if a < 1e-8:
            # clamp_min(1e-8): the scale is 1e-8 / 127 and amax maps below 127
            clamped += 1
            assert abs(int(q[r, i])) == round(float(a) / (1e-8 / 127)), r
            continue
        assert abs(int(q[r, i])) == 127 and np.sign(q[r, i]) == np.sign(x[r, i]), r
    assert clamped >= 1
    # rows 3..10: x = k + 0.5 against a scale of exactly 1: ties go to the even code
    inv = np.float32(1.0) / np.float32(127.0)
    assert np.float32(np.float32(127.0) * inv) == np.float32(1.0)
    for r in range(3, 11):
        half = x[r] - np.floor(x[r]) == 0.5
        assert half.sum() >= 100
        want = np.array([round(float(v)) for v in x[r][half]])  # Python round: half to even
        assert np.array_equal(q[r][half], want), r
    # constant vectors: every code +-127
    for r in range(43, 51):
        assert np.all(np.abs(q[r]) == 127), r
    # device vs CPU division disagree exactly on rows 60..63, at the x = amax / 2 elements
    qc = z["q8_cpu"]
    assert np.array_equal(q[:60], qc[:60])
    for r in range(60, 64):
        a = np.abs(x[r]).max()
        mid = np.abs(x[r]) == a / 2
        assert np.all(np.abs(q[r][mid]) == 64) and np.all(np.abs(qc[r][mid]) == 63), r
        assert np.array_equal(q[r][~mid], qc[r][~mid])


def test_codec_fixture_codes_within_half_step():
    """|x / s32 - code| <= 1/2 for unclamped codes, s32 the fp32 scale before fp16 rounding."""
    z = load("codec_int8.npz")
    x = bf16(z["x_bf16"]).astype(np.float64)
    amax = np.maximum(np.abs(x).max(-1), 1e-8)
    s32 = amax / 127.0
    t = x / s32[:, None]
    d = np.abs(t - z["q8_device"])
    assert np.all(d <= 0.5 + 1e-5)
    # INT4 round trip: |x - code * s16| <= s32 / 2 + 7 * |s32 - s16|, on rows whose fp16
    # scale is a normal number (>= 2^-14)
    s16 = f16(z["s4_device"]).astype(np.float64)
    d4 = OC.dequantize(z["q4_device"], f16(z["s4_device"]), 4)
    s4 = amax / 7.0
    normal = s16 >= 2.0 ** -14
    assert normal.sum() >= 50
    bound = 0.5 * s4 * (1 + 1e-6) + 7 * np.abs(s4 - s16)
    assert np.all(np.abs(d4 - x)[normal] <= bound[normal][:, None])


def test_oracle_reproduces_codec_fixture():
    z = load("codec_int8.npz")
    x = bf16(z["x_bf16"])
    for mode, qk, sk in (("device", "q8_device", "s8_device"), ("cpu", "q8_cpu", "s8_cpu")):
        q, s = OC.quantize(x, 8, mode)
        assert np.array_equal(q, z[qk]) and np.array_equal(s.view(np.uint16), z[sk])
    q, s = OC.quantize(x, 4, "device")
    assert np.array_equal(q, z["q4_device"]) and np.array_equal(s.view(np.uint16), z["s4_device"])


def test_codec_cpu_fixture_matches_torch_cpu_reference_lines():
    torch = pytest.importorskip("torch")
    z = load("codec_int8.npz")
    x = torch.from_numpy(z["x_bf16"].astype(np.int16)).view(torch.bfloat16)
    q, s = OC.quantize_torch_cpu(x, 8)
    assert np.array_equal(q.numpy(), z["q8_cpu"])
    assert np.array_equal(s.numpy().view(np.uint16), z["s8_cpu"])


# ----------------------------------------------------------------------------- accept
def softmax64(x, inv_t):
    x = np.asarray(x, np.float64) * float(inv_t)
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def verify64(tl, draft, dt, T, ua, ur, draft_is_probs):
    """engine/spec_decode.py:37-49 in float64, explicit uniforms, inverse-CDF draws."""
    inv_t = 1.0 / T
    p = softmax64(tl, inv_t)
    q = np.asarray(draft, np.float64) if draft_is_probs else softmax64(draft, inv_t)
    g = len(dt)
    k = g
    for i in range(g):
        ratio = min(1.0, p[i, dt[i]] / max(q[i, dt[i]], 1e-20))
        if ua[i] >= ratio:
            k = i
            break
    if k == g:
        w = p[g]
    else:
        w = np.maximum(p[k] - q[k], 0.0)
        if w.sum() <= 0:
            w = p[k]
    c = np.cumsum(w)
    tok = int(np.searchsorted(c, float(ur) * c[-1], side="right"))
    return list(dt[:k]) + [tok], k


def check_group(z, name, draft_is_probs=False):
    tl, dr, dt = z[f"{name}_target"], z[f"{name}_draft"], z[f"{name}_draft_tokens"]
    ua, ur, T = z[f"{name}_u_accept"], z[f"{name}_u_resample"], float(z[f"{name}_temperature"])
    acc, toks, marg = z[f"{name}_accepted_len"], z[f"{name}_tokens"], z[f"{name}_margin"]
    checked = 0
    for b in range(len(acc)):
        if marg[b] < 1e-5:
            continue
        out, k = verify64(tl[b], dr[b], dt[b], T, ua[b], ur[b], draft_is_probs)
        assert k == acc[b] and out == [int(t) for t in toks[b] if t >= 0], (name, b)
        checked += 1
    assert checked >= len(acc) // 2
    return tl, dr, dt, ua, ur, T, acc, toks, marg


def test_accept_v16_fixture_against_float64_restatement():
    z = load("accept_v16.npz")
    for name in ("t1", "t05"):
        tl, dr, dt, ua, ur, T, acc, toks, marg = check_group(z, name)
        g = dt.shape[1]
        assert acc[0] == g                              # p = q: every ratio is 1
        if name == "t1":
            assert acc[1] == g                          # q[d] = 0: ratio min(1, p / 1e-20) = 1
        assert acc[3] == 0 and marg[3] == 0             # u == ratio rejects (`u >= ratio`)
    tl, dr, dt, ua, ur, T, acc, toks, marg = check_group(z, "probs", draft_is_probs=True)
    # seq 2: q >= p elementwise, so the residual at the first rejection sums to 0 and the
    # token is drawn from p_k itself (engine/spec_decode.py:47-48)
    k = int(acc[2])
    assert k < dt.shape[1]
    p = softmax64(tl[2, k], 1.0 / T)
    assert np.all(np.maximum(OA.softmax32(tl[2, k]) - dr[2, k], 0) == 0)
    c = np.cumsum(p)
    assert toks[2, k] == int(np.searchsorted(c, float(ur[2]) * c[-1], side="right"))


def test_accept_v16_greedy_fixture_is_argmax_prefix_rule():
    z = load("accept_v16.npz")
    tl, dt = z["greedy_target"], z["greedy_draft_tokens"]
    acc, toks = z["greedy_accepted_len"], z["greedy_tokens"]
    am = tl.argmax(-1)
    for b in range(len(acc)):
        k = 0
        while k < dt.shape[1] and dt[b, k] == am[b, k]:
            k += 1
        assert acc[b] == k
        assert toks[b, :k + 1].tolist() == dt[b, :k].tolist() + [am[b, k]]


def fullv_inputs(z):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    B, g, V = int(z["B"]), int(z["gamma"]), int(z["V"])
    tl = mg.formula_logits([tuple(r) for r in z["target_params"]], V).reshape(B, g + 1, V)
    dl = mg.formula_logits([tuple(r) for r in z["draft_params"]], V).reshape(B, g, V)
    return tl, dl


def test_accept_fullv_fixture():
    z = load("accept_fullv.npz")
    tl, dl = fullv_inputs(z)
    dt, ua, ur = z["draft_tokens"], z["u_accept"], z["u_resample"]
    for b in range(int(z["B"])):
        assert z["margin"][b] > 1e-6
        out, k = verify64(tl[b], dl[b], dt[b], float(z["temperature"]), ua[b], ur[b], False)
        assert k == z["accepted_len"][b]
        assert out == [int(t) for t in z["tokens"][b] if t >= 0]
    # greedy with drafts = argmax of the target rows: everything accepted, bonus = argmax_g
    am = tl.argmax(-1)
    assert np.array_equal(z["greedy_accepted_len"], [4, 4])
    assert np.array_equal(z["greedy_tokens"], am)
    acc, toks, marg = OA.accept_batch(tl, dl, dt, float(z["temperature"]), ua, ur)
    assert np.array_equal(acc, z["accepted_len"]) and np.array_equal(toks, z["tokens"])


def test_oracle_reproduces_accept_v16_fixture():
    z = load("accept_v16.npz")
    for name in ("t1", "t05", "probs", "greedy"):
        acc, toks, marg = OA.accept_batch(z[f"{name}_target"], z[f"{name}_draft"],
                                          z[f"{name}_draft_tokens"], float(z[f"{name}_temperature"]),
                                          z[f"{name}_u_accept"], z[f"{name}_u_resample"],
                                          draft_is_probs=(name == "probs"))
        assert np.array_equal(acc, z[f"{name}_accepted_len"])
        assert np.array_equal(toks, z[f"{name}_tokens"])
        np.testing.assert_allclose(marg, z[f"{name}_margin"], rtol=0, atol=0)


# ----------------------------------------------------------------------------- attention
def attention_inputs(z):
    K = OP.dequantized_cache(z["k_codes"], f16(z["k_scale"]))
    V = OP.dequantized_cache(z["v_codes"], f16(z["v_scale"]))
    return bf16(z["q_bf16"]), K, V


def test_attention_fixture_closed_forms():
    z = load("attention_tiny.npz")
    q, K, V = attention_inputs(z)
    out, bs = z["out"], int(z["block_size"])
    cu, sl, tab = z["cu_seqlens_q"], z["seq_lens"], z["block_table"]
    Hq, Hkv = q.shape[1], K.shape[2]
    G = Hq // Hkv
    # sequence 2 has seq_len 5 and 5 new rows: its first row sees key 0 only
    b, r = 2, int(cu[2])
    assert sl[b] == cu[3] - cu[2]
    v0 = V[tab[b, 0], 0]                                  # [Hkv, D]
    np.testing.assert_allclose(out[r], np.repeat(v0, G, axis=0), rtol=0, atol=1e-6)
    # per-(row, head) float64 loop over the gathered keys
    for b in range(len(sl)):
        n, L = int(cu[b + 1] - cu[b]), int(sl[b])
        Kg, Vg = OP.gather(K, tab[b], L, bs), OP.gather(V, tab[b], L, bs)
        for j in range(n):
            vis = L - n + j + 1
            for h in range(0, Hq, 5):
                s = Kg[:vis, h // G].astype(np.float64) @ q[cu[b] + j, h].astype(np.float64)
                s *= 1.0 / np.sqrt(q.shape[-1])
                p = np.exp(s - s.max())
                o = (p / p.sum()) @ Vg[:vis, h // G].astype(np.float64)
                np.testing.assert_allclose(out[cu[b] + j, h], o, rtol=1e-5, atol=1e-6)


def test_oracle_reproduces_attention_fixture():
    z = load("attention_tiny.npz")
    q, K, V = attention_inputs(z)
    got = OP.attention(q, K, V, z["cu_seqlens_q"], z["seq_lens"], z["block_table"],
                       int(z["block_size"]))
    np.testing.assert_allclose(got, z["out"], rtol=1e-6, atol=1e-7)
