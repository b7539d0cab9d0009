"""Writes the golden fixtures of the verify/accept + paged-KV path (tests/golden/*.npz).

    python tests/golden/make_golden.py

Every fixture is data: inputs and the expected outputs of the reference's algorithm, computed
by the CPU oracle (oracle/), which restates engine/kv_tier_manager.py:21-41,
engine/spec_decode.py:12-49 and engine/model.py:244-247.  The special cases each fixture holds
(zero vectors, exact .5 ties, x20 outliers, p = q, q[d] = 0, zero residual, uniforms exactly on
the accept boundary, single-key causal rows) are checked against their closed forms in
tests/test_golden.py, and the GPU kernels are checked against the files in
tests/test_gpu_golden.py.  Files are written with numpy.savez_compressed (no pickled objects).

  codec_int8.npz      64 (token, head) vectors of D=128 (bf16 bits) -> INT8 codes + fp16 scales
                      (torch-GPU "tensor / scalar" semantics and torch-CPU true division), and
                      INT4 packed codes + scales.
  accept_v16.npz      rejection sampling at V=16: draft logits (T=1 and T=0.5), draft
                      probabilities given directly (zero-residual fallback), greedy.
  accept_fullv.npz    two sequences at V=128256, logits generated from integer formulas
                      (exact in fp32; the formula parameters are stored, not the logits).
  attention_tiny.npz  the geometry of tests/strided_kv_check.py:19-22 (seq_lens [37, 200, 5],
                      q_lens [1, 3, 5], Hq 32, Hkv 8, D 128, block size 16): INT8 codes + fp16
                      scales, bf16 q, float32 outputs of attention over the dequantised cache
                      (equal for the bf16 path given bf16(code * scale)).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import accept as OA  # noqa: E402
from oracle import codec as OC  # noqa: E402
from oracle import paged as OP  # noqa: E402

VOCAB = 128256


def bf16_bits(x):
    """float32 array -> uint16 bf16 bit patterns (round to nearest even)."""
    return (OC.bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------- codec
def codec_vectors(rng):
    D = 128
    rows = []
    rows.append(np.zeros(D, np.float32))                                   # 0: all zero
    rows.append(np.full(D, -0.0, np.float32))                              # 1: negative zeros
    v = np.zeros(D, np.float32)
    v[5] = 3.0                                                             # 2: one non-zero
    rows.append(v)
    # 3..10: exact .5 ties.  With amax = 127 the device scale is 127 * fl(1/127), which is
    # not 1, so ties are built against the computed scale: x = (k + 0.5) * s for small k.
    for i in range(8):
        s = np.float32(np.float32(127.0) * (np.float32(1.0) / np.float32(127.0)))
        ks = np.arange(-64, 64, dtype=np.float32)
        x = ((ks + np.float32(0.5)) * s).astype(np.float32)
        x[0] = np.float32(127.0)                                           # amax
        rows.append(OC.bf16_round(np.roll(x, i)))
    # 11..26: N(0,1) with x20 outliers (1% per element, plus one forced)
    for i in range(16):
        x = rng.standard_normal(D).astype(np.float32)
        mask = rng.random(D) < 0.01
        mask[rng.integers(D)] = True
        x[mask] *= 20
        rows.append(OC.bf16_round(x))
    # 27..34: tiny magnitudes (fp16 scale subnormal / underflow to 0)
    for e in (-10, -14, -16, -18, -20, -24, -27, -30):
        rows.append(OC.bf16_round(rng.standard_normal(D).astype(np.float32) * np.float32(2.0 ** e)))
    # 35..42: huge magnitudes (near the bf16 range top still finite in fp16 scale? scale
    # saturates to fp16 inf above 65504 * 127; keep within)
    for e in (4, 8, 12, 15):
        for sgn in (1, -1):
            x = rng.standard_normal(D).astype(np.float32) * np.float32(2.0 ** e)
            x[rng.integers(D)] = sgn * np.float32(2.0 ** (e + 2))
            rows.append(OC.bf16_round(x))
    # 43..50: constant vectors (every code +-127)
    for c in (1.0, -1.0, 0.5, 3.75, -1e-3, 100.0, -65504.0, 2.0 ** -20):
        rows.append(OC.bf16_round(np.full(D, c, np.float32)))
    # 51..59: uniform, integer-valued, alternating
    for i in range(9):
        if i < 4:
            x = rng.uniform(-1, 1, D).astype(np.float32)
        elif i < 7:
            x = rng.integers(-127, 128, D).astype(np.float32)
        else:
            x = np.where(np.arange(D) % 2 == 0, 1.0, -1.0).astype(np.float32) * np.float32(i)
            x[0] = np.float32(i * 2.5)
        rows.append(OC.bf16_round(x))
    # 60..63: amax in {1.1171875, 1.125, 1.3671875, 1.625} and x = amax / 2: amax * fl(1/127)
    # is one ulp below amax / 127, so x / scale is just above 63.5 on the device path (code 64)
    # and just below it with true division (code 63) -- the two modes disagree here.
    for a in (1.1171875, 1.125, 1.3671875, 1.625):
        x = np.where(np.arange(D) % 3 == 0, a / 2, -a / 2).astype(np.float32)
        x[7] = np.float32(a)
        x[9::5] = rng.uniform(-a, a, x[9::5].shape).astype(np.float32)
        rows.append(OC.bf16_round(x))
    X = np.stack(rows).astype(np.float32)
    assert X.shape == (64, D)
    return X


def make_codec(rng):
    X = codec_vectors(rng)
    q8d, s8d = OC.quantize(X, 8, "device")
    q8c, s8c = OC.quantize(X, 8, "cpu")
    q4d, s4d = OC.quantize(X, 4, "device")
    np.savez_compressed(os.path.join(HERE, "codec_int8.npz"),
                        x_bf16=bf16_bits(X),
                        q8_device=q8d, s8_device=s8d.view(np.uint16),
                        q8_cpu=q8c, s8_cpu=s8c.view(np.uint16),
                        q4_device=q4d, s4_device=s4d.view(np.uint16))


# ----------------------------------------------------------------------------- accept
def accept_group(rng, B, g, V, temperature, kind):
    """kind: 'logits' (draft logits), 'probs' (draft probabilities given), 'greedy'."""
    tl = (rng.standard_normal((B, g + 1, V)) * 2).astype(np.float32)
    if kind == "greedy":
        # drafts agree with the target argmax for a random prefix, then differ
        arg = tl.argmax(-1)
        dt = arg[:, :g].copy()
        cut = rng.integers(0, g + 1, B)
        for b in range(B):
            if cut[b] < g:
                dt[b, cut[b]] = (dt[b, cut[b]] + 1 + rng.integers(V - 1)) % V
        dl = (tl[:, :g] + rng.standard_normal((B, g, V)).astype(np.float32)).astype(np.float32)
        ua = rng.random((B, g)).astype(np.float32)
        ur = rng.random(B).astype(np.float32)
        return tl, dl, dt.astype(np.int32), ua, ur
    inv_t = OA.inv_temperature(temperature)
    dl = (tl[:, :g] + rng.standard_normal((B, g, V)).astype(np.float32) * 0.5).astype(np.float32)
    # special rows: p = q (b=0), q[d] = 0 (b=1: draft logit of the chosen token far below)
    dl[0] = tl[0, :g]
    if kind == "probs":
        q = OA.softmax32(dl, inv_t)
        # b=2: q >= p everywhere, so max(0, p - q) sums to 0 at the first rejection
        q[2] = np.maximum(OA.softmax32(tl[2, :g], inv_t) * np.float32(1.25), q[2])
        draft = q.astype(np.float32)
    else:
        draft = dl
        q = OA.softmax32(dl, inv_t)
    us = rng.random((B, g)).astype(np.float32)
    dt = np.zeros((B, g), np.int32)
    for b in range(B):
        for i in range(g):
            dt[b, i] = OA.inverse_cdf(q[b, i], us[b, i])[0]
    if kind == "logits":
        dl[1, :, :] = tl[1, :g]
        for i in range(g):
            dl[1, i, dt[1, i]] = np.float32(-400.0)      # q[d] underflows to 0 -> ratio 1
    ua = rng.random((B, g)).astype(np.float32)
    ur = rng.random(B).astype(np.float32)
    # b=3: every uniform exactly on its ratio (u >= ratio rejects: the reference's `>=`)
    p = OA.softmax32(tl, inv_t)
    qq = OA.softmax32(dl, inv_t) if kind == "logits" else draft
    for i in range(g):
        d = dt[3, i]
        ua[3, i] = np.minimum(p[3, i, d] / np.maximum(qq[3, i, d], np.float32(1e-20)),
                              np.float32(1.0)).astype(np.float32)
    # b=4: first uniform forced to 0.9999999 so the first draft is (almost surely) rejected
    ua[4, 0] = np.float32(0.9999999)
    return tl, draft, dt, ua, ur


def make_accept_v16(rng):
    V, g = 16, 4
    out = {}
    for name, B, T, kind in (("t1", 32, 1.0, "logits"), ("t05", 16, 0.5, "logits"),
                             ("probs", 16, 1.0, "probs"), ("greedy", 16, 0.0, "greedy")):
        tl, dr, dt, ua, ur = accept_group(rng, B, g, V, T, kind)
        acc, toks, marg = OA.accept_batch(tl, dr, dt, T, ua, ur, draft_is_probs=(kind == "probs"))
        out.update({f"{name}_target": tl, f"{name}_draft": dr, f"{name}_draft_tokens": dt,
                    f"{name}_u_accept": ua, f"{name}_u_resample": ur,
                    f"{name}_temperature": np.float32(T),
                    f"{name}_accepted_len": acc, f"{name}_tokens": toks,
                    f"{name}_margin": marg})
    np.savez_compressed(os.path.join(HERE, "accept_v16.npz"), **out)


def formula_logits(params, V):
    """Row r = ((j * a_r + c_r) mod m_r) / 128 - off_r, exact in fp32 (small integers / 2^7)."""
    j = np.arange(V, dtype=np.int64)
    rows = [(((j * a + c) % m).astype(np.float64) / 128.0 - off).astype(np.float32)
            for a, c, m, off in params]
    return np.stack(rows)


def fullv_params(B, g, seed):
    rng = np.random.default_rng(seed)
    tp = [(int(rng.integers(1, 1 << 20)) * 2 + 1, int(rng.integers(0, 1 << 20)),
           int(rng.integers(600, 1100)), 4.0) for _ in range(B * (g + 1))]
    # draft rows: the matching target row's parameters with a perturbed multiplier
    dp = []
    for b in range(B):
        for i in range(g):
            a, c, m, off = tp[b * (g + 1) + i]
            dp.append((a + 2 * int(rng.integers(0, 3)), c, m, off))
    return np.array(tp, np.float64), np.array(dp, np.float64)


def make_accept_fullv():
    B, g, V, T = 2, 4, VOCAB, 1.0
    tp, dp = fullv_params(B, g, 7)
    tl = formula_logits([tuple(r) for r in tp], V).reshape(B, g + 1, V)
    dl = formula_logits([tuple(r) for r in dp], V).reshape(B, g, V)
    inv_t = OA.inv_temperature(T)
    q = OA.softmax32(dl, inv_t)
    rng = np.random.default_rng(11)
    us = rng.random((B, g)).astype(np.float32)
    dt = np.array([[OA.inverse_cdf(q[b, i], us[b, i])[0] for i in range(g)] for b in range(B)],
                  np.int32)
    ua = rng.random((B, g)).astype(np.float32)
    ur = rng.random(B).astype(np.float32)
    acc, toks, marg = OA.accept_batch(tl, dl, dt, T, ua, ur)
    gacc, gtoks, _ = OA.accept_batch(tl, dl, tl[:, :g].argmax(-1).astype(np.int32), 0.0)
    np.savez_compressed(os.path.join(HERE, "accept_fullv.npz"),
                        target_params=tp, draft_params=dp, B=B, gamma=g, V=V,
                        temperature=np.float32(T), draft_tokens=dt, u_accept=ua, u_resample=ur,
                        accepted_len=acc, tokens=toks, margin=marg,
                        greedy_accepted_len=gacc, greedy_tokens=gtoks)


# ----------------------------------------------------------------------------- attention
def make_attention(rng):
    Hq, Hkv, D, bs = 32, 8, 128, 16
    seq_lens = np.array([37, 200, 5], np.int32)
    q_lens = np.array([1, 3, 5], np.int32)
    W = -(-seq_lens // bs)
    nblk = int(W.sum()) + 2                      # two blocks no sequence owns
    perm = rng.permutation(nblk)
    tables = np.zeros((3, int(W.max())), np.int32)
    o = 0
    for b in range(3):
        tables[b, :W[b]] = perm[o:o + W[b]]
        o += W[b]
    # codes/scales: N(0,1) with x20 outliers, quantised per (token, head)
    kv = rng.standard_normal((2, nblk, bs, Hkv, D)).astype(np.float32)
    kv[rng.random(kv.shape) < 0.01] *= 20
    codes, scales = OC.quantize(OC.bf16_round(kv), 8, "device")
    q = OC.bf16_round(rng.standard_normal((int(q_lens.sum()), Hq, D)).astype(np.float32))
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    K = OP.dequantized_cache(codes[0], scales[0])
    Vv = OP.dequantized_cache(codes[1], scales[1])
    out = OP.attention(q, K, Vv, cu, seq_lens, tables, bs).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "attention_tiny.npz"),
                        q_bf16=bf16_bits(q), k_codes=codes[0], v_codes=codes[1],
                        k_scale=scales[0].view(np.uint16), v_scale=scales[1].view(np.uint16),
                        block_table=tables, cu_seqlens_q=cu, seq_lens=seq_lens,
                        block_size=bs, out=out)


def main():
    make_codec(np.random.default_rng(1))
    make_accept_v16(np.random.default_rng(2))
    make_accept_fullv()
    make_attention(np.random.default_rng(3))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
