"""GPU parity: fused accept-sample kernel vs oracle.accept and vs the reference's verify lines
executed by torch on the same GPU (engine/spec_decode.py:37-49, explicit uniforms).

Bar: accepted lengths and emitted tokens bit-exact given the uniforms; a disagreement is
allowed only where the oracle reports the deciding uniform within 1e-6 of its boundary
(a tie), and every tie is printed.
"""
import numpy as np
import pytest
import torch

import iitj_llm_coopt_amd as M
from oracle import accept as OA

pytestmark = pytest.mark.gpu
TIE = 1e-6


def report(msg):
    print(msg, flush=True)


def config1_inputs(seed, B=8, g=4, V=128256, dev="cuda"):
    """Config 1: target N(0, 2^2) [B, g+1, V]; draft = target[:, :g] + N(0, 0.5^2); drafts
    sampled from the draft softmax at T=1 (oracle inverse CDF with seeded uniforms)."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    tl = torch.randn(B, g + 1, V, generator=gen, device=dev) * 2.0
    dl = tl[:, :g] + torch.randn(B, g, V, generator=gen, device=dev) * 0.5
    rng = np.random.default_rng(seed)
    q = OA.softmax32(dl.cpu().numpy())
    ud = rng.random((B, g), dtype=np.float32)
    dt = np.array([[OA.inverse_cdf(q[b, i], ud[b, i])[0] for i in range(g)] for b in range(B)])
    ua = rng.random((B, g), dtype=np.float32)
    ur = rng.random(B, dtype=np.float32)
    return tl, dl.contiguous(), dt, ua, ur


def compare(res, acc, toks, marg, label):
    got_acc = res.accepted_len.cpu().numpy()
    got_tok = res.tokens.cpu().numpy()
    mism, ties = 0, int((marg < TIE).sum())
    for b in range(len(acc)):
        if got_acc[b] != acc[b] or not np.array_equal(got_tok[b], toks[b]):
            mism += 1
            report(f"[{label}] seq {b}: kernel {got_tok[b].tolist()} oracle {toks[b].tolist()} "
                   f"margin {marg[b]:.3g}")
            assert marg[b] < TIE, f"{label}: mismatch on seq {b} outside the tie band"
    report(f"[{label}] B={len(acc)} mismatches={mism} ties(margin<1e-6)={ties} "
           f"accepted={got_acc.tolist()[:16]}")
    return mism


def test_greedy_known_answer_fp32_and_bf16(dev):
    """tests/test_units.py:47-52 through the kernel."""
    def onehot(tokens, V=10):
        x = torch.full((len(tokens), V), -1e4)
        x[torch.arange(len(tokens)), torch.tensor(tokens)] = 0
        return x
    tl = torch.stack([onehot([3, 5, 7, 9]), onehot([3, 5, 7, 9])]).to(dev)
    dt = torch.tensor([[3, 5, 1], [3, 5, 7]], device=dev)
    for dtype in (torch.float32, torch.bfloat16):
        res = M.accept(tl.to(dtype), None, dt, 0.0)
        assert res.to_lists() == [[3, 5, 7], [3, 5, 7, 9]]
        assert res.accepted_len.tolist() == [2, 3]
    assert M.verify(onehot([3, 5, 7, 9]).to(dev), [3, 5, 1], None, 0.0) == [3, 5, 7]


def test_greedy_batch_matches_argmax_prefix_rule(dev):
    """engine/engine.py:421-443 on bf16 logits (the graph path's logits dtype)."""
    gen = torch.Generator(device=dev).manual_seed(5)
    B, g, V = 32, 4, 128256
    tl = torch.randn(B, g + 1, V, generator=gen, device=dev).to(torch.bfloat16)
    am = tl.float().argmax(-1)
    dt = am[:, :g].clone()
    flip = torch.rand(B, g, generator=gen, device=dev) < 0.3
    dt = torch.where(flip, (dt + 1) % V, dt)
    res = M.accept(tl, None, dt, 0.0)
    acc, toks, _ = OA.accept_batch(tl.float().cpu().numpy(), None, dt.cpu().numpy(), 0.0)
    assert np.array_equal(res.accepted_len.cpu().numpy(), acc)
    assert np.array_equal(res.tokens.cpu().numpy(), toks)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config1_sampling_matches_oracle_up_to_ties(dev, seed):
    tl, dl, dt, ua, ur = config1_inputs(seed, dev=dev)
    res = M.accept(tl, dl, torch.from_numpy(dt).to(dev), 1.0, torch.from_numpy(ua).to(dev),
                   torch.from_numpy(ur).to(dev))
    acc, toks, marg = OA.accept_batch(tl.cpu().numpy(), dl.cpu().numpy(), dt, 1.0, ua, ur)
    compare(res, acc, toks, marg, f"config1 seed {seed}")


def test_b32_sampling_matches_oracle_up_to_ties(dev):
    tl, dl, dt, ua, ur = config1_inputs(11, B=32, dev=dev)
    res = M.accept(tl, dl, torch.from_numpy(dt).to(dev), 1.0, torch.from_numpy(ua).to(dev),
                   torch.from_numpy(ur).to(dev))
    acc, toks, marg = OA.accept_batch(tl.cpu().numpy(), dl.cpu().numpy(), dt, 1.0, ua, ur)
    assert compare(res, acc, toks, marg, "B=32") <= 1


def test_config1_matches_reference_lines_run_by_torch_on_gpu(dev):
    """The reference's verify (engine/spec_decode.py:37-49) executed by torch-ROCm with the
    same uniforms, draft_probs = torch.softmax(draft) as the engine keeps them (:404)."""
    tl, dl, dt, ua, ur = config1_inputs(3, dev=dev)
    probs = torch.softmax(dl, dim=-1)
    res = M.accept(tl, probs, torch.from_numpy(dt).to(dev), 1.0, torch.from_numpy(ua).to(dev),
                   torch.from_numpy(ur).to(dev), draft_is_probs=True)
    got = res.to_lists()
    _, _, marg = OA.accept_batch(tl.cpu().numpy(), probs.cpu().numpy(), dt, 1.0, ua, ur,
                                 draft_is_probs=True)
    for b in range(tl.shape[0]):
        ref = OA.verify_torch(tl[b], dt[b].tolist(), probs[b], 1.0, torch.from_numpy(ua[b]), ur[b])
        if got[b] != ref:
            report(f"[torch-ref] seq {b}: kernel {got[b]} torch {ref} margin {marg[b]:.3g}")
            assert marg[b] < TIE


def test_draft_probability_mode_and_ragged_gamma_and_row_offsets(dev):
    gen = torch.Generator(device=dev).manual_seed(6)
    B, g, V = 6, 4, 5000
    tl = torch.randn(B, g + 1, V, generator=gen, device=dev) * 2
    dl = tl[:, :g] + torch.randn(B, g, V, generator=gen, device=dev) * 0.5
    q = torch.softmax(dl, -1)
    dt = torch.randint(0, V, (B, g), generator=gen, device=dev)
    dt[:, 0] = tl[:, 0].argmax(-1)  # likely accepts
    ua = torch.rand(B, g, generator=gen, device=dev)
    ur = torch.rand(B, generator=gen, device=dev)
    gam = torch.tensor([4, 0, 2, 4, 1, 3], device=dev)
    # pack rows varlen, as build_batch lays out logits rows (spans), with junk rows between
    rows_t, rows_d, t0, d0 = [], [], [], []
    for b in range(B):
        t0.append(sum(r.shape[0] for r in rows_t))
        rows_t += [tl[b, :gam[b] + 1], torch.full((1, V), 7.0, device=dev)]
        d0.append(sum(r.shape[0] for r in rows_d))
        rows_d += [q[b, :gam[b]]]
    T = torch.cat(rows_t)
    Dp = torch.cat(rows_d + [torch.zeros(1, V, device=dev)])
    res = M.accept(T, Dp, dt, 1.0, ua, ur, draft_is_probs=True, gamma_per_seq=gam,
                   target_row0=torch.tensor(t0), draft_row0=torch.tensor(d0))
    acc, toks, marg = OA.accept_batch(tl.cpu().numpy(), q.cpu().numpy(), dt.cpu().numpy(), 1.0,
                                      ua.cpu().numpy(), ur.cpu().numpy(), draft_is_probs=True,
                                      gamma_per_seq=gam.cpu().numpy())
    compare(res, acc, toks, marg, "ragged")


@pytest.mark.parametrize("B,g,V,gam", [
    (2, 4, 128256, None),          # many chunks per row: the block-wide row combine
    (3, 64, 2000, [64, 0, 37]),    # gamma_max 64: the bonus row is row 64
    (5, 63, 2000, [63, 63, 10, 1, 0]),  # the widest gamma a single wave decides
])
def test_small_batch_and_long_gamma_match_oracle(dev, B, g, V, gam):
    gen = torch.Generator(device=dev).manual_seed(100 + g)
    tl = torch.randn(B, g + 1, V, generator=gen, device=dev) * 2.0
    # a draft close to the target, so long prefixes are accepted
    dl = (tl[:, :g] + torch.randn(B, g, V, generator=gen, device=dev) * 0.05).contiguous()
    rng = np.random.default_rng(g)
    q = OA.softmax32(dl.cpu().numpy())
    ud = rng.random((B, g), dtype=np.float32)
    dt = np.array([[OA.inverse_cdf(q[b, i], ud[b, i])[0] for i in range(g)] for b in range(B)])
    dt = dt.reshape(B, g).astype(np.int64)
    ua = rng.random((B, g), dtype=np.float32) * 0.9
    ur = rng.random(B, dtype=np.float32)
    kw = {}
    if gam is not None:
        kw["gamma_per_seq"] = torch.tensor(gam, device=dev)
    res = M.accept(tl, dl, torch.from_numpy(dt).to(dev), 1.0, torch.from_numpy(ua).to(dev),
                   torch.from_numpy(ur).to(dev), **kw)
    acc, toks, marg = OA.accept_batch(tl.cpu().numpy(), dl.cpu().numpy(), dt, 1.0, ua, ur,
                                      gamma_per_seq=None if gam is None else np.array(gam))
    compare(res, acc, toks, marg, f"B={B} gamma={g} V={V}")


def test_special_cases(dev):
    gen = torch.Generator(device=dev).manual_seed(7)
    V = 3000
    tl = torch.randn(3, V, generator=gen, device=dev)
    # identical draft: everything accepted, bonus from the last row
    res = M.accept(tl.view(1, 3, V), tl[:2].reshape(1, 2, V).contiguous(),
                   torch.tensor([[5, 9]], device=dev), 1.0,
                   torch.full((1, 2), 0.999, device=dev), torch.tensor([0.5], device=dev))
    assert res.accepted_len.item() == 2
    assert res.tokens[0, 2].item() == OA.inverse_cdf(OA.softmax32(tl[2].cpu().numpy()), 0.5)[0]
    # zero residual (q = 2p as "probabilities"): falls back to p_k
    p = torch.softmax(tl[:1].double(), -1).float()
    res = M.accept(tl[:2].reshape(1, 2, V).contiguous(), (2 * p).view(1, 1, V),
                   torch.tensor([[4]], device=dev), 1.0, torch.tensor([[0.75]], device=dev),
                   torch.tensor([0.3], device=dev), draft_is_probs=True)
    assert res.accepted_len.item() == 0
    assert res.tokens[0, 0].item() == OA.inverse_cdf(OA.softmax32(tl[0].cpu().numpy()), 0.3)[0]
    # out-of-vocabulary draft token is rejected at its position
    res = M.accept(tl.view(1, 3, V), tl[:2].reshape(1, 2, V).contiguous(),
                   torch.tensor([[int(tl[0].argmax()), V + 5]], device=dev), 1.0,
                   torch.tensor([[0.0, 0.0]], device=dev), torch.tensor([0.2], device=dev))
    assert res.accepted_len.item() == 1


def test_rejection_sampling_is_lossless_through_the_kernel(dev):
    """tests/test_units.py:55-67 as one batched launch: 40,000 sequences, V=5, one draft
    each drawn from a deliberately bad q; the first emitted token must follow p (atol 0.01)."""
    N, V = 40000, 5
    gen = torch.Generator(device=dev).manual_seed(8)
    p_logits = torch.log(torch.tensor([0.5, 0.2, 0.15, 0.1, 0.05], device=dev))
    q = torch.tensor([0.05, 0.05, 0.1, 0.4, 0.4], device=dev)
    d = torch.multinomial(q.expand(N, V), 1, generator=gen)
    tl = p_logits.expand(N, 2, V).contiguous()
    res = M.accept(tl, q.expand(N, 1, V).contiguous(), d, 1.0,
                   torch.rand(N, 1, generator=gen, device=dev),
                   torch.rand(N, generator=gen, device=dev), draft_is_probs=True)
    emp = torch.bincount(res.tokens[:, 0].long(), minlength=V).float() / N
    assert torch.allclose(emp, torch.softmax(p_logits, -1), atol=0.01), emp


def test_sample_and_softmax(dev):
    gen = torch.Generator(device=dev).manual_seed(9)
    N, V = 16, 128256
    x = torch.randn(N, V, generator=gen, device=dev) * 2
    tok, probs = M.sample(x, 0.0)
    assert probs is None and torch.equal(tok, x.argmax(-1))
    u = torch.rand(N, generator=gen, device=dev)
    tok, probs = M.sample(x, 0.7, uniforms=u)
    ref_tok, ref_p = OA.sample(x.cpu().numpy(), 0.7, u.cpu().numpy())
    # bit-exact tokens, except rows whose inverse-CDF boundary lies within 1e-6 (a tie by
    # either side's margin), which are reported
    res = M.accept(x, None, torch.empty((N, 0), dtype=torch.int32, device=dev), 0.7,
                   u_resample=u)
    assert torch.equal(res.tokens[:, 0].long(), tok)
    _, _, ref_m = OA.accept_batch(x.cpu().numpy()[:, None], None, np.zeros((N, 0), np.int32),
                                  0.7, None, u.cpu().numpy())
    got_m = res.margin.cpu().numpy()
    t = tok.cpu().numpy()
    for i in range(N):
        if t[i] != ref_tok[i]:
            report(f"[sample] row {i}: kernel {t[i]} oracle {ref_tok[i]} margins "
                   f"{got_m[i]:.3g} / {ref_m[i]:.3g}")
            assert min(got_m[i], ref_m[i]) < TIE, f"row {i} differs outside a tie"
    assert torch.allclose(probs.cpu(), torch.from_numpy(ref_p), rtol=1e-5, atol=1e-12)
    tok_g, _ = M.sample(x, 1.0, generator=torch.Generator(device=dev).manual_seed(1))
    assert tok_g.shape == (N,) and int(tok_g.min()) >= 0 and int(tok_g.max()) < V


@pytest.mark.parametrize("dtype,V,pad", [(torch.float32, 128256, 4), (torch.float32, 999, 0),
                                         (torch.bfloat16, 1001, 2), (torch.bfloat16, 128256, 8),
                                         (torch.float32, 7, 1)])
def test_softmax_layouts(dev, dtype, V, pad):
    """softmax(logits / T) for vector-aligned rows, rows whose length leaves a tail, and row
    strides that rule the vector loads out: within 1e-6 relative of the fp64 softmax."""
    gen = torch.Generator(device=dev).manual_seed(V + pad)
    base = (torch.randn(5, V + pad, generator=gen, device=dev) * 3).to(dtype)
    x = base[:, :V]
    probs = M.softmax(x, 0.8)
    ref = torch.softmax(x.double().cpu() / torch.tensor(0.8, dtype=torch.float32).double(), -1)
    assert torch.allclose(probs.double().cpu(), ref, rtol=1e-5, atol=1e-12)
    assert torch.allclose(probs.double().sum(-1).cpu(), torch.ones(5, dtype=torch.float64), atol=1e-5)
    # sample()'s probabilities (coopt_sample: written by the launch that draws)
    u = torch.rand(5, generator=gen, device=dev)
    tok, sprobs = M.sample(x, 0.8, uniforms=u)
    assert torch.allclose(sprobs.double().cpu(), ref, rtol=1e-5, atol=1e-12)
    assert torch.equal(tok, M.sample(x, 0.8, uniforms=u, return_probs=False)[0])


@pytest.mark.parametrize("N,V", [(1, 128256), (3, 128256), (2, 300000), (40, 50000)])
def test_sample_rows_of_many_chunks(dev, N, V):
    """sample() draws (coopt_sample) where one row spans more chunks than a wave has lanes
    (1 row of 128256: 125 chunks; 2 of 300000: 293), and a batch of many rows: tokens against
    the oracle's inverse CDF over the exactly rounded softmax (a differing row must be a tie
    on the oracle's side), probabilities within 1e-5 relative, and tokens equal to a
    gamma_max = 0 accept call's."""
    gen = torch.Generator(device=dev).manual_seed(N * 7 + V)
    x = torch.randn(N, V, generator=gen, device=dev) * 2.5
    u = torch.rand(N, generator=gen, device=dev)
    tok, probs = M.sample(x, 1.0, uniforms=u)
    ref_tok, ref_p = OA.sample(x.cpu().numpy(), 1.0, u.cpu().numpy())
    _, _, ref_m = OA.accept_batch(x.cpu().numpy()[:, None], None, np.zeros((N, 0), np.int32),
                                  1.0, None, u.cpu().numpy())
    t = tok.cpu().numpy()
    for i in range(N):
        if t[i] != ref_tok[i]:
            report(f"[sample N={N} V={V}] row {i}: kernel {t[i]} oracle {ref_tok[i]} "
                   f"oracle margin {ref_m[i]:.3g}")
            assert ref_m[i] < TIE, f"row {i} differs outside a tie"
    assert torch.allclose(probs.cpu(), torch.from_numpy(ref_p), rtol=1e-5, atol=1e-12)
    res = M.accept(x, None, torch.empty((N, 0), dtype=torch.int32, device=dev), 1.0,
                   u_resample=u)
    assert torch.equal(res.tokens[:, 0].long(), tok)
    assert int((res.accepted_len != 0).sum()) == 0
    report(f"[sample N={N} V={V}] {int((t == ref_tok).sum())}/{N} rows equal to the oracle")


@pytest.mark.parametrize("dtype,N,V", [(torch.float32, 12, 128256), (torch.bfloat16, 5, 50001)])
def test_sample_probs_reads_the_statistics_of_a_gamma0_accept(dev, dtype, N, V):
    """coopt_sample_probs: sample()'s probabilities (engine/spec_decode.py:16) for rows a
    gamma_max = 0 accept call just drew from, built from the row statistics that call left in
    its workspace.  Within 1e-5 relative of the fp64 softmax and of coopt_sample's own
    probabilities; a short workspace and T <= 0 are refused."""
    from iitj_llm_coopt_amd import _lib
    lib = _lib.load()
    gen = torch.Generator(device=dev).manual_seed(N + V)
    x = (torch.randn(N, V, generator=gen, device=dev) * 2.5).to(dtype)
    u = torch.rand(N, generator=gen, device=dev)
    T = 0.9
    need = int(lib.coopt_accept_sample_workspace(N, 0, V))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    M.accept(x, None, torch.empty((N, 0), dtype=torch.int32, device=dev), T, u_resample=u,
             workspace=ws)
    probs = torch.full((N, V), -1.0, dtype=torch.float32, device=dev)
    stream = _lib.stream_handle(dev)
    _lib.check(lib.coopt_sample_probs(_lib.dt_code(dtype), _lib.ptr(x), x.stride(0), N, V, T,
                                      _lib.ptr(ws), need, _lib.ptr(probs), V, stream),
               "coopt_sample_probs")
    ref = torch.softmax(x.double().cpu() / torch.tensor(T, dtype=torch.float32).double(), -1)
    assert torch.allclose(probs.double().cpu(), ref, rtol=1e-5, atol=1e-12)
    _, sprobs = M.sample(x, T, uniforms=u)
    assert torch.allclose(probs, sprobs, rtol=1e-5, atol=1e-12)
    rc = lib.coopt_sample_probs(_lib.dt_code(dtype), _lib.ptr(x), x.stride(0), N, V, T,
                                _lib.ptr(ws), need - 1, _lib.ptr(probs), V, stream)
    assert rc == _lib.COOPT_EWORKSPACE
    rc = lib.coopt_sample_probs(_lib.dt_code(dtype), _lib.ptr(x), x.stride(0), N, V, 0.0,
                                _lib.ptr(ws), need, _lib.ptr(probs), V, stream)
    assert rc == _lib.COOPT_EINVAL
    report(f"[sample_probs {dtype} N={N} V={V}] max |probs - fp64| "
           f"{(probs.double().cpu() - ref).abs().max().item():.3g}")


def test_verify_signature_with_generator(dev):
    gen = torch.Generator(device=dev).manual_seed(10)
    V = 1000
    tl = torch.randn(3, V, generator=gen, device=dev)
    q = torch.softmax(torch.randn(2, V, generator=gen, device=dev), -1)
    out = M.verify(tl, [1, 2], q, 1.0, generator=gen)
    assert 1 <= len(out) <= 3 and all(0 <= t < V for t in out)
