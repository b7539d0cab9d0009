"""CPU: pins oracle.accept (restating engine/spec_decode.py:12-49, engine/engine.py:421-446)."""
import numpy as np
import torch

from oracle import accept as A


def onehot_logits(tokens, vocab=10):
    x = np.full((len(tokens), vocab), -1e4, np.float32)
    x[np.arange(len(tokens)), tokens] = 0
    return x


def test_greedy_verify_accepts_matching_prefix():
    """Known-answer test of tests/test_units.py:47-52."""
    out, k, _ = A.verify(onehot_logits([3, 5, 7, 9]), [3, 5, 1], None, temperature=0)
    assert out == [3, 5, 7] and k == 2
    out, k, _ = A.verify(onehot_logits([3, 5, 7, 9]), [3, 5, 7], None, temperature=0)
    assert out == [3, 5, 7, 9] and k == 3


def test_greedy_argmax_ties_take_first_index():
    x = np.zeros((2, 6), np.float32)
    x[0, [2, 4]] = 1.0
    x[1, [1, 5]] = 2.0
    out, k, _ = A.verify(x, [2], None, temperature=0)
    assert out == [2, 1] and k == 1


def test_rejection_sampling_is_lossless():
    """tests/test_units.py:55-67 with explicit seeded uniforms: the first emitted token follows
    the target distribution whatever the draft proposes (atol 0.01 over 40,000 draws)."""
    rng = np.random.default_rng(0)
    V, N = 5, 40000
    p_logits = np.log(np.array([0.5, 0.2, 0.15, 0.1, 0.05], np.float32))
    q = np.array([0.05, 0.05, 0.1, 0.4, 0.4], np.float32)
    counts = np.zeros(V)
    tl = np.stack([p_logits, p_logits])
    ds = rng.choice(V, size=N, p=q / q.sum())
    ua = rng.random(N, dtype=np.float32)
    ur = rng.random(N, dtype=np.float32)
    for i in range(N):
        out, _, _ = A.verify(tl, [int(ds[i])], q[None], 1.0, [ua[i]], ur[i], draft_is_probs=True)
        counts[out[0]] += 1
    target = A.softmax32(p_logits)
    assert np.allclose(counts / N, target, atol=0.01), counts / N


def test_exact_output_distribution_by_enumeration():
    """Brute force at V=6: integrate the accept branch exactly (P(u < ratio) = ratio) and the
    resample branch over a 4000-point midpoint grid of u_resample; the first-token
    distribution must equal p to grid resolution."""
    rng = np.random.default_rng(1)
    V, M = 6, 4000
    tl = rng.standard_normal((2, V)).astype(np.float32) * 2
    dl = rng.standard_normal((1, V)).astype(np.float32) * 2
    p = A.softmax32(tl)[0].astype(np.float64)
    q = A.softmax32(dl)[0].astype(np.float64)
    grid = ((np.arange(M) + 0.5) / M).astype(np.float32)
    dist = np.zeros(V)
    for d in range(V):
        ratio = min(1.0, p[d] / q[d])
        dist[d] += q[d] * ratio                      # accepted: emits d
        if ratio < 1.0:                              # rejected: emits a residual draw
            rej = np.zeros(V)
            for u in grid:
                out, k, _ = A.verify(tl, [d], dl, 1.0, [np.float32(0.9999999)], u)
                assert k == 0
                rej[out[0]] += 1.0 / M
            dist += q[d] * (1 - ratio) * rej
    assert np.allclose(dist, p, atol=2.0 / M), (dist, p)


def test_identical_draft_accepts_everything_and_draws_bonus_from_last_row():
    rng = np.random.default_rng(2)
    tl = rng.standard_normal((4, 50)).astype(np.float32)
    out, k, _ = A.verify(tl, [1, 2, 3], tl[:3], 1.0, [0.999, 0.999, 0.999], 0.5)
    assert k == 3 and out[:3] == [1, 2, 3]
    assert out[3] == A.inverse_cdf(A.softmax32(tl[3]), 0.5)[0]


def test_zero_draft_probability_is_accepted():
    tl = np.zeros((2, 8), np.float32)
    q = np.full((1, 8), 1 / 7, np.float32)
    q[0, 3] = 0.0
    out, k, _ = A.verify(tl, [3], q, 1.0, [0.999], 0.1, draft_is_probs=True)
    assert k == 1 and out[0] == 3


def test_zero_residual_falls_back_to_target_row():
    """engine/spec_decode.py:48: residual.sum() == 0 -> sample from p_k (q = 2p here)."""
    rng = np.random.default_rng(3)
    tl = rng.standard_normal((2, 16)).astype(np.float32)
    p = A.softmax32(tl)
    q = (2 * p[:1]).astype(np.float32)
    for u in (0.05, 0.5, 0.95):
        out, k, _ = A.verify(tl, [4], q, 1.0, [0.75], u, draft_is_probs=True)
        assert k == 0 and out[0] == A.inverse_cdf(p[0], u)[0]


def test_out_of_vocab_draft_is_rejected():
    tl = np.zeros((3, 8), np.float32)
    out, k, _ = A.verify(tl, [1, 99], tl[:2], 1.0, [0.5, 0.0], 0.3)
    assert k == 1 and out[0] == 1


def test_inverse_cdf_skips_zero_weights_and_reports_margin():
    w = np.array([0, 0.25, 0, 0.25, 0.5, 0], np.float32)
    assert A.inverse_cdf(w, 0.0)[0] == 1
    assert A.inverse_cdf(w, 0.25)[0] == 3       # boundary: cdf[1] = 0.25 is not > 0.25
    j, m = A.inverse_cdf(w, 0.3)
    assert j == 3 and abs(m - 0.05) < 1e-7
    assert A.inverse_cdf(w, np.float32(0.99999994))[0] == 4


def test_batched_accept_equals_per_sequence_verify_with_ragged_gamma():
    rng = np.random.default_rng(4)
    B, g, V = 6, 4, 40
    tl = rng.standard_normal((B, g + 1, V)).astype(np.float32)
    dl = tl[:, :g] + 0.5 * rng.standard_normal((B, g, V)).astype(np.float32)
    dt = rng.integers(0, V, (B, g))
    ua, ur = rng.random((B, g), dtype=np.float32), rng.random(B, dtype=np.float32)
    gam = np.array([4, 0, 2, 4, 1, 3])
    acc, toks, _ = A.accept_batch(tl, dl, dt, 1.0, ua, ur, gamma_per_seq=gam)
    for b in range(B):
        out, k, _ = A.verify(tl[b, :gam[b] + 1], dt[b, :gam[b]], dl[b, :gam[b]], 1.0,
                             ua[b, :gam[b]], ur[b])
        assert acc[b] == k and toks[b, :k + 1].tolist() == out and (toks[b, k + 1:] == -1).all()


def test_softmax32_is_exactly_rounded():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((3, 1000)) * 4).astype(np.float32)
    ref = torch.softmax(torch.from_numpy(x).double(), -1).float().numpy()
    assert np.array_equal(A.softmax32(x), ref)


def test_reference_lines_run_by_torch_agree_up_to_ties():
    """verify_torch executes engine/spec_decode.py:37-49 with torch (CPU here).  Its fp32
    softmax differs from the exactly rounded one by a few ulp, so decisions may only differ
    where the oracle reports a tie (margin < 1e-6)."""
    rng = np.random.default_rng(6)
    V, g, n, ties, diffs = 3000, 4, 300, 0, 0
    for _ in range(n):
        tl = (rng.standard_normal((g + 1, V)) * 2).astype(np.float32)
        dl = tl[:g] + (rng.standard_normal((g, V)) * 0.5).astype(np.float32)
        q = A.softmax32(dl)
        d = [int(rng.choice(V, p=q[i].astype(np.float64) / q[i].sum(dtype=np.float64)))
             for i in range(g)]
        ua, ur = rng.random(g, dtype=np.float32), np.float32(rng.random())
        out, k, m = A.verify(tl, d, q, 1.0, ua, ur, draft_is_probs=True)
        ref = A.verify_torch(torch.from_numpy(tl), d, torch.from_numpy(q), 1.0,
                             torch.from_numpy(ua), ur)
        ties += m < 1e-6
        if out != ref:
            diffs += 1
            assert m < 1e-6, (out, ref, m)
    assert diffs <= ties
