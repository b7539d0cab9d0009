"""Speculative acceptance with explicit uniforms, restating engine/spec_decode.py:12-49.

Reference (spec_decode.py):
  sample  (:12-17)  T <= 0: argmax; else probs = softmax(logits / T), multinomial(probs, 1)
  verify  (:20-49)  greedy (:30-35): accept while argmax(target_i) == d_i, emit argmax_k.
                    sampling: p = softmax(target / T) (:37);
                    ratio_i = min(1, p_i[d_i] / max(q_i[d_i], 1e-20)) (:38-40);
                    u = rand(g) (:41); rejected = u >= ratio (:42);
                    none rejected: bonus ~ p_g (:43-45); else k = first rejection (:46),
                    residual = max(0, p_k - q_k), normalised, or p_k if it sums to 0 (:47-48),
                    token ~ residual (:49).
  batched greedy accept, engine/engine.py:421-443 (same rule, one argmax for the batch).

Explicit randomness: the uniforms of :41 are passed in (u_accept), and the draws of
multinomial (:44, :49) become one inverse-CDF draw with u_resample: the smallest j with
cumsum(w)[j] > u * sum(w), cumulative sums in float64.
Numerics: "logits / T" is evaluated as logits * fp32(1/T) (torch's GPU path for a Python
scalar divisor); softmax is the exactly rounded fp32 value (computed in float64, rounded
once), the value every accurate fp32 implementation approximates within a few ulp;
ratios and residuals are fp32 operations on those fp32 probabilities, as in the reference.

margin = min over the deciding comparisons of |u_i - ratio_i| and, for the inverse CDF,
min(tau - cdf[j-1], cdf[j] - tau) / sum(w); a decision with margin below ~1e-6 may flip
between two correct fp32 implementations and is reported as a tie.

Pinned by tests/test_oracle_accept.py: the greedy known-answer test of
tests/test_units.py:47-52, the losslessness test of tests/test_units.py:55-67 (first-token
distribution within 0.01 of the target's over 40,000 draws), closed-form special cases
(p = q accepts everything; q[d] = 0 accepts; zero residual falls back to p_k), brute-force
enumeration of the output distribution at V <= 8, and verify_torch (the reference lines
executed by torch with the same uniforms).
"""
import numpy as np


def softmax32(logits, inv_t=np.float32(1.0)):
    """Exactly rounded fp32 softmax of fp32(logits * inv_t) over the last axis."""
    x = (np.asarray(logits, dtype=np.float32) * np.float32(inv_t)).astype(np.float32)
    m = x.max(axis=-1, keepdims=True).astype(np.float64)
    e = np.exp(x.astype(np.float64) - m)
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def inv_temperature(temperature: float):
    return np.float32(1.0) / np.float32(temperature)


def inverse_cdf(w, u):
    """Smallest j with cumsum(w)[j] > u * sum(w) (float64 sums); returns (j, margin)."""
    c = np.cumsum(np.asarray(w, dtype=np.float32).astype(np.float64))
    total = c[-1]
    tau = np.float64(np.float32(u)) * total
    j = int(np.searchsorted(c, tau, side="right"))
    if j >= len(c):  # tau within rounding of the total: last element with mass
        nz = np.nonzero(np.asarray(w) > 0)[0]
        return (int(nz[-1]) if len(nz) else len(c) - 1), 0.0
    lo = c[j - 1] if j > 0 else 0.0
    return j, float(min(tau - lo, c[j] - tau) / total) if total > 0 else 0.0


def verify(target_logits, draft_tokens, draft, temperature, u_accept=None, u_resample=None,
           draft_is_probs=False):
    """One sequence.  Returns (tokens, k, margin): tokens = drafts[:k] + [emitted]."""
    d = [int(t) for t in draft_tokens]
    g = len(d)
    tl = np.asarray(target_logits, dtype=np.float32)
    V = tl.shape[-1]
    if not temperature > 0:  # spec_decode.py:30-35 / engine.py:439-443
        tgt = tl.argmax(axis=-1)
        k = 0
        while k < g and tgt[k] == d[k]:
            k += 1
        return d[:k] + [int(tgt[k])], k, float("inf")
    inv_t = inv_temperature(temperature)
    p = softmax32(tl, inv_t)
    if g:
        q = np.asarray(draft, dtype=np.float32) if draft_is_probs else softmax32(draft, inv_t)
    margin, k = float("inf"), g
    for i in range(g):
        ratio = np.float32(0.0)
        if 0 <= d[i] < V:
            ratio = np.minimum(p[i, d[i]] / np.maximum(q[i, d[i]], np.float32(1e-20)),
                               np.float32(1.0)).astype(np.float32)
        ui = np.float32(u_accept[i])
        margin = min(margin, abs(float(ui) - float(ratio)))
        if ui >= ratio:
            k = i
            break
    if k == g:
        w = p[g]
    else:
        r = np.maximum(p[k] - q[k], np.float32(0.0)).astype(np.float32)
        w = r if r.sum(dtype=np.float64) > 0 else p[k]
    tok, m2 = inverse_cdf(w, u_resample)
    return d[:k] + [tok], k, min(margin, m2)


def accept_batch(target, draft, draft_tokens, temperature, u_accept=None, u_resample=None,
                 draft_is_probs=False, gamma_per_seq=None):
    """Batched verify: target [B, gmax+1, V], draft [B, gmax, V] -> (acc_len, tokens, margin)."""
    dt = np.asarray(draft_tokens)
    B, gmax = dt.shape
    acc = np.zeros(B, np.int32)
    toks = np.full((B, gmax + 1), -1, np.int32)
    marg = np.zeros(B, np.float64)
    for b in range(B):
        g = gmax if gamma_per_seq is None else int(gamma_per_seq[b])
        out, k, m = verify(np.asarray(target[b])[:g + 1], dt[b, :g],
                           None if draft is None or g == 0 else np.asarray(draft[b])[:g],
                           temperature,
                           None if u_accept is None else np.asarray(u_accept)[b, :g],
                           None if u_resample is None else np.asarray(u_resample)[b],
                           draft_is_probs)
        acc[b], marg[b] = k, m
        toks[b, :len(out)] = out
    return acc, toks, marg


def sample(logits, temperature, uniforms=None):
    """spec_decode.py:12-17 with inverse-CDF draws: -> (tokens [N], probs [N, V] or None)."""
    x = np.asarray(logits, dtype=np.float32)
    if not temperature > 0:
        return x.argmax(axis=-1), None
    p = softmax32(x, inv_temperature(temperature))
    toks = np.array([inverse_cdf(p[i], uniforms[i])[0] for i in range(x.shape[0])])
    return toks, p


def verify_torch(target_logits, draft_tokens, draft_probs, temperature, u_accept, u_resample):
    """engine/spec_decode.py:37-49 executed by torch on the tensors' device, the uniforms of
    :41 passed in and the multinomial draws of :44/:49 replaced by the inverse CDF."""
    import torch

    g = len(draft_tokens)
    p = torch.softmax(target_logits / temperature, dim=-1)
    if g:
        d = torch.tensor(list(draft_tokens), device=p.device)
        idx = torch.arange(g, device=p.device)
        ratio = (p[idx, d] / draft_probs[idx, d].clamp_min(1e-20)).clamp(max=1.0)
        rejected = (u_accept.to(p.device) >= ratio).nonzero()
    if g == 0 or len(rejected) == 0:
        dist, prefix = p[g], list(draft_tokens)
    else:
        k = rejected[0].item()
        residual = (p[k] - draft_probs[k]).clamp_min(0)
        dist = residual / residual.sum() if residual.sum() > 0 else p[k]
        prefix = list(draft_tokens)[:k]
    c = torch.cumsum(dist.double(), 0)
    tau = float(np.float32(u_resample)) * c[-1]
    tok = int(torch.searchsorted(c, tau.reshape(1), right=True).item())
    tok = min(tok, dist.numel() - 1)
    return prefix + [tok]
