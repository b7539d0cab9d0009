"""Checks SpecDecoder steps against oracle.spec_step.  TEST INFRASTRUCTURE ONLY (tests/ and
bench.py's cpu_baseline leg); the product never imports it.

Per step, from the state the GPU step starts from (caches, token histories, lengths and the
step's row of the uniform table, copied to the host):
  decisions   the oracle step, teacher-forced on the GPU step's logits, must take the same
              decisions: which sequences speculate, every draft token, every accepted length
              and emitted token -- bit-exact, except a decision within TIE of its boundary,
              which is reported and ends the comparison of that sequence;
  state       the GPU's token histories, num_computed and draft_computed after the step equal
              the oracle's (engine/engine.py:463-470), and so do the step's counters;
  logits      the oracle's own logits (its bf16 torch-CPU forward) against the GPU's: the
              largest difference, relative to the largest logit, within `logit_tol`;
  KV cache    the GPU step changed no cache entry outside the slots the oracle wrote, and
              the written entries are within `kv_tol` of the oracle's (bf16: relative to
              max(1, |value|); INT8: dequantised values relative to the vector's range,
              127 * scale).
A tolerance of None reports the largest difference without asserting on it (a deep model's
bf16 rounding differences grow with depth; decisions are compared either way).
The forward is not bit-reproducible across GEMM implementations (MFMA partial sums against a
CPU GEMM), so logits and caches are compared with a tolerance and the decisions are compared
bit-exactly from the same logits.
"""
from collections import Counter

import numpy as np
import torch

from . import spec_step as OS

TIE = 1e-6


def _weights(model):
    """Row-major CPU copies of a RandomLlama's weights."""
    c = model.to("cpu")
    return {"embed": c.embed, "lm_head": c.lm_head, "norm": c.norm,
            "layers": [dict(L) for L in c.layers]}


def _shape(s):
    return OS.Shape(s.hidden, s.heads, s.kv_heads, s.head_dim, s.vocab, s.eps, s.rope_theta)


def _cache_copy(kv):
    return [tuple(None if t is None else t.detach().cpu().contiguous() for t in L) for L in kv.layers]


class StepChecker:
    def __init__(self, dec, logit_tol=5e-2, kv_tol=3e-2, tie=TIE):
        self.dec = dec
        self.target = OS.OracleLlama(_shape(dec.t.s), _weights(dec.t), dec.max_len)
        self.draft = OS.OracleLlama(_shape(dec.d.s), _weights(dec.d), dec.max_len)
        self.logit_tol, self.kv_tol, self.tie = logit_tol, kv_tol, tie
        self.diverged = set()          # sequence ids no longer compared (a tie flipped)
        self.stats = Counter()
        self.worst = Counter()         # largest logit / KV errors seen
        self.log = []

    # ---- before the GPU step ----
    def before(self):
        dec = self.dec
        n, dc = dec.n.cpu().tolist(), dec.dc.cpu().tolist()
        hist = dec.hist.cpu()
        self.seqs = [OS.Seq(hist[b, :n[b]].tolist(), n[b] - 1, dc[b], dec.gamma[b])
                     for b in range(dec.B)]
        self.ids = list(dec.seq_ids)
        self.pre = (_cache_copy(dec.tkv), _cache_copy(dec.dkv))
        self.counters = (int(dec.emitted), int(dec.drafted), int(dec.accepted))
        row = int(dec.u_ctr) % dec.u_table.shape[0]
        u = dec.u_table[row].cpu().numpy()
        gm, Bc = dec.gmax, dec.Bcap
        self.u_draft = u[: gm * Bc].reshape(gm, Bc) if gm else np.zeros((0, Bc), np.float32)
        self.u_acc = u[gm * Bc: 2 * gm * Bc].reshape(Bc, gm)
        self.u_res = u[2 * gm * Bc:]

    # ---- after it ----
    def after(self, run_oracle=True):
        """Runs the oracle step (teacher-forced) and compares; returns the oracle's wall time."""
        import time

        dec = self.dec
        Bc, G, S_t, S_c = dec.last_key
        V = dec.t.s.vocab
        gpu_dl = dec.draft_logits[:Bc].float().cpu()
        gpu_tl = dec.target_logits[: Bc * S_t].float().cpu().view(Bc, S_t, V)
        gpu_dt = dec.draft_tok[:Bc].cpu().numpy()
        geff = dec.gamma_eff[:Bc].cpu().numpy()
        acc = dec.res.accepted_len.cpu().numpy()
        toks = dec.res.tokens.cpu().numpy()
        gmarg = dec.res.margin.cpu().numpy()
        n_drafts = Counter()

        def hook(stage, i, slots, mine):
            if stage == "draft":
                for b in slots:
                    n_drafts[b] += 1
                return gpu_dl[slots, i]
            return torch.cat([gpu_tl[b, : n_drafts[b] + 1] for b in slots])

        tc = OS.PagedCache([tuple(None if t is None else t.clone() for t in L) for L in self.pre[0]],
                           dec.tkv.block_table.cpu().numpy(), dec.tkv.block_size, dec.tkv.kv_dtype)
        dcch = OS.PagedCache([tuple(None if t is None else t.clone() for t in L) for L in self.pre[1]],
                             dec.dkv.block_table.cpu().numpy(), dec.dkv.block_size, dec.dkv.kv_dtype)
        t0 = time.perf_counter()
        rec, own = OS.step(self.seqs, self.target, self.draft, tc, dcch, dec.T, self.u_draft,
                           self.u_acc, self.u_res, catchup_cap=S_c, logits_hook=hook)
        secs = time.perf_counter() - t0
        self._compare(rec, own, tc, dcch, gpu_dl, gpu_tl, gpu_dt, geff, acc, toks, gmarg, S_t)
        return secs

    def _flip(self, b, what, margin):
        self.stats["ties"] += 1
        self.log.append(f"slot {b} (seq {self.ids[b]}): {what} differs at margin {margin:.3g}")
        self.diverged.add(self.ids[b])

    def _compare(self, rec, own, tc, dcch, gpu_dl, gpu_tl, gpu_dt, geff, acc, toks, gmarg, S_t):
        dec, st = self.dec, self.stats
        flipped = set()
        for b, r in enumerate(rec):
            if self.ids[b] in self.diverged:
                continue
            st["sequences"] += 1
            # which sequences speculate, and how many drafts
            assert len(r.drafts) == int(geff[b]), \
                f"slot {b}: oracle drafted {len(r.drafts)}, GPU verified {geff[b]} drafts"
            for i, t in enumerate(r.drafts):
                st["draft_tokens"] += 1
                if int(gpu_dt[b, i]) != t:
                    assert r.margins[i] < self.tie, \
                        f"slot {b}: draft {i} GPU {gpu_dt[b, i]} oracle {t} margin {r.margins[i]:.3g}"
                    self._flip(b, f"draft {i}", r.margins[i])
                    flipped.add(b)
                    break
            if b in flipped:
                continue
            st["accept_decisions"] += 1
            got = toks[b, : int(acc[b]) + 1].tolist()
            if int(acc[b]) != r.k or got != r.new:
                m = min(r.margin, float(gmarg[b]))
                assert m < self.tie, f"slot {b}: accept GPU {got} oracle {r.new} margin {m:.3g}"
                self._flip(b, "accept", m)
                flipped.add(b)
                continue
            st["emitted_tokens"] += len(r.new)
        # state after the step
        n, dc = dec.n.cpu().tolist(), dec.dc.cpu().tolist()
        hist = dec.hist.cpu()
        for b, s in enumerate(self.seqs):
            if self.ids[b] in self.diverged:
                continue
            assert hist[b, : n[b]].tolist() == s.tokens, f"slot {b}: token history differs"
            assert n[b] - 1 == s.num_computed and dc[b] == s.draft_computed, \
                f"slot {b}: (num_computed, draft_computed) GPU {(n[b] - 1, dc[b])} " \
                f"oracle {(s.num_computed, s.draft_computed)}"
        if not flipped and not self.diverged:
            e0, d0, a0 = self.counters
            assert int(dec.emitted) - e0 == sum(len(r.new) for r in rec)
            assert int(dec.drafted) - d0 == sum(len(r.drafts) for r in rec)
            assert int(dec.accepted) - a0 == sum(r.k for r in rec if r.drafts)
        # logits: the oracle's own forward against the GPU's
        skip = {b for b in range(len(rec)) if self.ids[b] in self.diverged}
        for (stage, i), (slots, mine) in own.items():
            if stage == "draft":
                ref = gpu_dl[slots, i]
                keep = [j for j, b in enumerate(slots) if b not in skip]
                mine, ref = mine[keep], ref[keep]
            else:
                rows = []
                for b in slots:
                    rows.append((b, len(rec[b].drafts) + 1))
                ref = torch.cat([gpu_tl[b, :k] for b, k in rows])
                keep = np.concatenate([[b not in skip] * k for b, k in rows]).astype(bool)
                mine, ref = mine[torch.from_numpy(keep)], ref[torch.from_numpy(keep)]
            if mine.numel() == 0:
                continue
            err = float((mine - ref).abs().max() / max(1.0, float(ref.abs().max())))
            key = "logit_err_draft" if stage == "draft" else "logit_err_target"
            self.worst[key] = max(self.worst[key], err)
            assert self.logit_tol is None or err <= self.logit_tol, \
                f"{stage} {i}: logits differ by {err:.3g} (relative)"
            agree = (mine.argmax(-1) == ref.argmax(-1)).float().mean().item()
            st[key.replace("err", "argmax_rows")] += mine.shape[0]
            st[key.replace("err", "argmax_agree")] += round(agree * mine.shape[0])
        if flipped or self.diverged:
            return   # a diverged sequence's writes differ by construction
        for name, pre, oc, gkv in (("target", self.pre[0], tc, dec.tkv), ("draft", self.pre[1], dcch, dec.dkv)):
            written = np.unique(np.asarray(oc.written, dtype=np.int64))
            mask = np.zeros(pre[0][0].shape[0] * oc.block_size, dtype=bool)
            mask[written] = True
            post = _cache_copy(gkv)
            for li in range(len(pre)):
                self._kv_error(name, li, pre[li], oc.layers[li], post[li], mask, oc.block_size)

    def _kv_error(self, name, li, pre, orc, post, mask, bs):
        """Entries outside the written slots unchanged; written ones close to the oracle's."""
        flat = lambda t: t.reshape(t.shape[0] * bs, *t.shape[2:])
        w = torch.from_numpy(mask)
        for j in range(len(pre)):
            if pre[j] is None:
                continue
            a, g = flat(pre[j]), flat(post[j])
            assert torch.equal(a[~w], g[~w]), f"{name} layer {li}: GPU wrote outside the step's slots"
        if pre[2] is None:       # bf16
            for j in range(2):
                o, g = flat(orc[j])[w].float(), flat(post[j])[w].float()
                err = float(((o - g).abs() / o.abs().clamp(min=1.0)).max()) if o.numel() else 0.0
                self.worst[f"kv_err_{name}"] = max(self.worst[f"kv_err_{name}"], err)
                assert self.kv_tol is None or err <= self.kv_tol, f"{name} layer {li}: KV differs by {err:.3g}"
        else:                    # INT8: dequantised values, relative to each vector's range
            for j in range(2):
                oq, os_ = flat(orc[j])[w].float(), flat(orc[j + 2])[w].float()
                gq, gs = flat(post[j])[w].float(), flat(post[j + 2])[w].float()
                od, gd = oq * os_.unsqueeze(-1), gq * gs.unsqueeze(-1)
                rng = (os_ * 127).clamp(min=1e-6).unsqueeze(-1)
                err = float(((od - gd).abs() / rng).max()) if od.numel() else 0.0
                self.worst[f"kv_err_{name}"] = max(self.worst[f"kv_err_{name}"], err)
                assert self.kv_tol is None or err <= self.kv_tol, \
                    f"{name} layer {li}: INT8 KV differs by {err:.3g}"
        self.stats[f"kv_layers_{name}"] += 1

    def summary(self):
        s = dict(self.stats)
        s.update({k: round(v, 5) for k, v in self.worst.items()})
        s["diverged_sequences"] = len(self.diverged)
        return s
