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

noise_floor() (after after()) measures those differences against a float32 reference: the
same step from the same state, teacher-forced on the same GPU logits, with the weights, the
activations, RoPE tables and the bf16 caches' values in float32 (an INT8 cache keeps its
codes: the format, not a rounding).  It returns the GPU's error against that reference next
to the bf16 oracle's own -- the bf16 noise floor, the rule of the reference's
tests/m4_correctness.py:146-151 (agree at least as well as two implementations of the same
model agree with each other).
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
        self.ref32 = None              # float32 reference models, built by noise_floor()
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
        self.seqs0 = [OS.Seq(list(x.tokens), x.num_computed, x.draft_computed, x.gamma)
                      for x in self.seqs]
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
        tc, dcch = self._caches(torch.bfloat16)
        t0 = time.perf_counter()
        rec, own = OS.step(self.seqs, self.target, self.draft, tc, dcch, dec.T, self.u_draft,
                           self.u_acc, self.u_res, catchup_cap=S_c,
                           logits_hook=self._hook(gpu_dl, gpu_tl))
        secs = time.perf_counter() - t0
        self._last = (rec, own, tc, dcch, gpu_dl, gpu_tl, S_c)
        self._compare(rec, own, tc, dcch, gpu_dl, gpu_tl, gpu_dt, geff, acc, toks, gmarg, S_t)
        return secs

    @staticmethod
    def _hook(gpu_dl, gpu_tl):
        """Teacher forcing: the decisions are taken from the GPU step's logits."""
        n_drafts = Counter()

        def hook(stage, i, slots, mine):
            if stage == "draft":
                for b in slots:
                    n_drafts[b] += 1
                return gpu_dl[slots, i]
            return torch.cat([gpu_tl[b, : n_drafts[b] + 1] for b in slots])
        return hook

    def _caches(self, dtype):
        """Oracle caches holding the GPU's pre-step contents; dtype float32 widens the bf16
        caches and dequantises INT8 entries to float32."""
        dec = self.dec

        def copy(t):
            if t is None:
                return None
            return t.float() if (dtype == torch.float32 and t.dtype == torch.bfloat16) else t.clone()

        return tuple(OS.PagedCache([tuple(copy(t) for t in L) for L in pre],
                                   kv.block_table.cpu().numpy(), kv.block_size, kv.kv_dtype, dtype)
                     for pre, kv in ((self.pre[0], dec.tkv), (self.pre[1], dec.dkv)))

    def noise_floor(self):
        """The last checked step against a float32 reference forward (see the module
        docstring).  Returns {quantity: (GPU error, bf16 oracle error)} for the target and
        draft logits (max |x - ref| / max |ref| and the RMS ratio ||x - ref|| / ||ref||), the
        written KV entries (bf16 caches: max |x - ref| / max(1, |ref|) and RMS; INT8 caches:
        dequantised, relative to each vector's range 127 * scale, max and RMS), and the
        fraction of logit rows whose argmax differs from the reference's."""
        dec = self.dec
        rec16, own16, tc16, dc16, gpu_dl, gpu_tl, S_c = self._last
        if self.ref32 is None:
            def w32(model):
                w = _weights(model)
                f = lambda t: t.float()
                return {"embed": f(w["embed"]), "lm_head": f(w["lm_head"]), "norm": f(w["norm"]),
                        "layers": [{k: f(v) for k, v in L.items()} for L in w["layers"]]}
            self.ref32 = (OS.OracleLlama(_shape(dec.t.s), w32(dec.t), dec.max_len, torch.float32),
                          OS.OracleLlama(_shape(dec.d.s), w32(dec.d), dec.max_len, torch.float32))
        seqs = [OS.Seq(list(x.tokens), x.num_computed, x.draft_computed, x.gamma) for x in self.seqs0]
        tc32, dc32 = self._caches(torch.float32)
        rec32, own32 = OS.step(seqs, self.ref32[0], self.ref32[1], tc32, dc32, dec.T, self.u_draft,
                               self.u_acc, self.u_res, catchup_cap=S_c,
                               logits_hook=self._hook(gpu_dl, gpu_tl))
        assert [r.new for r in rec32] == [r.new for r in rec16], "teacher-forced decisions differ"
        out = {}

        def pair(key, gpu, o16, ref):
            def errs(x):
                d = (x - ref).abs()
                return (float(d.max()) / max(float(ref.abs().max()), 1e-30),
                        float(d.pow(2).sum().sqrt()) / max(float(ref.pow(2).sum().sqrt()), 1e-30),
                        float((x.argmax(-1) != ref.argmax(-1)).float().mean()))
            g, o = errs(gpu), errs(o16)
            for i, name in enumerate(("max", "rms", "argmax_differs")):
                prev = out.get(f"{key}_{name}", (0.0, 0.0))
                out[f"{key}_{name}"] = (max(prev[0], g[i]), max(prev[1], o[i]))

        for (stage, i), (slots, ref) in own32.items():
            o16 = own16[(stage, i)][1]
            if stage == "draft":
                gpu = gpu_dl[slots, i]
            else:
                gpu = torch.cat([gpu_tl[b, : len(rec32[b].drafts) + 1] for b in slots])
            pair("logits_" + stage, gpu, o16, ref)
        post = (_cache_copy(dec.tkv), _cache_copy(dec.dkv))
        for name, o16c, o32c, gpost in (("target", tc16, tc32, post[0]), ("draft", dc16, dc32, post[1])):
            bs = o32c.block_size
            written = np.unique(np.asarray(o32c.written, dtype=np.int64))
            idx = torch.from_numpy(written)
            flat = lambda t: t.reshape(t.shape[0] * bs, *t.shape[2:])[idx]
            for li in range(len(gpost)):
                if gpost[li][2] is None:      # bf16 cache: values
                    for j in range(2):
                        ref = flat(o32c.layers[li][j]).float()
                        den = ref.abs().clamp(min=1.0)
                        for who, x in (("gpu", flat(gpost[li][j]).float()),
                                       ("o16", flat(o16c.layers[li][j]).float())):
                            d = (x - ref).abs()
                            e = (float((d / den).max()), float(d.pow(2).mean().sqrt()) /
                                 max(float(ref.pow(2).mean().sqrt()), 1e-30))
                            self._kv_acc(out, f"kv_{name}", who, e)
                else:                         # INT8: dequantised, per vector range
                    for j in range(2):
                        rq, rs = flat(o32c.layers[li][j]).float(), flat(o32c.layers[li][j + 2]).float()
                        ref = rq * rs.unsqueeze(-1)
                        rng = (rs * 127).clamp(min=1e-6).unsqueeze(-1)
                        for who, cc in (("gpu", gpost[li]), ("o16", o16c.layers[li])):
                            x = flat(cc[j]).float() * flat(cc[j + 2]).float().unsqueeze(-1)
                            d = (x - ref).abs() / rng
                            e = (float(d.max()), float(d.pow(2).mean().sqrt()))
                            self._kv_acc(out, f"kv_{name}", who, e)
        return out

    @staticmethod
    def _kv_acc(out, key, who, e):
        for i, name in enumerate(("max", "rms")):
            g, o = out.get(f"{key}_{name}", (0.0, 0.0))
            out[f"{key}_{name}"] = (max(g, e[i]), o) if who == "gpu" else (g, max(o, e[i]))

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
