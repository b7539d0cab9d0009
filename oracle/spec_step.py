"""One speculative decoding step on the CPU, restating the reference engine.  TEST
INFRASTRUCTURE ONLY: tests/ and bench.py's cpu_baseline leg use it as the checker of
SpecDecoder's step; the product never imports it.

Restated (reference file:line):
  Llama forward           engine/model.py:181-213 (forward_reference: fp32 RMSNorm cast to
                          bf16 (:85-89), neox RoPE in bf16 ops (:92-94, :196-200), K/V written
                          to the paged cache before attention reads them (:201-203), residual
                          adds in bf16), RoPE tables :120-124, logits :215-218
  varlen batch            engine/batch.py:23-55 (one item = tokens appended at `start`)
  draft phase             engine/engine.py:338-404 (catch-up items for lag <= 2, lagging
                          sequences catch up over lag - 1 tokens with gamma forced to 0, the
                          per-step proposal loop over the still-active sequences)
  verify items            engine/engine.py:414-417 ([last token] + drafts, all logits)
  accept                  engine/engine.py:421-446 (greedy: one argmax + prefix compare;
                          sampling: verify() per sequence, sample() for gamma 0)
  append + rollback       engine/engine.py:463-470 (num_computed = len - 1, draft_computed
                          clamped to it)
with three deliberate substitutions:
  * attention is oracle.paged's closed form (bottom-right causal mask, GQA) in fp32 over the
    cache, not vLLM's FlashAttention (third-party, absent; see oracle/paged.py);
  * an INT8 target cache stores oracle.codec.quantize(k) on write and attends over
    dequantize(...) in bf16 (eval/quality.py:48-52);
  * random draws are explicit uniforms (oracle.accept: inverse-CDF sampling, u < ratio).
Every sequence decodes (no prefill chunks in the step), as in the build's step; the catch-up
of a lagging sequence is bounded per step by `catchup_cap` (None: the reference's budget,
taken as unbounded).

Teacher forcing.  `logits_hook(stage, i, slots, logits)` is called with the oracle's own
logits rows for the sequences `slots` at each decision point -- ("draft", i) for the i-th
proposal round, ("target", 0) for the verify rows (concatenated per sequence) -- and returns
the logits the decision is taken from.  A test passes the GPU step's logits there, so the
oracle decides from the same numbers the kernels saw and every decision can be compared
exactly, while the oracle's own logits are kept in the record for a tolerance check.

Pinned by tests/test_oracle_spec_step.py: the stages reduce to the pinned oracle functions
(attention == oracle.paged.attention, slots == oracle.paged.slot_mapping, codec ==
oracle.codec), rms_norm / RoPE against their closed forms, the varlen layout against
build_batch's definition, and the draft phase / rollback bookkeeping against hand-worked
cases (lag 1 and 2, lagging catch-up, gamma 0, the all-accepted bonus).
"""
import math
from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F

from . import accept as OA
from . import codec as OC


# ---- model -------------------------------------------------------------------------------

def rope_tables(theta: float, head_dim: int, max_pos: int, dtype=torch.bfloat16):
    """engine/model.py:69-71, 120-124 without rope_scaling: fp32 angles, cast to dtype."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rms_norm(x, weight, eps):
    """engine/model.py:85-89."""
    dtype = x.dtype
    x = x.float()
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return weight * x.to(dtype)


def rotate_half(x):
    """engine/model.py:92-94."""
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


@dataclass
class Shape:
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    eps: float = 1e-5
    rope_theta: float = 500000.0


class PagedCache:
    """One model's per-layer caches in the reference layout [NB, bs, Hkv, D] (bf16, or int8
    codes with fp16 scales [NB, bs, Hkv]) and its per-slot block tables [slots, W].
    value_dtype: the type INT8 entries are dequantised to before attention (bf16, as
    dequantize() returns them; float32 for an fp32 reference forward)."""

    def __init__(self, layers, block_table, block_size, kv_dtype, value_dtype=torch.bfloat16):
        self.layers = [list(L) for L in layers]       # (k, v, k_scale, v_scale) per layer
        self.block_table = np.asarray(block_table, dtype=np.int64)
        self.block_size = block_size
        self.kv_dtype = kv_dtype
        self.value_dtype = value_dtype
        self.written = []                             # slots written since reset_log()

    def reset_log(self):
        self.written = []

    def slots(self, slot, start, end):
        """engine/block_manager.py:216-220 for one sequence's positions [start, end)."""
        pos = np.arange(start, end, dtype=np.int64)
        bs = self.block_size
        return self.block_table[slot][pos // bs] * bs + pos % bs

    def write(self, layer, k, v, slots):
        """engine/model.py:201-203 (kc[blk, off] = k); INT8: quantize-on-write."""
        kc, vc, ks, vs = self.layers[layer]
        slots = np.asarray(slots, dtype=np.int64)
        blk = torch.from_numpy(slots // self.block_size)
        off = torch.from_numpy(slots % self.block_size)
        if self.kv_dtype == "int8":
            for x, cache, scale in ((k, kc, ks), (v, vc, vs)):
                q, s = OC.quantize(x.float().numpy(), 8)
                cache[blk, off] = torch.from_numpy(q)
                scale[blk, off] = torch.from_numpy(s)
        else:
            kc[blk, off] = k.to(kc.dtype)
            vc[blk, off] = v.to(vc.dtype)
        if layer == 0:
            self.written.extend(slots.tolist())

    def gather(self, layer, slot, L):
        """Keys / values at positions [0, L) of a sequence, as the bf16 values attended over
        (INT8: dequantize(q, s, 8, bf16), engine/kv_tier_manager.py:34-41)."""
        kc, vc, ks, vs = self.layers[layer]
        s = self.slots(slot, 0, L)
        blk = torch.from_numpy(s // self.block_size)
        off = torch.from_numpy(s % self.block_size)
        if self.kv_dtype == "int8":
            K = (kc[blk, off].float() * ks[blk, off].float().unsqueeze(-1)).to(self.value_dtype)
            V = (vc[blk, off].float() * vs[blk, off].float().unsqueeze(-1)).to(self.value_dtype)
            return K, V
        return kc[blk, off], vc[blk, off]


def attend(q, cache, layer, items, scale):
    """Paged causal GQA attention in fp32 (oracle.paged.attention_seq's closed form): query j
    of an item with n new rows and L = start + n keys sees keys [0, L - n + j]."""
    T, H, D = q.shape
    out = torch.empty_like(q)
    row = 0
    for slot, toks, start in items:
        n = len(toks)
        L = start + n
        K, V = cache.gather(layer, slot, L)
        Hkv = K.shape[1]
        G = H // Hkv
        Kh = K.float().permute(1, 2, 0)                              # [Hkv, D, L]
        Vh = V.float().permute(1, 0, 2)                              # [Hkv, L, D]
        Q = q[row:row + n].float().view(n, Hkv, G, D).permute(1, 0, 2, 3).reshape(Hkv, n * G, D)
        s = torch.matmul(Q, Kh) * scale
        lim = torch.repeat_interleave(L - n + torch.arange(n), G)
        s = s.masked_fill(torch.arange(L)[None, None, :] > lim[None, :, None], float("-inf"))
        o = torch.matmul(torch.softmax(s, -1), Vh)
        out[row:row + n] = o.view(Hkv, n, G, D).permute(1, 0, 2, 3).reshape(n, H, D).to(q.dtype)
        row += n
    return out


class OracleLlama:
    """engine/model.py:181-218 on the CPU.  weights: embed, lm_head, norm and per layer
    ln1, ln2, qkv [(H + 2 Hkv) D, hidden], o, gate_up [2 F, hidden], down -- row-major, in the
    compute dtype (bf16 as the reference runs; float32 for a reference forward without bf16
    roundings, whose RoPE tables are then float32 too)."""

    def __init__(self, shape: Shape, weights: dict, max_pos: int, dtype=torch.bfloat16):
        self.s, self.w = shape, weights
        self.cos, self.sin = rope_tables(shape.rope_theta, shape.head_dim, max_pos, dtype)
        self.scale = 1.0 / math.sqrt(shape.head_dim)

    def forward(self, cache: PagedCache, items, all_logits):
        """items: [(slot, tokens, start)] (engine/batch.py:23-55 layout); returns fp32 logits
        of every row of an item with all_logits[i], else of its last row, in item order."""
        s, w = self.s, self.w
        H, Hkv, D = s.heads, s.kv_heads, s.head_dim
        ids = torch.tensor([t for _, toks, _ in items for t in toks], dtype=torch.int64)
        pos = torch.cat([torch.arange(st, st + len(toks)) for _, toks, st in items])
        slots = np.concatenate([cache.slots(sl, st, st + len(toks)) for sl, toks, st in items])
        rows, off = [], 0
        for (sl, toks, st), full in zip(items, all_logits):
            rows.extend(range(off, off + len(toks)) if full else [off + len(toks) - 1])
            off += len(toks)
        T = ids.numel()
        cos, sin = self.cos[pos].unsqueeze(1), self.sin[pos].unsqueeze(1)
        x = F.embedding(ids, w["embed"])
        for i, L in enumerate(w["layers"]):
            h = rms_norm(x, L["ln1"], s.eps)
            q, k, v = F.linear(h, L["qkv"]).split([H * D, Hkv * D, Hkv * D], dim=-1)
            q, k, v = q.reshape(T, H, D), k.reshape(T, Hkv, D), v.reshape(T, Hkv, D)
            q = q * cos + rotate_half(q) * sin
            k = k * cos + rotate_half(k) * sin
            cache.write(i, k, v, slots)
            attn = attend(q, cache, i, items, self.scale)
            x = x + F.linear(attn.reshape(T, H * D), L["o"])
            h = rms_norm(x, L["ln2"], s.eps)
            gate, up = F.linear(h, L["gate_up"]).chunk(2, dim=-1)
            x = x + F.linear(F.silu(gate) * up, L["down"])
        x = rms_norm(x[torch.tensor(rows, dtype=torch.int64)], w["norm"], s.eps)
        return F.linear(x, w["lm_head"]).float()


# ---- the step ----------------------------------------------------------------------------

@dataclass
class Seq:
    """The per-sequence state the step reads and updates (engine/engine.py:33-62)."""
    tokens: list
    num_computed: int
    draft_computed: int
    gamma: int = 0
    accepted_total: int = 0
    drafted_total: int = 0


@dataclass
class SeqRecord:
    drafts: list = field(default_factory=list)
    proposed: bool = False
    catchup: int = 0          # draft tokens processed by the catch-up forward
    new: list = field(default_factory=list)
    k: int = 0
    margin: float = float("inf")
    margins: list = field(default_factory=list)  # each draft sample's inverse-CDF margin


def _sample_rows(logits, temperature, u):
    """spec_decode.sample (engine/spec_decode.py:12-17) with inverse-CDF draws: tokens,
    probs (None when greedy) and each row's margin."""
    x = logits.float().numpy()
    if not temperature > 0:
        return x.argmax(axis=-1).tolist(), None, [float("inf")] * len(x)
    p = OA.softmax32(x, OA.inv_temperature(temperature))
    out = [OA.inverse_cdf(p[r], u[r]) for r in range(len(x))]
    return [t for t, _ in out], p, [m for _, m in out]


def step(seqs, target: OracleLlama, draft: OracleLlama, tcache: PagedCache, dcache: PagedCache,
         temperature, u_draft, u_acc, u_res, catchup_cap=None, logits_hook=None):
    """One engine step over `seqs` (index = slot).  u_draft[i][b], u_acc[b][i], u_res[b]:
    the uniforms of draft round i, accept test i and the emitted token of sequence b.
    Mutates seqs and the caches; returns (records per slot, own logits per stage)."""
    hook = logits_hook or (lambda stage, i, slots, x: x)
    rec = [SeqRecord() for _ in seqs]
    own = {}
    # ---- draft phase (engine/engine.py:338-404) ----
    items, owners, spec = [], [], []
    for b, s in enumerate(seqs):
        if s.gamma <= 0:
            continue
        lag = len(s.tokens) - s.draft_computed
        if lag <= 2:
            spec.append(b)
            items.append((b, s.tokens[s.draft_computed:], s.draft_computed))
            owners.append((b, len(s.tokens), True))
            continue
        s.gamma = 0
        n = lag - 1 if catchup_cap is None else min(lag - 1, catchup_cap)
        if n > 0:
            items.append((b, s.tokens[s.draft_computed:s.draft_computed + n], s.draft_computed))
            owners.append((b, s.draft_computed + n, False))
    dprobs = {b: [] for b in spec}
    if items:
        logits = draft.forward(dcache, items, [False] * len(items))
        props = []
        for r, (b, end, proposes) in enumerate(owners):
            rec[b].catchup = end - seqs[b].draft_computed
            seqs[b].draft_computed = end
            if proposes:
                props.append((b, r))
                rec[b].proposed = True
        for i in range(max((seqs[b].gamma for b in spec), default=0)):
            if i > 0:
                active = [b for b in spec if seqs[b].gamma > i]
                if not active:
                    break
                logits = draft.forward(dcache, [(b, [rec[b].drafts[-1]], seqs[b].draft_computed)
                                                for b in active], [False] * len(active))
                props = [(b, r) for r, b in enumerate(active)]
                for b in active:
                    seqs[b].draft_computed += 1
            slots = [b for b, _ in props]
            mine = logits[torch.tensor([r for _, r in props], dtype=torch.int64)]
            own[("draft", i)] = (slots, mine)
            use = hook("draft", i, slots, mine)
            toks, probs, margins = _sample_rows(use, temperature, [u_draft[i][b] for b in slots])
            for j, b in enumerate(slots):
                rec[b].drafts.append(int(toks[j]))
                rec[b].margins.append(margins[j])
                if probs is not None:
                    dprobs[b].append(probs[j])
    # ---- target verify (engine/engine.py:414-420) ----
    order = list(range(len(seqs)))
    titems = [(b, [seqs[b].tokens[-1]] + rec[b].drafts, seqs[b].num_computed) for b in order]
    full = [bool(rec[b].drafts) for b in order]
    mine = target.forward(tcache, titems, full)
    own[("target", 0)] = (order, mine)
    logits = hook("target", 0, order, mine)
    # ---- accept (engine/engine.py:421-461) ----
    spans, row = [], 0
    for b in order:
        n = len(rec[b].drafts) + 1
        spans.append((row, n))
        row += n
    greedy = not temperature > 0
    for b, (r0, n) in zip(order, spans):
        s, d = seqs[b], rec[b].drafts
        x = logits[r0:r0 + n].numpy()
        if greedy:
            tgt = x.argmax(axis=-1).tolist()
            k = 0
            while k < len(d) and tgt[k] == d[k]:
                k += 1
            new, margin = d[:k] + [tgt[k]], float("inf")
        elif d:
            new, k, margin = OA.verify(x, d, np.stack(dprobs[b]), temperature,
                                       np.asarray(u_acc[b][:len(d)], np.float32), u_res[b],
                                       draft_is_probs=True)
        else:
            toks, _, m = _sample_rows(logits[r0:r0 + 1], temperature, [u_res[b]])
            new, k, margin = [int(toks[0])], 0, m[0]
        if d:
            s.accepted_total += k
            s.drafted_total += len(d)
        rec[b].new, rec[b].k, rec[b].margin = [int(t) for t in new], k, margin
        # _append without stop conditions (engine/engine.py:293-308), then the rollback
        s.tokens.extend(rec[b].new)
        s.num_computed = len(s.tokens) - 1
        s.draft_computed = min(s.draft_computed, len(s.tokens) - 1)
    return rec, own
