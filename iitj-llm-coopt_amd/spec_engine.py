"""One speculative decoding step on the gfx950 kernels, device-resident and graph-capturable.

The draft proposes gamma tokens autoregressively, the target scores all gamma + 1 positions in
one forward over its paged (INT8) KV cache, and the fused accept kernel keeps a prefix plus
one target token -- the decode path of Engine.step / _draft_phase (engine/engine.py:325-470)
for a batch in which every sequence is decoding:
  draft catch-up over tokens[draft_computed:] (lag 1 or 2)      engine/engine.py:358-378
  gamma draft proposals, sampled at temperature T                engine/engine.py:384-404
  verify item [last token] + drafts, logits at every position    engine/engine.py:414-417
  accept (greedy prefix rule / rejection sampling)               engine/engine.py:421-446
  rollback: num_computed = len - 1, draft_computed clamped        engine/engine.py:463-470
Rollback needs no cache writes: KV beyond a sequence's length is simply overwritten by its
next step (slots are a pure function of position and block table).

Everything per step lives on the device (token history, lengths, block tables), shapes are
fixed (the padded layout of engine/cuda_graphs.py:7-16: the catch-up forward has stride 2,
a lag-1 sequence's second row is padding whose KV write is skipped), so a whole step can be
captured in one HIP graph.  Models are Llama-shaped with random weights; the kernels are
reached through an `ops` object (HipOps here) so the same step can run on other backends.
"""
import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from . import _lib
from .attention import (paged_attention, paged_attention_qkv, qkv_attention_supported,
                        workspace_bytes)
from .batch import row_slots
from .fused import (LinearPartials, linear, linear_silu, pack_gate_up_weight, pack_linear_weight,
                    rms_norm, rope_,
                    row_major, silu_and_mul)
from .kv_cache import allocate_kv_cache, qkv_rope_and_cache, reshape_and_cache_flash
from .spec_decode import AcceptResult, accept

__all__ = ["LlamaShape", "TARGET_LLAMA31_8B", "DRAFT_LLAMA32_1B", "RandomLlama", "PagedKV",
           "HipOps", "SpecDecoder"]


@dataclass(frozen=True)
class LlamaShape:
    hidden: int
    ffn: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    rope_theta: float = 500000.0
    eps: float = 1e-5
    tie_embeddings: bool = False

    def params(self) -> int:
        qkv = (self.heads + 2 * self.kv_heads) * self.head_dim * self.hidden
        o = self.heads * self.head_dim * self.hidden
        mlp = 3 * self.ffn * self.hidden
        per_layer = qkv + o + mlp + 2 * self.hidden
        emb = self.vocab * self.hidden
        return self.layers * per_layer + emb * (1 if self.tie_embeddings else 2) + self.hidden


TARGET_LLAMA31_8B = LlamaShape(4096, 14336, 32, 32, 8, 128, 128256, 500000.0)
DRAFT_LLAMA32_1B = LlamaShape(2048, 8192, 16, 32, 8, 64, 128256, 500000.0, tie_embeddings=True)


class RandomLlama:
    """Llama decoder with N(0, std^2) weights (unit norms), bf16 on `device`."""

    def __init__(self, shape: LlamaShape, device, seed=0, std=0.02, max_pos=8192,
                 dtype=torch.bfloat16, packed=None):
        self.s, self.device, self.dtype = shape, torch.device(device), dtype
        self.packed = tuple(self.PACKED if packed is None else packed)
        g = torch.Generator(device=self.device).manual_seed(seed)

        def w(*size):
            return (torch.randn(*size, generator=g, device=self.device, dtype=torch.float32)
                    * std).to(dtype)

        H, D = shape.hidden, shape.head_dim
        self.embed = w(shape.vocab, H)
        self.lm_head = self.embed if shape.tie_embeddings else w(shape.vocab, H)
        self.norm = torch.ones(H, device=self.device, dtype=dtype)
        self.layers = []
        for _ in range(shape.layers):
            self.layers.append({
                "ln1": torch.ones(H, device=self.device, dtype=dtype),
                "ln2": torch.ones(H, device=self.device, dtype=dtype),
                "qkv": w((shape.heads + 2 * shape.kv_heads) * D, H),
                "o": w(H, shape.heads * D),
                "gate_up": w(2 * shape.ffn, H),
                "down": w(H, shape.ffn),
            })
        if self.device.type == "cuda":
            self._pack()
        inv = 1.0 / (shape.rope_theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
        freqs = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv)
        emb = torch.cat((freqs, freqs), dim=-1)           # neox layout, as HF Llama
        self.cos = emb.cos().to(device=self.device, dtype=dtype)
        self.sin = emb.sin().to(device=self.device, dtype=dtype)
        self.scale = 1.0 / math.sqrt(D)

    # Projections kept tile-packed as well on the GPU: those that stream through coopt_linear
    # at verify row counts.  A model run only at draft row counts (<= 64) streams gate_up
    # through it too, and its logits projection, and passes
    # packed=("qkv", "o", "gate_up", "down", "lm_head").  At 160 rows the target's lm_head
    # runs on torch's GEMM, and so does its gate_up: the fused gate_up + SiLU kernel takes 160
    # rows too, but the step measured 11.72 ms with it against 11.58 ms with hipBLASLt.
    PACKED = ("qkv", "o", "down")

    def _pack(self):
        ok = lambda w, r=16: w.shape[0] % r == 0 and w.shape[1] % 128 == 0  # tile granularity
        for L in self.layers:
            for k in self.packed:
                if k in L and ok(L[k], 32 if k == "gate_up" else 16):
                    # gate_up: gate / up tiles interleaved, for the fused SiLU epilogue
                    L[k] = pack_gate_up_weight(L[k]) if k == "gate_up" else pack_linear_weight(L[k])
        if "lm_head" in self.packed and ok(self.lm_head):
            self.lm_head = pack_linear_weight(self.lm_head)   # embed keeps the row-major copy

    def to(self, device):
        """A copy of the weights on another device (same values)."""
        other = object.__new__(RandomLlama)
        other.s, other.device, other.dtype = self.s, torch.device(device), self.dtype
        other.packed = self.packed
        other.embed = self.embed.to(device)
        other.lm_head = other.embed if self.s.tie_embeddings else row_major(self.lm_head).to(device)
        other.norm = self.norm.to(device)
        other.layers = [{k: row_major(v).to(device) for k, v in L.items()} for L in self.layers]
        if other.device.type == "cuda":
            other._pack()
        other.cos, other.sin, other.scale = self.cos.to(device), self.sin.to(device), self.scale
        return other

    def forward(self, ops, kv, ids, pos, slots, meta, logits_out=None, keep_rows=None):
        """ids/pos/slots [T]; meta: attention metadata for ops.attend; returns logits [T, V],
        or only the rows `keep_rows` (int64 indices into the T rows) of them.

        The layer structure of the reference's fused forward (engine/model.py:220-255): the
        residual stream x is updated in place by the fused add + RMSNorm, RoPE rotates q and k
        in place inside the qkv projection's output, K/V are written to the paged cache before
        attention reads them back."""
        s = self.s
        T = ids.shape[0]
        H, Hkv, D = s.heads, s.kv_heads, s.head_dim
        x = F.embedding(ids, self.embed)                       # residual stream
        d = None
        for li, L in enumerate(self.layers):
            h = ops.rms_norm(x if d is None else d, None if d is None else x, L["ln1"], s.eps)
            # qkv projection, RoPE, the KV write and attention (engine/model.py:238-247):
            # split-K partials straight into one launch that reduces them, writes the paged
            # cache and attends (ops.attend_qkv), or into the epilogue launch that writes q
            # and the cache, then attention
            qkv = ops.linear(h, L["qkv"], defer_reduce=True)
            attend_qkv = getattr(ops, "attend_qkv", None)
            attn = None if attend_qkv is None else attend_qkv(
                kv, li, qkv, pos, self.cos, self.sin, slots, meta, self.scale, H, Hkv, D)
            if attn is None:
                q = ops.qkv_epilogue(kv, li, qkv, pos, self.cos, self.sin, slots, H, Hkv, D)
                attn = ops.attend(kv, li, q, meta, self.scale)
            # gate_up + SiLU·mul is one launch at draft row counts (linear_silu); o, down and
            # otherwise gate_up feed only the fused add + norm or SiLU, which reduce their
            # split-K partials as they read them
            o = ops.linear(attn.reshape(T, H * D), L["o"], defer_reduce=True)
            h = ops.rms_norm(o, x, L["ln2"], s.eps)
            d = ops.linear(ops.linear_silu(h, L["gate_up"]), L["down"], defer_reduce=True)
        h = ops.rms_norm(d, x, self.norm, s.eps)
        if keep_rows is not None:
            h = h.index_select(0, keep_rows)
        return ops.linear(h, self.lm_head, out=logits_out)


class PagedKV:
    """Per-layer paged caches of one model plus the batch's block tables.

    Every sequence owns `width` blocks of a shared pool, handed out in a seeded random order
    (block tables scattered over the pool, as in a long-running server)."""

    def __init__(self, shape: LlamaShape, batch: int, max_tokens: int, kv_dtype: str, device,
                 block_size=16, seed=0):
        self.kv_dtype, self.block_size = kv_dtype, block_size
        self.width = -(-max_tokens // block_size)
        self.num_blocks = batch * self.width + 1
        perm = np.random.default_rng(seed).permutation(self.num_blocks)
        table = perm[: batch * self.width].reshape(batch, self.width).astype(np.int32)
        self.block_table = torch.from_numpy(table).to(device)
        self.layers = [allocate_kv_cache(self.num_blocks, block_size, shape.kv_heads,
                                         shape.head_dim, kv_dtype, device=device)
                       for _ in range(shape.layers)]

    def slots(self, pos):
        """pos [B, S] int64 -> cache slots [B*S] int64 (engine/block_manager.py:216-220)."""
        bs = self.block_size
        blk = torch.gather(self.block_table.long(), 1, pos // bs)
        return (blk * bs + pos % bs).reshape(-1)

    def nbytes(self):
        return sum(t.numel() * t.element_size() for L in self.layers for t in L if t is not None)

    def to(self, device):
        """A copy (same block tables and cache contents) on another device."""
        other = object.__new__(PagedKV)
        other.kv_dtype, other.block_size = self.kv_dtype, self.block_size
        other.width, other.num_blocks = self.width, self.num_blocks
        other.block_table = self.block_table.to(device)
        other.layers = [tuple(None if t is None else t.to(device) for t in L) for L in self.layers]
        return other


class HipOps:
    """The gfx950 kernels behind the step, with preallocated workspaces (capture-safe).
    fuse_qkv: run each layer's qkv epilogue inside its attention launch where the shape
    allows (attend_qkv); the results are the same bit for bit."""

    def __init__(self, device, fuse_qkv=True):
        self.device = torch.device(device)
        self.fuse_qkv = fuse_qkv
        self._ws = {}
        self._retired = []   # outgrown workspaces, kept alive for graphs that captured them

    def workspace(self, key, nbytes):
        """A device buffer of at least nbytes for `key`.  A larger request replaces the buffer,
        but the old one is kept alive: a graph captured earlier still writes through its
        address (graphs of the smaller shapes keep using it, which is safe because replays
        run in stream order)."""
        buf = self._ws.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                self._retired.append(buf)
            buf = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=self.device)
            self._ws[key] = buf
        return buf

    def write(self, kv: PagedKV, layer, k, v, slots):
        kc, vc, ks, vs = kv.layers[layer]
        reshape_and_cache_flash(k, v, kc, vc, slots, kv.kv_dtype, ks, vs)

    def rms_norm(self, x, residual, w, eps):
        return rms_norm(x, w, eps, residual=residual)

    def rope(self, q, k, pos, cos, sin):
        rope_(q, k, pos, cos, sin)

    def qkv_epilogue(self, kv: "PagedKV", layer, qkv, pos, cos, sin, slots, H, Hkv, D):
        kc, vc, ks, vs = kv.layers[layer]
        return qkv_rope_and_cache(qkv, pos, cos, sin, kc, vc, slots, H, Hkv, D, kv.kv_dtype,
                                  ks, vs)

    def silu_mul(self, gate_up):
        return silu_and_mul(gate_up)

    def row_slots(self, kv: "PagedKV", start, S, n_real):
        return row_slots(kv.block_table, start, S, kv.block_size, n_real)

    def linear_silu(self, x, w):
        return linear_silu(x, w)

    def linear(self, x, w, out=None, defer_reduce=False):
        return linear(x, w, out=out, defer_reduce=defer_reduce)

    def attend(self, kv: PagedKV, layer, q, meta, scale):
        kc, vc, ks, vs = kv.layers[layer]
        cu, seq_lens, S, max_k = meta
        B = seq_lens.numel()
        nb = workspace_bytes(B, q.shape[1], kc.shape[2], q.shape[2], S, max_k)
        ws = self.workspace(("attn", q.shape[2]), nb)
        return paged_attention(q, kc, vc, cu, seq_lens, kv.block_table[:B], S, max_k, scale, ks,
                               vs, workspace=ws)

    def attend_qkv(self, kv: PagedKV, layer, qkv, pos, cos, sin, slots, meta, scale, H, Hkv, D):
        """qkv_epilogue + attend as one launch, or None where that launch does not take the
        shape (the caller then makes the two calls)."""
        if not self.fuse_qkv or (isinstance(qkv, LinearPartials) and qkv.ks > 4):
            return None
        kc, vc, ks, vs = kv.layers[layer]
        cu, seq_lens, S, max_k = meta
        B = seq_lens.numel()
        if not qkv_attention_supported(kv.kv_dtype, B, H, Hkv, D, S, max_k):
            return None
        ws = self.workspace(("attn", D), workspace_bytes(B, H, Hkv, D, S, max_k))
        return paged_attention_qkv(qkv, pos, cos, sin, slots, kc, vc, cu, seq_lens,
                                   kv.block_table[:B], S, max_k, H, scale, kv.kv_dtype, ks, vs,
                                   workspace=ws)

    def sample(self, logits, u, temperature, out=None):
        """One token per row: inverse-CDF draw from softmax(logits / T) (argmax if T <= 0)."""
        N, V = logits.shape
        empty = self._empty_tokens(N)
        ws = self.workspace(("acc", 0), _lib.load().coopt_accept_sample_workspace(N, 0, V))
        res = accept(logits, None, empty, temperature, u_resample=u, workspace=ws, out=out)
        return res.tokens[:, 0]

    def accept(self, target_logits, draft_logits, draft_tokens, temperature, u_acc, u_res,
               out=None, gamma_per_seq=None, target_row0=None, draft_row0=None):
        B, g = draft_tokens.shape
        V = target_logits.shape[-1]
        ws = self.workspace(("acc", 1), _lib.load().coopt_accept_sample_workspace(B, g, V))
        return accept(target_logits, draft_logits, draft_tokens, temperature, u_acc, u_res,
                      gamma_per_seq=gamma_per_seq, target_row0=target_row0,
                      draft_row0=draft_row0, workspace=ws, out=out)

    def _empty_tokens(self, n):
        key = ("empty", n)
        t = self._ws.get(key)
        if t is None:
            t = torch.empty((n, 0), dtype=torch.int32, device=self.device)
            self._ws[key] = t
        return t



def target_strides(gamma_max: int):
    """Verify strides the step is bucketed by: {1} and gamma + 1 for gamma in
    (1, 2, 3, 4, 6, 8) up to gamma_max, plus gamma_max + 1 (engine/engine.py:221-225)."""
    return sorted({1} | {g + 1 for g in (1, 2, 3, 4, 6, 8) if g <= gamma_max}
                  | ({gamma_max + 1} if gamma_max else set()))


BATCH_BUCKETS = (1, 2, 4, 8, 16, 32, 64, 96, 128, 160, 192, 224, 256)  # engine/engine.py:161


class SpecDecoder:
    """A batch of sequences decoding speculatively, every step device-resident.

    Per sequence b (its slot) and step, with gamma[b] the caller's draft length
    (engine/engine.py:325-470 for a batch in which every sequence decodes):
      lag = len(tokens) - draft_computed
      gamma[b] > 0 and lag <= 2   speculate: the draft catches up over tokens[dc:] and
                                  proposes gamma[b] tokens; the target verifies
                                  [last] + drafts; rejection sampling keeps a prefix + 1
      gamma[b] > 0 and lag > 2    lagging: the draft catches up over min(lag - 1, S_c) tokens
                                  and proposes nothing; the target decodes one token
      gamma[b] == 0               plain decode: one target token, the draft is not run
    followed by the rollback of engine/engine.py:463-470 (num_computed = len - 1,
    draft_computed clamped to it).  Rollback needs no cache writes: KV beyond a sequence's
    length is overwritten by its next step (slots are a function of position and table).

    Shapes are bucketed as the reference's graph runner buckets them (engine/cuda_graphs.py:
    7-16, 68-104): the first Bc slots of the state are one step's batch, Bc the smallest batch
    bucket >= the live sequences, and the slots past the live ones are dummy sequences (all
    rows padding: no KV write, seq_len = S, outputs discarded).  G = max gamma[b] drafting
    rounds run; the target verify has stride S_t = the smallest stride >= G + 1, and a
    sequence's rows past its own gamma + 1 are padding (slot -1, seq_len = start + S_t, so
    the bottom-right causal mask keeps real rows exact).  The draft catch-up has stride
    S_c = 2, or more when a lagging sequence needs it.  One HIP graph is captured per
    (Bc, G) bucket with S_c = 2; a step that needs a longer catch-up runs eagerly, as the
    reference runs such draft batches outside its graphs.

    The draft catch-up of a lagging sequence runs in one eager step of up to max_catchup
    rows (S_c: the next power of two >= the largest lag - 1, capped there); a longer lag
    takes several steps (engine/engine.py:365-372 bounds it by the step's token budget the
    same way).  At more than 64 / (Hq / Hkv) rows the draft's attention runs in query windows.
    At most max_steps steps run (the history and the block tables are sized for them).

    Random draws come from a uniform table (set_uniforms): step i reads row i of it.  Row
    layout, for the Bcap = max bucket slots and gamma_max:
      [0, gmax*Bcap)                   u_draft[i, b] at i*Bcap + b  (inverse-CDF draw of draft i)
      [gmax*Bcap, 2*gmax*Bcap)         u_acc[b, i] at b*gmax + i    (accept test of draft i)
      [2*gmax*Bcap, (2*gmax+1)*Bcap)   u_res[b]                     (emitted token's draw)
    so a step's decisions are a pure function of the state, the logits and its row.
    """

    def __init__(self, target: RandomLlama, draft: RandomLlama, batch: int, gamma: int,
                 prompt_len: int, max_steps: int, ops=None, target_kv="int8", draft_kv="auto",
                 temperature=1.0, block_size=16, seed=0, batch_buckets=None, max_catchup=64):
        dev = target.device
        if int(max_catchup) < 2:
            raise ValueError("max_catchup must be >= 2 (the graphs' catch-up stride)")
        if int(max_steps) < 1:
            raise ValueError("max_steps must be >= 1")
        self.t, self.d = target, draft
        self.max_steps, self.steps_run = int(max_steps), 0
        self.P, self.T, self.gmax = prompt_len, temperature, gamma
        self.ops = ops or HipOps(dev)
        self.strides = target_strides(gamma)
        self.smax = self.strides[-1]
        buckets = tuple(sorted(BATCH_BUCKETS if batch_buckets is None else batch_buckets))
        self.buckets = tuple(b for b in buckets if b < batch) + (min([b for b in buckets if b >= batch] or [batch]),)
        self.Bcap = self.buckets[-1]
        self.max_catchup = max_catchup
        # positions reach n - 1 + S_t - 1 (verify) and dc + S_c - 1 (catch-up) past the tokens
        self.max_len = prompt_len + 1 + max_steps * (gamma + 1) + self.smax + max_catchup + 2
        Bc = self.Bcap
        self.tkv = PagedKV(target.s, Bc, self.max_len, target_kv, dev, block_size, seed)
        self.dkv = PagedKV(draft.s, Bc, self.max_len, draft_kv, dev, block_size, seed + 1)
        i64 = dict(dtype=torch.int64, device=dev)
        self.hist = torch.zeros((Bc, self.max_len), **i64)
        self.n = torch.zeros(Bc, **i64)          # tokens so far
        self.dc = torch.zeros(Bc, **i64)         # draft KV length (draft_computed)
        self.gamma_dev = torch.zeros(Bc, **i64)  # the caller's gamma per slot (0: dummy)
        self.live_dev = torch.zeros(Bc, dtype=torch.bool, device=dev)
        self.gamma_eff = torch.zeros(Bc, dtype=torch.int32, device=dev)  # drafts verified
        self.emitted = torch.zeros((), **i64)
        self.drafted = torch.zeros((), **i64)
        self.accepted = torch.zeros((), **i64)
        V = target.s.vocab
        self.draft_logits = torch.empty((Bc, self.smax - 1, V), dtype=torch.bfloat16, device=dev)
        self.target_logits = torch.empty((Bc * self.smax, V), dtype=torch.bfloat16, device=dev)
        # proposal i of slot b at prop[i, b]: each draft sample writes its row in place
        self.prop = torch.zeros((self.smax - 1, Bc), dtype=torch.int32, device=dev)
        self.nu = Bc * (2 * gamma + 1)
        self.u = torch.zeros(self.nu, dtype=torch.float32, device=dev)
        self.u_ctr = torch.zeros((), **i64)
        self.graphs = {}
        g = torch.Generator().manual_seed(seed + 17)
        self.set_uniforms(torch.rand((max_steps + 8, self.nu), generator=g))
        # accept outputs; the token rows are [Bc, S_t] per verify stride (contiguous)
        self._acc_len = torch.zeros(Bc, dtype=torch.int32, device=dev)
        self._margin = torch.zeros(Bc, dtype=torch.float32, device=dev)
        self._acc_tok = {S: torch.zeros((Bc, S), dtype=torch.int32, device=dev) for S in self.strides}
        # the step's bookkeeping (coopt_spec_step_*): catch-up, proposal and verify rows
        i32 = dict(dtype=torch.int32, device=dev)
        self._cu_start, self._cu_nreal, self._cu_keep = (torch.zeros(Bc, **i64) for _ in range(3))
        self._cu_tok = torch.zeros(Bc * max_catchup, **i64)
        self._pr_start = torch.zeros((max(self.smax - 2, 1), Bc), **i64)
        self._pr_nreal = torch.zeros((max(self.smax - 2, 1), Bc), **i64)
        self._v_start, self._v_nreal, self._dc_final = (torch.zeros(Bc, **i64) for _ in range(3))
        self._vtok = {S: torch.zeros((Bc, S), **i32) for S in self.strides}
        self._dtok = {S: torch.zeros((Bc, max(S - 1, 1)), **i32) for S in self.strides}
        self._s_len = torch.zeros(Bc, **i32)          # sample outputs other than the token
        self._s_margin = torch.zeros(Bc, dtype=torch.float32, device=dev)
        self.res = AcceptResult(self._acc_len, self._acc_tok[self.smax], self._margin)
        self._cu = {}
        self._row0 = {}
        self.pool = None
        self.last_key = None
        self.B = batch                      # live sequences: slots [0, B)
        self.seq_ids = list(range(batch))   # the caller's id of the sequence in each slot
        self.gamma = [gamma] * batch        # the caller's draft lengths
        self.lag_lo = [1] * batch           # host bounds on len(tokens) - draft_computed
        self.lag_hi = [1] * batch
        self._sync_live()

    # ---- caller inputs ----------------------------------------------------------------
    @property
    def g(self):
        return self.gmax

    @property
    def draft_tok(self):
        """The last step's proposals as [slot, i] (a view of the proposal-major buffer)."""
        return self.prop.t()

    def set_uniforms(self, table):
        """table [rows, (2*gamma_max + 1) * Bcap] fp32 (layout in the class docstring); the next
        step reads row 0, and a step past the last row raises.  A table with as many rows as
        the current one is copied into it, so captured graphs keep reading the right memory
        (their launches hold its address and row count); a table of another size replaces it
        and drops the captured graphs, which are captured again on their next replay."""
        table = torch.as_tensor(table, dtype=torch.float32)
        if table.dim() != 2 or table.shape[1] != self.nu or table.shape[0] < 1:
            raise ValueError(f"uniform table must be [rows >= 1, {self.nu}]")
        cur = getattr(self, "u_table", None)
        if cur is not None and cur.shape == table.shape:
            cur.copy_(table)
        else:
            self.u_table = table.to(self.hist.device).contiguous()
            self.graphs.clear()
        self.u_ctr.zero_()
        self.u_used = 0

    def set_gamma(self, gamma):
        """Draft length per live sequence (int or one per slot); 0 = plain decoding."""
        g = [int(gamma)] * self.B if isinstance(gamma, int) else [int(x) for x in gamma]
        if len(g) != self.B or any(x < 0 or x > self.gmax for x in g):
            raise ValueError(f"gamma must be {self.B} values in [0, {self.gmax}]")
        self.gamma = g
        self._sync_live()

    def retire(self, slot):
        """Drops the sequence in `slot`: the last live sequence moves into it (its history,
        lengths and both block-table rows, so its KV stays where it is)."""
        if not 0 <= slot < self.B:
            raise ValueError("no live sequence in that slot")
        last = self.B - 1
        if slot != last:
            for t in (self.hist, self.n, self.dc, self.tkv.block_table, self.dkv.block_table):
                a, b = t[slot].clone(), t[last].clone()
                t[slot].copy_(b)
                t[last].copy_(a)
            for lst in (self.gamma, self.lag_lo, self.lag_hi, self.seq_ids):
                lst[slot] = lst[last]
        for lst in (self.gamma, self.lag_lo, self.lag_hi, self.seq_ids):
            lst.pop()
        self.B -= 1
        self._sync_live()

    def _sync_live(self):
        live = torch.zeros(self.Bcap, dtype=torch.bool)
        live[: self.B] = True
        gam = torch.zeros(self.Bcap, dtype=torch.int64)
        gam[: self.B] = torch.tensor(self.gamma, dtype=torch.int64)
        self.live_dev.copy_(live)
        self.gamma_dev.copy_(gam)

    # ---- prefill (not part of the timed step) -------------------------------------------
    @torch.inference_mode()
    def prefill(self, prompts: torch.Tensor, u_first: torch.Tensor):
        """prompts [B, P] int64.  Runs both models over the prompt (attention over the prompt
        in fp32 SDPA, KV written through the paged write kernel), samples the first token
        from the target and sets num_computed = P (engine/engine.py:427-436)."""
        B, P = prompts.shape
        if B != self.B:
            raise ValueError(f"{self.B} prompts expected")
        self.hist[:B, :P] = prompts
        pos = torch.arange(P, device=self.hist.device).expand(B, P)
        for model, kv in ((self.t, self.tkv), (self.d, self.dkv)):
            logits = self._prefill_model(model, kv, prompts, pos)
            if model is self.t:
                first = self.ops.sample(logits, u_first, self.T)
        self.hist[:B, P] = first.long()
        self.n[:B] = P + 1
        self.dc[:B] = P
        self.lag_lo, self.lag_hi = [1] * B, [1] * B
        if self.hist.is_cuda:
            torch.cuda.synchronize(self.hist.device)

    def _prefill_model(self, model, kv, ids, pos):
        s = model.s
        B, P = ids.shape
        H, Hkv, D = s.heads, s.kv_heads, s.head_dim
        T = B * P
        flat_pos = pos.reshape(-1).contiguous()
        blk = torch.gather(kv.block_table[:B].long(), 1, pos // kv.block_size)
        slots = (blk * kv.block_size + pos % kv.block_size).reshape(-1)
        x = F.embedding(ids.reshape(-1), model.embed)
        d = None
        for li, L in enumerate(model.layers):
            h = self.ops.rms_norm(x if d is None else d, None if d is None else x, L["ln1"], s.eps)
            qkv = F.linear(h, row_major(L["qkv"]))
            q = qkv[:, : H * D].view(T, H, D)
            k = qkv[:, H * D: (H + Hkv) * D].view(T, Hkv, D)
            v = qkv[:, (H + Hkv) * D:].view(T, Hkv, D)
            self.ops.rope(q, k, flat_pos, model.cos, model.sin)
            self.ops.write(kv, li, k, v, slots)
            # prompt attention in fp32 (plain causal over the prompt; GQA expanded)
            qf = q.reshape(B, P, H, D).transpose(1, 2).float()
            kf = k.reshape(B, P, Hkv, D).transpose(1, 2).float().repeat_interleave(H // Hkv, 1)
            vf = v.reshape(B, P, Hkv, D).transpose(1, 2).float().repeat_interleave(H // Hkv, 1)
            a = F.scaled_dot_product_attention(qf.contiguous(), kf.contiguous(), vf.contiguous(),
                                               is_causal=True, scale=model.scale)
            attn = a.transpose(1, 2).reshape(T, H * D).to(x.dtype)
            o = F.linear(attn, row_major(L["o"]))
            h = self.ops.rms_norm(o, x, L["ln2"], s.eps)
            d = F.linear(self.ops.silu_mul(F.linear(h, row_major(L["gate_up"]))), row_major(L["down"]))
        last_d = d.view(B, P, -1)[:, -1].contiguous()
        last_x = x.view(B, P, -1)[:, -1].contiguous()
        h = self.ops.rms_norm(last_d, last_x, model.norm, s.eps)
        return F.linear(h, row_major(model.lm_head))

    # ---- buckets ----------------------------------------------------------------------
    def bucket(self):
        """(Bc, G, S_t, S_c) of the next step, from the host's gamma and lag bounds."""
        Bc = next(b for b in self.buckets if b >= self.B)
        G = max(self.gamma, default=0)
        S_t = next(S for S in self.strides if S >= G + 1)
        need = max([self.lag_hi[b] - 1 for b in range(self.B) if self.gamma[b] > 0] + [2])
        S_c = 2 if need <= 2 else min(self.max_catchup, 1 << (need - 1).bit_length())
        return Bc, G, S_t, S_c

    def _advance_host(self, S_c):
        for b in range(self.B):
            lo, hi, g = self.lag_lo[b], self.lag_hi[b], self.gamma[b]
            if g == 0:
                lo, hi = lo + 1, hi + 1
            elif hi <= 2 or lo <= 2:
                lo, hi = 1, 2      # speculated (lag 1 or 2 after), or caught up from lag 3
            else:
                lo, hi = max(2, lo - S_c + 1), max(2, hi - S_c + 1)
            self.lag_lo[b], self.lag_hi[b] = lo, hi

    def _meta(self, Bc, S):
        key = (Bc, S)
        if key not in self._cu:
            self._cu[key] = torch.arange(Bc + 1, dtype=torch.int32, device=self.hist.device) * S
        return self._cu[key]

    def _rows0(self, Bc, S):
        key = (Bc, S)
        if key not in self._row0:
            self._row0[key] = torch.arange(Bc, dtype=torch.int32, device=self.hist.device) * S
        return self._row0[key]

    # ---- one speculative step -------------------------------------------------------------
    def _rows(self, model, kv, Bc, start, S, tokens, n_real, logits_out=None, keep_rows=None):
        """Forward S rows per sequence at positions start..start+S-1 over slots [0, Bc); rows
        j >= n_real[b] are padding (KV write skipped, seq_len = start + S as in the padded
        graph layout).  Positions, slots and seq_lens come from one coopt_row_slots launch."""
        pos, slots, seq_lens = self.ops.row_slots(kv, start, S, n_real)
        meta = (self._meta(Bc, S), seq_lens, S, self.max_len)
        return model.forward(self.ops, kv, tokens.reshape(-1), pos.reshape(-1), slots, meta,
                             logits_out=logits_out, keep_rows=keep_rows)

    @torch.inference_mode()
    def _step(self, Bc, G, S_t, S_c):
        T = self.T
        gm, Bcap = self.gmax, self.Bcap
        u_draft = self.u[: gm * Bcap].view(gm, Bcap)
        u_acc = self.u[gm * Bcap: 2 * gm * Bcap].view(Bcap, gm)
        u_res = self.u[2 * gm * Bcap:]
        vt, dt = self._vtok[S_t], self._dtok[S_t]
        lib, dev = _lib.load(), self.hist.device
        stream = _lib.stream_handle(dev)
        # the step's uniforms, each sequence's mode, and every row the draft and the verify run
        # (engine/engine.py:354-389, 414-417): one launch
        _lib.check(lib.coopt_spec_step_begin(
            _lib.ptr(self.u_table), self.u_table.shape[0], self.nu, _lib.ptr(self.u_ctr),
            _lib.ptr(self.u), _lib.ptr(self.live_dev), _lib.ptr(self.gamma_dev), _lib.ptr(self.n),
            _lib.ptr(self.dc), _lib.ptr(self.hist), self.hist.stride(0), self.max_len, Bc, G, S_c,
            S_t, _lib.ptr(self.gamma_eff), _lib.ptr(self._cu_start), _lib.ptr(self._cu_nreal),
            _lib.ptr(self._cu_tok), _lib.ptr(self._cu_keep), _lib.ptr(self._pr_start),
            _lib.ptr(self._pr_nreal), self._pr_start.stride(0), _lib.ptr(self._v_start),
            _lib.ptr(self._v_nreal), _lib.ptr(vt), _lib.ptr(self._dc_final), stream),
            "coopt_spec_step_begin")
        if G > 0:
            # draft catch-up over tokens[dc : dc + m] (stride S_c); only the row the first
            # proposal is drawn from goes through the logits projection
            self._rows(self.d, self.dkv, Bc, self._cu_start[:Bc], S_c, self._cu_tok[: Bc * S_c],
                       self._cu_nreal[:Bc], logits_out=self.draft_logits[:Bc, 0],
                       keep_rows=self._cu_keep[:Bc])
            self._sample(0, Bc, u_draft[0, :Bc])
            for i in range(1, G):
                self._rows(self.d, self.dkv, Bc, self._pr_start[i - 1, :Bc], 1, self.prop[i - 1, :Bc],
                           self._pr_nreal[i - 1, :Bc], logits_out=self.draft_logits[:Bc, i])
                self._sample(i, Bc, u_draft[i, :Bc])
        # target verify over [last token] + drafts (stride S_t; rows past gamma_eff + 1 padding)
        _lib.check(lib.coopt_spec_step_verify_tokens(
            _lib.ptr(self.prop), self.prop.stride(0), Bc, S_t, _lib.ptr(vt), _lib.ptr(dt), stream),
            "coopt_spec_step_verify_tokens")
        self._rows(self.t, self.tkv, Bc, self._v_start[:Bc], S_t, vt[:Bc], self._v_nreal[:Bc],
                   logits_out=self.target_logits[: Bc * S_t])
        res = AcceptResult(self._acc_len[:Bc], self._acc_tok[S_t][:Bc], self._margin[:Bc])
        res = self.ops.accept(self.target_logits[: Bc * S_t], self.draft_logits.view(Bcap * (self.smax - 1), -1),
                              dt[:Bc, : S_t - 1], T, u_acc[:Bc, : S_t - 1], u_res[:Bc],
                              out=res, gamma_per_seq=self.gamma_eff[:Bc],
                              target_row0=self._rows0(Bc, S_t), draft_row0=self._rows0(Bc, self.smax - 1))
        # append drafts[:k] + [token] to live histories; rollback is the length update
        # (engine/engine.py:444-446, 455, 463-470): one launch
        _lib.check(lib.coopt_spec_step_commit(
            _lib.ptr(self.live_dev), _lib.ptr(res.accepted_len), _lib.ptr(res.tokens), S_t,
            _lib.ptr(self.gamma_eff), _lib.ptr(self._dc_final), _lib.ptr(self.n), _lib.ptr(self.dc),
            _lib.ptr(self.hist), self.hist.stride(0), self.max_len, _lib.ptr(self.emitted),
            _lib.ptr(self.drafted), _lib.ptr(self.accepted), Bc, stream), "coopt_spec_step_commit")

    def _sample(self, i, Bc, u):
        """Draft token i of every slot, drawn from draft_logits[:, i] into prop[i] in place."""
        out = AcceptResult(self._s_len[:Bc], self.prop[i, :Bc].view(Bc, 1), self._s_margin[:Bc])
        self.ops.sample(self.draft_logits[:Bc, i], u, self.T, out=out)

    def _check_room(self):
        """Raises before a step the history, the block tables or the uniform table cannot
        hold: the kernels would otherwise drop the history writes past max_len and reuse
        uniform rows (the row index wraps)."""
        if self.steps_run >= self.max_steps:
            raise RuntimeError(f"max_steps ({self.max_steps}) steps have run; the decoder's "
                               "history and block tables are sized for that many")
        if self.u_used >= self.u_table.shape[0]:
            raise RuntimeError(f"the uniform table's {self.u_table.shape[0]} rows are used up; "
                               "call set_uniforms with a new table")

    def step(self):
        """One eager step (same device work as a graph replay, launched from the host)."""
        self._check_room()
        key = self.bucket()
        self._step(*key)
        self._finish(key)

    def _finish(self, key):
        Bc, S_t = key[0], key[2]
        self.res = AcceptResult(self._acc_len[:Bc], self._acc_tok[S_t][:Bc], self._margin[:Bc])
        self.last_key = key
        self.steps_run += 1
        self.u_used += 1
        self._advance_host(key[3])

    def capture(self, key=None):
        """Records the step of bucket `key` = (Bc, G, S_t, 2) (default: the next step's) into
        a HIP graph.  Side-effect free: the warm-up pass and the recording run with every
        slot a dummy, and the uniform row counter is restored."""
        key = self.bucket() if key is None else key
        if key[3] != 2:
            raise ValueError("graphs are captured with the stride-2 draft catch-up")
        dev = self.hist.device
        ctr = self.u_ctr.clone()
        self.live_dev.zero_()
        self.gamma_dev.zero_()
        if self.pool is None:
            self.pool = torch.cuda.graph_pool_handle()
        s = torch.cuda.Stream(device=dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            self._step(*key)
        torch.cuda.current_stream(dev).wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=self.pool):
            self._step(*key)
        self.graphs[key] = g
        self.u_ctr.copy_(ctr)
        self._sync_live()
        torch.cuda.synchronize(dev)
        return key

    def replay(self):
        """One step through the captured graph of its bucket (captured on first use); steps
        whose draft catch-up needs more than 2 rows run eagerly."""
        self._check_room()
        key = self.bucket()
        if key[3] != 2:
            return self.step()
        if key not in self.graphs:
            self.capture(key)
        self.graphs[key].replay()
        self._finish(key)

    # ---- views for inspection ------------------------------------------------------------
    def state(self):
        """Host copy of the live sequences' (tokens, num_computed = len - 1, draft_computed)."""
        n, dc, hist = self.n.cpu().tolist(), self.dc.cpu().tolist(), self.hist.cpu()
        return [(hist[b, : n[b]].tolist(), n[b] - 1, dc[b]) for b in range(self.B)]
