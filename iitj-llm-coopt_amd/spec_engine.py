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
from .attention import paged_attention, workspace_bytes
from .batch import row_slots
from .fused import (linear, linear_silu, pack_gate_up_weight, pack_linear_weight, rms_norm, rope_,
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

    def forward(self, ops, kv, ids, pos, slots, meta, logits_out=None):
        """ids/pos/slots [T]; meta: attention metadata for ops.attend; returns logits [T, V].

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
            # qkv projection, RoPE and the KV write: split-K partials straight into one
            # epilogue launch that writes q and the paged cache (engine/model.py:238-243)
            qkv = ops.linear(h, L["qkv"], defer_reduce=True)
            q = ops.qkv_epilogue(kv, li, qkv, pos, self.cos, self.sin, slots, H, Hkv, D)
            attn = ops.attend(kv, li, q, meta, self.scale)
            # gate_up + SiLU·mul is one launch at draft row counts (linear_silu); o, down and
            # otherwise gate_up feed only the fused add + norm or SiLU, which reduce their
            # split-K partials as they read them
            o = ops.linear(attn.reshape(T, H * D), L["o"], defer_reduce=True)
            h = ops.rms_norm(o, x, L["ln2"], s.eps)
            d = ops.linear(ops.linear_silu(h, L["gate_up"]), L["down"], defer_reduce=True)
        h = ops.rms_norm(d, x, self.norm, s.eps)
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
    """The gfx950 kernels behind the step, with preallocated workspaces (capture-safe)."""

    def __init__(self, device):
        self.device = torch.device(device)
        self._ws = {}

    def workspace(self, key, nbytes):
        buf = self._ws.get(key)
        if buf is None or buf.numel() < nbytes:
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
        return paged_attention(q, kc, vc, cu, seq_lens, kv.block_table, S, max_k, scale, ks, vs,
                               workspace=ws)

    def sample(self, logits, u, temperature, out=None):
        """One token per row: inverse-CDF draw from softmax(logits / T) (argmax if T <= 0)."""
        N, V = logits.shape
        empty = self._empty_tokens(N)
        ws = self.workspace(("acc", 0), _lib.load().coopt_accept_sample_workspace(N, 0, V))
        res = accept(logits, None, empty, temperature, u_resample=u, workspace=ws, out=out)
        return res.tokens[:, 0]

    def accept(self, target_logits, draft_logits, draft_tokens, temperature, u_acc, u_res,
               out=None):
        B, g = draft_tokens.shape
        V = target_logits.shape[-1]
        ws = self.workspace(("acc", 1), _lib.load().coopt_accept_sample_workspace(B, g, V))
        return accept(target_logits, draft_logits, draft_tokens, temperature, u_acc, u_res,
                      workspace=ws, out=out)

    def _empty_tokens(self, n):
        key = ("empty", n)
        t = self._ws.get(key)
        if t is None:
            t = torch.empty((n, 0), dtype=torch.int32, device=self.device)
            self._ws[key] = t
        return t


class SpecDecoder:
    """Batch of B sequences decoding speculatively with gamma drafts per step."""

    def __init__(self, target: RandomLlama, draft: RandomLlama, batch: int, gamma: int,
                 prompt_len: int, max_steps: int, ops=None, target_kv="int8", draft_kv="auto",
                 temperature=1.0, block_size=16, seed=0):
        dev = target.device
        self.t, self.d, self.B, self.g = target, draft, batch, gamma
        self.P, self.T = prompt_len, temperature
        self.ops = ops or HipOps(dev)
        self.max_len = prompt_len + 1 + max_steps * (gamma + 1) + gamma + 2
        self.tkv = PagedKV(target.s, batch, self.max_len, target_kv, dev, block_size, seed)
        self.dkv = PagedKV(draft.s, batch, self.max_len, draft_kv, dev, block_size, seed + 1)
        self.hist = torch.zeros((batch, self.max_len), dtype=torch.int64, device=dev)
        self.n = torch.zeros(batch, dtype=torch.int64, device=dev)    # tokens so far
        self.dc = torch.zeros(batch, dtype=torch.int64, device=dev)   # draft KV length
        self.emitted = torch.zeros((), dtype=torch.int64, device=dev)
        self.drafted = torch.zeros((), dtype=torch.int64, device=dev)
        self.accepted = torch.zeros((), dtype=torch.int64, device=dev)
        V = target.s.vocab
        self.draft_logits = torch.empty((batch, gamma, V), dtype=torch.bfloat16, device=dev)
        self.target_logits = torch.empty((batch * (gamma + 1), V), dtype=torch.bfloat16,
                                         device=dev)
        self.draft_tok = torch.zeros((batch, gamma), dtype=torch.int32, device=dev)
        self.u = torch.zeros(batch * (2 * gamma + 1), dtype=torch.float32, device=dev)
        self.res = AcceptResult(torch.empty(batch, dtype=torch.int32, device=dev),
                                torch.empty((batch, gamma + 1), dtype=torch.int32, device=dev),
                                torch.empty(batch, dtype=torch.float32, device=dev))
        self.cu = {S: torch.arange(batch + 1, dtype=torch.int32, device=dev) * S
                   for S in (1, 2, gamma + 1)}
        self.ar = {S: torch.arange(S, dtype=torch.int64, device=dev) for S in (1, 2, gamma + 1)}
        self.graph = None

    # ---- prefill (not part of the timed step) -------------------------------------------
    @torch.inference_mode()
    def prefill(self, prompts: torch.Tensor, u_first: torch.Tensor):
        """prompts [B, P] int64.  Runs both models over the prompt (attention over the prompt
        in fp32 SDPA, KV written through the paged write kernel), samples the first token
        from the target and sets num_computed = P (engine/engine.py:427-436)."""
        B, P = prompts.shape
        self.hist[:, :P] = prompts
        pos = torch.arange(P, device=self.hist.device).expand(B, P)
        for model, kv in ((self.t, self.tkv), (self.d, self.dkv)):
            logits = self._prefill_model(model, kv, prompts, pos)
            if model is self.t:
                first = self.ops.sample(logits, u_first, self.T)
        self.hist[:, P] = first.long()
        self.n.fill_(P + 1)
        self.dc.fill_(P)
        torch.cuda.synchronize(self.hist.device)

    def _prefill_model(self, model, kv, ids, pos):
        s = model.s
        B, P = ids.shape
        H, Hkv, D = s.heads, s.kv_heads, s.head_dim
        T = B * P
        flat_pos = pos.reshape(-1).contiguous()
        slots = kv.slots(pos)
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

    # ---- one speculative step -------------------------------------------------------------
    def _rows(self, model, kv, start, S, tokens, n_real, logits_out=None):
        """Forward S rows per sequence at positions start..start+S-1; rows j >= n_real[b] are
        padding (KV write skipped, seq_len = start + S as in the padded graph layout).
        Positions, slots and seq_lens come from one coopt_row_slots launch."""
        pos, slots, seq_lens = self.ops.row_slots(kv, start, S, n_real)
        meta = (self.cu[S], seq_lens, S, self.max_len)
        return model.forward(self.ops, kv, tokens.reshape(-1), pos.reshape(-1), slots, meta,
                             logits_out=logits_out)

    @torch.inference_mode()
    def step(self):
        B, g, T = self.B, self.g, self.T
        u = torch.rand(self.u.shape, device=self.u.device, out=self.u)
        u_draft, u_acc, u_res = u[: B * g].view(g, B), u[B * g: 2 * B * g].view(B, g), u[2 * B * g:]
        n, dc = self.n, self.dc
        lag = n - dc                                                 # 1 or 2
        # draft catch-up over tokens[dc:n] as a stride-2 padded batch
        idx = (dc.unsqueeze(1) + self.ar[2]).clamp(max=self.max_len - 1)
        toks2 = torch.gather(self.hist, 1, idx)
        logits = self._rows(self.d, self.dkv, dc, 2, toks2, lag).view(B, 2, -1)
        last = torch.gather(logits, 1, (lag - 1).view(B, 1, 1).expand(B, 1, logits.shape[-1]))
        self.draft_logits[:, 0] = last[:, 0]
        tok = self.ops.sample(self.draft_logits[:, 0], u_draft[0], T)
        self.draft_tok[:, 0] = tok
        for i in range(1, g):
            start = n - 1 + i
            self._rows(self.d, self.dkv, start, 1, self.draft_tok[:, i - 1].long(), None,
                       logits_out=self.draft_logits[:, i])
            self.draft_tok[:, i] = self.ops.sample(self.draft_logits[:, i], u_draft[i], T)
        # target verify over [last token] + drafts
        vt = torch.cat([torch.gather(self.hist, 1, (n - 1).unsqueeze(1)), self.draft_tok.long()], 1)
        self._rows(self.t, self.tkv, n - 1, g + 1, vt, None, logits_out=self.target_logits)
        res = self.ops.accept(self.target_logits.view(B, g + 1, -1), self.draft_logits,
                              self.draft_tok, T, u_acc, u_res, out=self.res)
        acc = res.accepted_len.long()
        # append drafts[:k] + [token] to the history; rollback is the length update
        pos = (n.unsqueeze(1) + self.ar[g + 1]).clamp(max=self.max_len - 1)
        keep = self.ar[g + 1].unsqueeze(0) <= acc.unsqueeze(1)
        old = torch.gather(self.hist, 1, pos)
        self.hist.scatter_(1, pos, torch.where(keep, res.tokens.long(), old))
        new_n = n + acc + 1
        self.dc.copy_(torch.minimum(n + g - 1, new_n - 1))
        self.n.copy_(new_n)
        self.emitted += (acc + 1).sum()
        self.drafted += B * g
        self.accepted += acc.sum()

    def to(self, device, ops):
        """A copy of the decoder's full state (weights, caches, history) on another device,
        stepping through `ops` -- e.g. to time the same step on the host cores."""
        other = object.__new__(SpecDecoder)
        other.__dict__.update(self.__dict__)
        other.t, other.d = self.t.to(device), self.d.to(device)
        other.tkv, other.dkv = self.tkv.to(device), self.dkv.to(device)
        other.ops = ops
        for name in ("hist", "n", "dc", "emitted", "drafted", "accepted", "draft_logits",
                     "target_logits", "draft_tok", "u"):
            setattr(other, name, getattr(self, name).to(device))
        other.res = AcceptResult(*(t.to(device) for t in (self.res.accepted_len,
                                                            self.res.tokens, self.res.margin)))
        other.cu = {k: v.to(device) for k, v in self.cu.items()}
        other.ar = {k: v.to(device) for k, v in self.ar.items()}
        other.graph = None
        return other

    def capture(self):
        """Records one step into a HIP graph (call after a warm-up step)."""
        s = torch.cuda.Stream(device=self.hist.device)
        s.wait_stream(torch.cuda.current_stream(self.hist.device))
        with torch.cuda.stream(s):
            self.step()
        torch.cuda.current_stream(self.hist.device).wait_stream(s)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.step()

    def replay(self):
        self.graph.replay()
