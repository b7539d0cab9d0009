"""CPU kernels for the speculative step, built from the oracle.  TEST INFRASTRUCTURE ONLY:
bench.py's cpu_baseline leg times SpecDecoder.step with these ops on the host cores (the
reference's path restated on the CPU); the product never imports this module.

  write   KV write with INT8 quantise-on-write      oracle.codec / oracle.paged.kv_write*
  attend  paged causal GQA attention, fp32 torch     oracle.paged.attention_seq (same closed
          math on the dequantised (bf16) cache       form, in fp32 torch for speed)
  sample  inverse-CDF draw from softmax(logits/T)    oracle.accept.sample
  accept  rejection sampling with explicit uniforms  oracle.accept.accept_batch
  row_slots  positions / slots / seq_lens of a padded  oracle.paged.slot_mapping's formula
          row batch                                  (engine/block_manager.py:216-220)
"""
import numpy as np
import torch

from . import accept as OA
from . import codec as OC


class OracleOps:
    """torch-CPU / oracle versions of every stage HipOps runs on the GPU."""

    def rms_norm(self, x, residual, w, eps):
        # engine/model.py:85-89 (fused add first when a residual is given, :236/:249/:254)
        if residual is not None:
            residual.copy_(residual + x)
            x = residual
        xf = x.float()
        return w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)

    def rope(self, q, k, pos, cos, sin):
        # engine/model.py:92-94, 199-200 (neox half split)
        c, s = cos[pos].unsqueeze(1), sin[pos].unsqueeze(1)
        for x in (q, k):
            x1, x2 = x.chunk(2, dim=-1)
            x.copy_(x * c + torch.cat((-x2, x1), dim=-1) * s)

    def row_slots(self, kv, start, S, n_real):
        # engine/block_manager.py:216-220 (slot = table[p // bs] * bs + p % bs) for rows
        # start[b] + j; padding rows (j >= n_real[b]) and positions past the table get -1
        bs = kv.block_size
        pos = start.unsqueeze(1) + torch.arange(S, dtype=torch.int64)
        blk = pos // bs
        width = kv.block_table.shape[1]
        ok = (blk >= 0) & (blk < width)
        if n_real is not None:
            ok &= torch.arange(S).unsqueeze(0) < n_real.unsqueeze(1)
        table = kv.block_table.long()
        slots = torch.gather(table, 1, blk.clamp(0, width - 1)) * bs + pos % bs
        slots = torch.where(ok, slots, torch.full_like(slots, -1)).reshape(-1)
        return pos, slots, (start + S).to(torch.int32)

    def linear_silu(self, x, w):
        # engine/model.py:250-252: silu_and_mul(F.linear(h, gate_up))
        return self.silu_mul(self.linear(x, w))

    def silu_mul(self, gate_up):
        gate, up = gate_up.chunk(2, dim=-1)
        return torch.nn.functional.silu(gate) * up

    def qkv_epilogue(self, kv, layer, qkv, pos, cos, sin, slots, H, Hkv, D):
        # engine/model.py:238-243: split, RoPE on q and k, K/V into the paged cache
        T = qkv.shape[0]
        q = qkv[:, : H * D].view(T, H, D)
        k = qkv[:, H * D: (H + Hkv) * D].view(T, Hkv, D)
        v = qkv[:, (H + Hkv) * D:].view(T, Hkv, D)
        self.rope(q, k, pos, cos, sin)
        self.write(kv, layer, k, v, slots)
        return q

    def linear(self, x, w, out=None, defer_reduce=False):
        # the projections, F.linear without bias (engine/model.py:238, 248, 250, 253)
        if out is not None:
            return torch.matmul(x, w.t(), out=out)
        return torch.nn.functional.linear(x, w)

    def write(self, kv, layer, k, v, slots):
        kc, vc, ks, vs = kv.layers[layer]
        slots = slots.cpu()
        ok = slots >= 0
        blk, off = slots[ok] // kv.block_size, slots[ok] % kv.block_size
        if kv.kv_dtype == "int8":
            for x, cache, scale in ((k, kc, ks), (v, vc, vs)):
                q, s = OC.quantize(x[ok].float().numpy(), 8)
                cache[blk, off] = torch.from_numpy(q)
                scale[blk, off] = torch.from_numpy(s)
        else:
            kc[blk, off] = k[ok]
            vc[blk, off] = v[ok]

    def attend(self, kv, layer, q, meta, scale):
        kc, vc, ks, vs = kv.layers[layer]
        cu, seq_lens, S, _ = meta
        T, H, D = q.shape
        Hkv = kc.shape[2]
        G = H // Hkv
        out = torch.empty_like(q)
        bs = kv.block_size
        for b in range(seq_lens.numel()):
            q0, q1, L = int(cu[b]), int(cu[b + 1]), int(seq_lens[b])
            n = q1 - q0
            pos = torch.arange(L)
            blk, off = kv.block_table[b].long()[pos // bs], pos % bs
            if kv.kv_dtype == "int8":
                K = (kc[blk, off].float() * ks[blk, off].float().unsqueeze(-1)).to(torch.bfloat16)
                V = (vc[blk, off].float() * vs[blk, off].float().unsqueeze(-1)).to(torch.bfloat16)
            else:
                K, V = kc[blk, off], vc[blk, off]
            Kh = K.float().permute(1, 2, 0)                      # [Hkv, D, L]
            Vh = V.float().permute(1, 0, 2)                      # [Hkv, L, D]
            Q = q[q0:q1].float().view(n, Hkv, G, D).permute(1, 0, 2, 3).reshape(Hkv, n * G, D)
            s = torch.matmul(Q, Kh) * scale                      # [Hkv, n*G, L]
            lim = torch.repeat_interleave(L - n + torch.arange(n), G)
            s = s.masked_fill(torch.arange(L)[None, None, :] > lim[None, :, None], float("-inf"))
            p = torch.softmax(s, -1)
            o = torch.matmul(p, Vh)                              # [Hkv, n*G, D]
            out[q0:q1] = o.view(Hkv, n, G, D).permute(1, 0, 2, 3).reshape(n, H, D).to(q.dtype)
        return out

    def sample(self, logits, u, temperature, out=None):
        toks, _ = OA.sample(logits.float().numpy(), temperature, u.numpy())
        return torch.from_numpy(np.asarray(toks, np.int32))

    def accept(self, target_logits, draft_logits, draft_tokens, temperature, u_acc, u_res,
               out=None):
        acc, toks, marg = OA.accept_batch(target_logits.float().numpy(),
                                          draft_logits.float().numpy(), draft_tokens.numpy(),
                                          temperature, u_acc.numpy(), u_res.numpy())
        res = out
        res.accepted_len.copy_(torch.from_numpy(acc))
        res.tokens.copy_(torch.from_numpy(toks))
        res.margin.copy_(torch.from_numpy(marg.astype(np.float32)))
        return res
