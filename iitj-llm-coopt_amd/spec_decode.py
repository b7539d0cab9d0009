"""Speculative acceptance on gfx950: the batched fused accept-sample kernel behind the
reference's spec_decode call surface.

Reference (mohsinmubarak/iitj-llm-coopt):
  sample(logits, temperature, generator)                    engine/spec_decode.py:12-17
  verify(target_logits, draft_tokens, draft_probs, T, gen)  engine/spec_decode.py:20-49
  batched greedy accept / per-sequence verify loop          engine/engine.py:421-446

The kernel takes its random draws explicitly: u_accept[b, i] decides draft i of sequence b
(accepted iff u < min(1, p/q)), and u_resample[b] draws the emitted token by inverse CDF
(the smallest j with cumsum(w)[j] > u * sum(w)) from the normalised max(0, p_k - q_k)
residual (p_k if it sums to 0), or from p_g when all g drafts are accepted.  Given the same
uniforms the accepted lengths and tokens are deterministic.  When the reference-compatible
sample()/verify() are called with a torch.Generator instead, the uniforms are drawn from it;
the output distribution is the target's (the rejection sampler is lossless), but the exact
tokens differ from the reference's torch.multinomial stream.
"""
from dataclasses import dataclass

import torch

from . import _lib

__all__ = ["AcceptResult", "accept", "sample", "verify", "softmax"]

_WS = _lib.WorkspaceCache()


@dataclass
class AcceptResult:
    accepted_len: torch.Tensor  # [B] int32: k, the number of accepted drafts
    tokens: torch.Tensor        # [B, gamma_max + 1] int32: drafts[:k] + [emitted], then -1
    margin: torch.Tensor        # [B] fp32: distance of the deciding uniforms to their boundary

    def to_lists(self):
        """Per-sequence token lists, as verify() returns them (one device->host copy)."""
        acc = self.accepted_len.tolist()
        toks = self.tokens.tolist()
        return [row[: k + 1] for row, k in zip(toks, acc)]


def _rows(x):
    if x is None:
        return None, 0
    if x.dim() == 3:
        x = x.reshape(-1, x.shape[-1]) if x.is_contiguous() else x.contiguous().view(-1, x.shape[-1])
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("logits/probability rows must be [rows, V] with contiguous V")
    return x, x.stride(0)


def accept(target_logits, draft, draft_tokens, temperature, u_accept=None, u_resample=None,
           draft_is_probs=False, gamma_per_seq=None, target_row0=None, draft_row0=None,
           out=None, workspace=None) -> AcceptResult:
    """Batched acceptance for B sequences with up to gamma_max drafts each.

    target_logits [B, gamma_max+1, V] (or [rows, V] with target_row0[b] = first row of b),
    fp32 or bf16; draft [B, gamma_max, V] draft logits (softmax(draft/T) is formed in the
    kernel) or, with draft_is_probs, fp32 draft probabilities; draft_tokens [B, gamma_max].
    temperature <= 0 selects the greedy rule (argmax, accept while equal).
    out / workspace: optional preallocated AcceptResult and uint8 scratch buffer (neither
    allocates then, so the call can be recorded into a HIP graph).  workspace="static" runs
    coopt_accept_sample_noalloc, whose workspace is the library's own per-GPU device array
    (sizes up to coopt_accept_sample_noalloc_max_bytes(); overlapping calls on one GPU race).
    """
    tgt, tstride = _rows(target_logits)
    _lib.require_cuda(tgt, draft_tokens)
    dev = tgt.device
    if tgt.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("target logits must be fp32 or bf16")
    V = tgt.shape[1]
    dtok = draft_tokens.to(device=dev, dtype=torch.int32).contiguous()
    if dtok.dim() != 2:
        raise ValueError("draft_tokens must be [B, gamma_max]")
    B, gmax = dtok.shape
    greedy = not (temperature > 0)
    drf, dstride = (None, 0) if (greedy or gmax == 0) else _rows(draft)
    if drf is not None:
        _lib.require_cuda(drf)
        if draft_is_probs and drf.dtype != torch.float32:
            raise ValueError("draft probabilities must be fp32")
        if not draft_is_probs and drf.dtype != tgt.dtype:
            raise ValueError("draft logits must have the target logits' dtype")
        if drf.shape[1] != V:
            raise ValueError("draft rows must have the target's vocabulary size")
    if target_row0 is None and tgt.shape[0] < B * (gmax + 1):
        raise ValueError(f"target logits have {tgt.shape[0]} rows, need B*(gamma_max+1)")
    if drf is not None and draft_row0 is None and drf.shape[0] < B * gmax:
        raise ValueError(f"draft rows {drf.shape[0]} < B*gamma_max")
    if not greedy:
        if u_resample is None or (gmax > 0 and u_accept is None):
            raise ValueError("sampling needs u_accept [B, gamma_max] and u_resample [B]")
    ua = None if u_accept is None else u_accept.to(device=dev, dtype=torch.float32).contiguous()
    ur = None if u_resample is None else u_resample.to(device=dev, dtype=torch.float32).contiguous()
    if ua is not None and ua.numel() < B * gmax:
        raise ValueError("u_accept must have B*gamma_max entries")
    if ur is not None and ur.numel() < B:
        raise ValueError("u_resample must have B entries")

    def i32(x):
        if x is None:
            return None
        x = torch.as_tensor(x)
        return x.to(device=dev, dtype=torch.int32).contiguous()

    # Row offsets given as host data are bounds-checked here (no device sync needed); device
    # tensors are the caller's responsibility, like the cu_seqlens of the attention call.
    for row0, rows, span, name in ((target_row0, tgt.shape[0], gmax + 1, "target_row0"),
                                   (draft_row0, 0 if drf is None else drf.shape[0], gmax,
                                    "draft_row0")):
        if row0 is not None and not (isinstance(row0, torch.Tensor) and row0.is_cuda):
            r = torch.as_tensor(row0).to(torch.int64)
            g = torch.full_like(r, gmax) if gamma_per_seq is None else \
                torch.as_tensor(gamma_per_seq).cpu().to(torch.int64)
            extent = g + (1 if span == gmax + 1 else 0)
            if r.numel() != B or (r < 0).any() or ((r + extent) > rows).any():
                raise ValueError(f"{name} points outside the {rows} rows given")
    gam, t0, d0 = i32(gamma_per_seq), i32(target_row0), i32(draft_row0)
    if out is None:
        out = AcceptResult(torch.empty(B, dtype=torch.int32, device=dev),
                           torch.empty((B, gmax + 1), dtype=torch.int32, device=dev),
                           torch.empty(B, dtype=torch.float32, device=dev))
    lib = _lib.load()
    if isinstance(workspace, str):
        if workspace != "static":
            raise ValueError('workspace must be a tensor, None or "static"')
        _lib.check(lib.coopt_accept_sample_noalloc(
            _lib.dt_code(tgt.dtype), _lib.ptr(tgt), tstride, _lib.ptr(t0),
            1 if draft_is_probs else 0, _lib.ptr(drf), dstride, _lib.ptr(d0),
            _lib.ptr(dtok), _lib.ptr(gam), _lib.ptr(ua), _lib.ptr(ur), float(temperature),
            B, gmax, V, _lib.ptr(out.accepted_len), _lib.ptr(out.tokens), _lib.ptr(out.margin),
            _lib.stream_handle(dev)), "coopt_accept_sample_noalloc")
        return out
    need = int(lib.coopt_accept_sample_workspace(B, gmax, V))
    if workspace is None:
        ws = _WS.get(need, dev)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} bytes, "
                         f"{need} needed")
    else:
        ws = workspace
    _lib.check(lib.coopt_accept_sample(
        _lib.dt_code(tgt.dtype), _lib.ptr(tgt), tstride, _lib.ptr(t0),
        1 if draft_is_probs else 0, _lib.ptr(drf), dstride, _lib.ptr(d0),
        _lib.ptr(dtok), _lib.ptr(gam), _lib.ptr(ua), _lib.ptr(ur), float(temperature),
        B, gmax, V, _lib.ptr(out.accepted_len), _lib.ptr(out.tokens), _lib.ptr(out.margin),
        _lib.ptr(ws), ws.numel() * ws.element_size(), _lib.stream_handle(dev)),
        "coopt_accept_sample")
    return out


def softmax(logits, temperature: float):
    """softmax(logits * (1/T)) over the last dim, fp32 [N, V]."""
    x, stride = _rows(logits)
    _lib.require_cuda(x)
    probs = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    lib = _lib.load()
    _lib.check(lib.coopt_softmax(_lib.dt_code(x.dtype), _lib.ptr(x), stride, x.shape[0],
                                 x.shape[1], float(temperature), _lib.ptr(probs), x.shape[1],
                                 _lib.stream_handle(x.device)), "coopt_softmax")
    return probs


def sample(logits: torch.Tensor, temperature: float, generator=None, uniforms=None,
           return_probs=True):
    """logits [N, V] -> (tokens [N] int64, probs [N, V] fp32 or None when greedy).

    Greedy (T <= 0): argmax, first index on ties.  Otherwise one inverse-CDF draw per row
    from softmax(logits / T) with `uniforms` [N] (or uniforms drawn from `generator`).
    """
    x, _ = _rows(logits)
    _lib.require_cuda(x)
    N = x.shape[0]
    empty = torch.empty((N, 0), dtype=torch.int32, device=x.device)
    if temperature <= 0:
        res = accept(x, None, empty, 0.0)
        return res.tokens[:, 0].long(), None
    if uniforms is None:
        uniforms = torch.rand(N, generator=generator, device=x.device)
    if not return_probs:
        res = accept(x, None, empty, temperature, u_resample=uniforms)
        return res.tokens[:, 0].long(), None
    # tokens and probabilities from one draw (coopt_sample: the row statistics, then one
    # launch that writes the probabilities and draws from them)
    lib = _lib.load()
    V = x.shape[1]
    need = int(lib.coopt_accept_sample_workspace(N, 0, V))
    ws = _WS.get(need, x.device)
    u = uniforms.to(device=x.device, dtype=torch.float32).contiguous()
    if u.numel() < N:
        raise ValueError("uniforms must have one entry per row")
    tokens = torch.empty(N, dtype=torch.int32, device=x.device)
    probs = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    _lib.check(lib.coopt_sample(_lib.dt_code(x.dtype), _lib.ptr(x), x.stride(0), N, V,
                                float(temperature), _lib.ptr(u), _lib.ptr(tokens), None,
                                _lib.ptr(probs), V, _lib.ptr(ws), ws.numel() * ws.element_size(),
                                _lib.stream_handle(x.device)), "coopt_sample")
    return tokens.long(), probs


def verify(target_logits: torch.Tensor, draft_tokens, draft_probs, temperature: float,
           generator=None, uniforms=None) -> list:
    """Rejection sampling for one sequence (engine/spec_decode.py:20-49 signature).

    target_logits [g+1, V]; draft_tokens: g ints; draft_probs [g, V] fp32 (None if greedy).
    uniforms: optional fp32 [g+1] = (u_accept..., u_resample); drawn from `generator` if None.
    Returns the accepted draft prefix plus the target's correction or bonus token.
    """
    _lib.require_cuda(target_logits)
    dev = target_logits.device
    g = len(draft_tokens)
    dt = torch.tensor([list(draft_tokens)], dtype=torch.int32, device=dev).view(1, g)
    tl = target_logits.float() if target_logits.dtype not in (torch.float32, torch.bfloat16) \
        else target_logits
    if temperature <= 0:
        return accept(tl.view(1, g + 1, -1), None, dt, 0.0).to_lists()[0]
    if uniforms is None:
        uniforms = torch.rand(g + 1, generator=generator, device=dev)
    uniforms = uniforms.to(device=dev, dtype=torch.float32).view(-1)
    q = None if g == 0 else draft_probs.to(device=dev, dtype=torch.float32).reshape(g, -1)
    res = accept(tl.reshape(g + 1, -1), q, dt, temperature, u_accept=uniforms[:g].view(1, g),
                 u_resample=uniforms[g:g + 1], draft_is_probs=True)
    return res.to_lists()[0]
