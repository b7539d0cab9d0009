"""Fused elementwise stages of the Llama forward around the verify path, on gfx950 kernels.

Counterparts of the vLLM ops the reference's forward calls (engine/model.py:234-254):
  rms_norm(x, weight, eps, residual=None, out=None)   _ops.rms_norm / _ops.fused_add_rms_norm
  rope_(q, k, positions, cos, sin)                     _ops.rotary_embedding (neox, in place)
  silu_and_mul(gate_up, out=None)                      torch.ops._C.silu_and_mul
"""
import torch

from . import _lib

__all__ = ["rms_norm", "rope_", "silu_and_mul"]


def _bf16_rows(t, name):
    if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
        raise ValueError(f"{name} must be bf16 with a contiguous last dimension")


def rms_norm(x, weight, eps, residual=None, out=None):
    """out = rmsnorm(x) * weight; with `residual`, first residual += x in place (fused add)."""
    _lib.require_cuda(x, weight, residual, out)
    for t, n in ((x, "x"), (weight, "weight")):
        _bf16_rows(t, n)
    x2 = x.reshape(-1, x.shape[-1])
    if not x2.is_contiguous():
        raise ValueError("x must be contiguous")
    if residual is not None and (residual.shape != x.shape or not residual.is_contiguous()):
        raise ValueError("residual must be contiguous with x's shape")
    if out is None:
        out = torch.empty_like(x)
    _lib.check(_lib.load().coopt_rms_norm(_lib.ptr(x), _lib.ptr(residual), _lib.ptr(weight),
                                          _lib.ptr(out), x2.shape[0], x2.shape[1], float(eps),
                                          _lib.stream_handle(x.device)), "coopt_rms_norm")
    return out


def rope_(q, k, positions, cos, sin):
    """In-place neox rotary embedding of q [T, Hq, D] and k [T, Hkv, D] (views allowed)."""
    _lib.require_cuda(q, k, positions, cos, sin)
    for t, n in ((q, "q"), (k, "k"), (cos, "cos"), (sin, "sin")):
        _bf16_rows(t, n)
    T, Hq, D = q.shape
    if k.shape[0] != T or k.shape[2] != D or positions.dtype != torch.int64 or positions.numel() != T:
        raise ValueError("q/k/positions shapes disagree")
    if cos.shape != sin.shape or cos.stride() != sin.stride() or cos.shape[1] < D // 2:
        raise ValueError("cos/sin tables must be [max_pos, >= D/2] alike")
    positions = positions.contiguous()
    _lib.check(_lib.load().coopt_rope(_lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k),
                                      k.stride(0), k.stride(1), _lib.ptr(positions), _lib.ptr(cos),
                                      _lib.ptr(sin), cos.stride(0), cos.shape[0], T, Hq, k.shape[1],
                                      D, _lib.stream_handle(q.device)), "coopt_rope")
    return q, k


def silu_and_mul(gate_up, out=None):
    """[T, 2F] -> [T, F]: silu(gate) * up."""
    _lib.require_cuda(gate_up, out)
    _bf16_rows(gate_up, "gate_up")
    if not gate_up.is_contiguous():
        raise ValueError("gate_up must be contiguous")
    T, F2 = gate_up.shape
    if out is None:
        out = torch.empty((T, F2 // 2), dtype=gate_up.dtype, device=gate_up.device)
    _lib.check(_lib.load().coopt_silu_mul(_lib.ptr(gate_up), _lib.ptr(out), T, F2 // 2,
                                          _lib.stream_handle(gate_up.device)), "coopt_silu_mul")
    return out
