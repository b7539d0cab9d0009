"""Symmetric absmax INT8/INT4 codec, restating engine/kv_tier_manager.py:21-41.

Reference (kv_tier_manager.py:21-31):
    scale = x.abs().amax(-1, keepdim=True).float().clamp_min(1e-8) / qmax
    q = torch.round(x.float() / scale).clamp(-qmax, qmax).to(torch.int8)
    (INT4: q + 8, pack even -> low nibble, odd -> high nibble)
    return q, scale.squeeze(-1).to(torch.float16)
The reference runs it on GPU tensors (swap_out, kv_tier_manager.py:99; eval/quality.py:51),
where torch evaluates "tensor / python scalar" as tensor * fp32(1 / scalar).  mode="device"
(default) restates that; mode="cpu" is torch-CPU's true division.  Everything else is the
same in both: fp32 clamp at fp32(1e-8), IEEE fp32 x / scale, round half to even, fp16 scale
with round-to-nearest-even.

Pinned by: the closed form itself (numpy float32 arithmetic is IEEE), the special cases
tested in tests/test_oracle_codec.py (|x| = amax -> +-127, exact .5 ties to even, all-zero
vectors -> scale 0 in fp16 and codes 0, x20 outliers), agreement with a literal torch-CPU
restatement of the reference lines in mode="cpu", and dequantize(quantize(x)) error bounds.
"""
import numpy as np

QMAX = {8: 127, 4: 7}


def quantize(x, bits: int, mode: str = "device"):
    """x: float array [..., D] (values of bf16/fp16/fp32) -> (codes, fp16 scales [...]).

    bits 8: int8 codes [..., D]; bits 4: uint8 [..., D/2] packed nibbles.
    """
    qmax = QMAX[bits]
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=-1) if x.shape[-1] else np.zeros(x.shape[:-1], np.float32)
    amax = np.maximum(amax.astype(np.float32), np.float32(1e-8))
    if mode == "device":
        s32 = amax * (np.float32(1.0) / np.float32(qmax))
    elif mode == "cpu":
        s32 = amax / np.float32(qmax)
    else:
        raise ValueError(mode)
    s32 = s32.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(x / s32[..., None])
    q = np.clip(r, -qmax, qmax).astype(np.int8)
    if bits == 4:
        u = (q.astype(np.int16) + 8).astype(np.uint8)
        q = (u[..., 0::2] | (u[..., 1::2] << 4)).astype(np.uint8)
    return q, s32.astype(np.float16)


def dequantize(q, scale, bits: int):
    """-> float32 values float(code) * float(scale); callers round to their dtype."""
    q = np.asarray(q)
    if bits == 4:
        lo = (q & 0x0F).astype(np.int16) - 8
        hi = (q >> 4).astype(np.int16) - 8
        q = np.stack((lo, hi), axis=-1).reshape(*q.shape[:-1], q.shape[-1] * 2)
    return q.astype(np.float32) * np.asarray(scale, dtype=np.float16).astype(np.float32)[..., None]


def quantize_torch_cpu(x, bits: int):
    """The reference lines (kv_tier_manager.py:21-31) run verbatim by torch on the CPU."""
    import torch

    qmax = 127 if bits == 8 else 7
    scale = x.abs().amax(-1, keepdim=True).float().clamp_min(1e-8) / qmax
    q = torch.round(x.float() / scale).clamp(-qmax, qmax).to(torch.int8)
    if bits == 4:
        q = q + 8
        q = (q[..., 0::2] | (q[..., 1::2] << 4)).to(torch.uint8)
    return q, scale.squeeze(-1).to(torch.float16)


def bf16_round(x):
    """float32 -> nearest bf16 value (ties to even), returned as float32."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16).astype(np.uint32)
    r = np.where(nan, (u.astype(np.uint32) | 0x00400000) & 0xFFFF0000, r)
    return r.view(np.float32).reshape(a.shape)
