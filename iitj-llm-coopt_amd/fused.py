"""Fused elementwise stages of the Llama forward around the verify path, on gfx950 kernels.

Counterparts of the vLLM ops the reference's forward calls (engine/model.py:234-254):
  rms_norm(x, weight, eps, residual=None, out=None)   _ops.rms_norm / _ops.fused_add_rms_norm
  rope_(q, k, positions, cos, sin)                     _ops.rotary_embedding (neox, in place)
  silu_and_mul(gate_up, out=None)                      torch.ops._C.silu_and_mul
  linear(x, weight, out=None)                          F.linear projections (model.py:238-253)
  pack_linear_weight(weight)                           the weight in tile-packed form, for linear
"""
import ctypes

import torch
import torch.nn.functional as F

from . import _lib

__all__ = ["rms_norm", "rope_", "silu_and_mul", "linear", "LinearPartials", "LINEAR_MAX_ROWS",
           "PackedWeight", "pack_linear_weight", "pack_gate_up_weight", "linear_silu",
           "row_major"]

LINEAR_MAX_ROWS = 256
_WS = _lib.WorkspaceCache()


def _bf16_rows(t, name):
    if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
        raise ValueError(f"{name} must be bf16 with a contiguous last dimension")


class LinearPartials:
    """The unreduced output of linear(..., defer_reduce=True): `ks` fp32 slices of shape
    [rows_padded, N] in the linear workspace whose sum is the layer's output.  It is valid
    until the next linear() call on the same stream (which reuses the workspace); rms_norm()
    and silu_and_mul() reduce it while reading."""

    def __init__(self, buf, ks, rows, rows_padded, n, shape, device):
        self.buf, self.ks, self.rows, self.rows_padded, self.n = buf, ks, rows, rows_padded, n
        self.shape, self.device = shape, device

    def reduce(self):
        """The bf16 output itself (the sum of the slices in order, rounded once)."""
        part = self.buf[: self.ks * self.rows_padded * self.n * 4].view(torch.float32)
        part = part.view(self.ks, self.rows_padded, self.n)[:, : self.rows]
        acc = part[0].clone()
        for k in range(1, self.ks):
            acc += part[k]
        return acc.to(torch.bfloat16).view(self.shape)


def rms_norm(x, weight, eps, residual=None, out=None):
    """out = rmsnorm(x) * weight; with `residual`, first residual += x in place (fused add).
    x may be a LinearPartials (the split-K output of linear(..., defer_reduce=True)), reduced
    in the same pass."""
    if isinstance(x, LinearPartials):
        return _rms_norm_partials(x, weight, eps, residual, out)
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


def _rms_norm_partials(xp, weight, eps, residual, out):
    _lib.require_cuda(weight, residual, out)
    _bf16_rows(weight, "weight")
    if weight.numel() != xp.n or xp.n > 8192:
        raise ValueError("weight must match the partials' width (at most 8192)")
    if residual is not None and (tuple(residual.shape) != tuple(xp.shape) or not residual.is_contiguous()):
        raise ValueError("residual must be contiguous with the layer output's shape")
    if out is None:
        out = torch.empty(xp.shape, dtype=torch.bfloat16, device=xp.device)
    _lib.check(_lib.load().coopt_rms_norm_partials(
        _lib.ptr(xp.buf), xp.ks, xp.rows_padded * xp.n, _lib.ptr(residual), _lib.ptr(weight),
        _lib.ptr(out), xp.rows, xp.n, float(eps), _lib.stream_handle(xp.device)),
        "coopt_rms_norm_partials")
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
    """[T, 2F] -> [T, F]: silu(gate) * up.  gate_up may be a LinearPartials (the split-K output
    of linear(..., defer_reduce=True)), reduced in the same pass."""
    if isinstance(gate_up, LinearPartials):
        xp = gate_up
        _lib.require_cuda(out)
        F = xp.n // 2
        if xp.n % 16:
            raise ValueError("gate_up width must be a multiple of 16")
        if out is None:
            out = torch.empty(xp.shape[:-1] + (F,), dtype=torch.bfloat16, device=xp.device)
        _lib.check(_lib.load().coopt_silu_mul_partials(
            _lib.ptr(xp.buf), xp.ks, xp.rows_padded * xp.n, _lib.ptr(out), xp.rows, F,
            _lib.stream_handle(xp.device)), "coopt_silu_mul_partials")
        return out
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


class PackedWeight:
    """A projection weight [N, K] kept twice: row-major (`weight`, for torch's GEMM at
    prefill-sized row counts) and tile-packed (`packed`, coopt_linear_pack_weight's layout, for
    the weight-streaming kernel).  linear() picks the copy its path reads; both give the same
    result bit for bit on the kernel path."""

    def __init__(self, weight, packed, gate_up=False):
        # gate_up: packed by coopt_linear_pack_gate_up (gate / up tiles interleaved), read only
        # by linear_silu; linear() then streams the row-major copy
        self.weight, self.packed, self.gate_up = weight, packed, gate_up

    @property
    def shape(self):
        return self.weight.shape

    @property
    def dtype(self):
        return self.weight.dtype

    @property
    def device(self):
        return self.weight.device


def row_major(weight):
    """The row-major [N, K] tensor of a weight (a PackedWeight's first copy, else itself)."""
    return weight.weight if isinstance(weight, PackedWeight) else weight


def pack_gate_up_weight(weight):
    """PackedWeight of a bf16 [2F, K] gate_up weight for linear_silu (F a multiple of 16, K of
    128): one coopt_linear_pack_gate_up launch at model load."""
    _lib.require_cuda(weight)
    if weight.dtype != torch.bfloat16 or weight.dim() != 2 or weight.stride(-1) != 1:
        raise ValueError("weight must be a bf16 [2F, K] matrix with contiguous rows")
    N2, K = weight.shape
    if N2 % 32 or K % 128:
        raise ValueError("packing needs 2F a multiple of 32 and K a multiple of 128")
    packed = torch.empty(N2 * K, dtype=torch.bfloat16, device=weight.device)
    _lib.check(_lib.load().coopt_linear_pack_gate_up(
        _lib.ptr(weight), weight.stride(0), N2 // 2, K, _lib.ptr(packed),
        _lib.stream_handle(weight.device)), "coopt_linear_pack_gate_up")
    return PackedWeight(weight, packed, gate_up=True)


def linear_silu(x, weight, out=None):
    """silu_and_mul(linear(x, weight)) (engine/model.py:250-252).  With a gate_up PackedWeight
    and a shape the fused kernel takes (coopt_linear_silu_supported: draft or verify row counts
    with K unsplit), one
    coopt_linear_silu_packed launch, bit-identical to the two-step path; otherwise the two
    steps."""
    if isinstance(weight, PackedWeight) and weight.gate_up:
        K = x.shape[-1]
        x2 = x.reshape(-1, K)
        M, F = x2.shape[0], weight.shape[0] // 2
        lib = _lib.load()
        if (x.dtype == torch.bfloat16 and x.is_cuda and lib.coopt_linear_silu_supported(M, F, K)):
            _lib.require_cuda(x, out)
            if x2.stride(-1) != 1 or x2.stride(0) % 8:
                x2 = x2.contiguous()
            if out is None:
                out = torch.empty(x.shape[:-1] + (F,), dtype=torch.bfloat16, device=x.device)
            y2 = out.view(-1, F)
            _lib.check(lib.coopt_linear_silu_packed(
                _lib.ptr(x2), x2.stride(0), _lib.ptr(weight.packed), M, F, K, _lib.ptr(y2),
                y2.stride(0), _lib.stream_handle(x.device)), "coopt_linear_silu_packed")
            return out
    return silu_and_mul(linear(x, weight, defer_reduce=True), out=out)


def pack_linear_weight(weight):
    """PackedWeight of a bf16 [N, K] weight on the GPU (N a multiple of 16, K of 128): one
    coopt_linear_pack_weight launch at model load."""
    _lib.require_cuda(weight)
    if weight.dtype != torch.bfloat16 or weight.dim() != 2 or weight.stride(-1) != 1:
        raise ValueError("weight must be a bf16 [N, K] matrix with contiguous rows")
    N, K = weight.shape
    if N % 16 or K % 128:
        raise ValueError("packing needs N a multiple of 16 and K a multiple of 128")
    packed = torch.empty(N * K, dtype=torch.bfloat16, device=weight.device)
    _lib.check(_lib.load().coopt_linear_pack_weight(
        _lib.ptr(weight), weight.stride(0), N, K, _lib.ptr(packed),
        _lib.stream_handle(weight.device)), "coopt_linear_pack_weight")
    return PackedWeight(weight, packed)


def linear(x, weight, out=None, defer_reduce=False):
    """x [..., K] @ weight[N, K]^T -> [..., N], bf16 with fp32 accumulation (no bias), as the
    reference's projections (F.linear at engine/model.py:238, 248, 250, 253).

    The weight-streaming kernel coopt_linear takes bf16 operands with K a multiple of 128 at
    up to LINEAR_MAX_ROWS rows, and runs where it measured faster than torch's GEMM on MI355X:
    up to 64 rows (draft steps), or N <= 8192 outputs at any supported row count (the verify
    step's qkv / o / down projections).  Other shapes -- prefill-sized row counts, and the
    wide gate_up / lm_head outputs at verify row counts -- go to torch (hipBLASLt).

    defer_reduce=True (no `out`): on the kernel path, return a LinearPartials instead of the
    tensor, for rms_norm() or silu_and_mul() to reduce in their own pass; other paths return
    the tensor.

    `weight` may be a PackedWeight: the kernel path then streams its tile-packed copy
    (coopt_linear_packed), torch's path its row-major one."""
    packed = weight.packed if isinstance(weight, PackedWeight) and not weight.gate_up else None
    if isinstance(weight, PackedWeight):
        weight = weight.weight
    _lib.require_cuda(x, weight, out)
    K = x.shape[-1]
    N = weight.shape[0]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    if (M > LINEAR_MAX_ROWS or K % 128 or N % 4 or x.dtype != torch.bfloat16
            or weight.dtype != torch.bfloat16 or weight.dim() != 2 or weight.shape[1] != K
            or (M > 64 and N > 8192)):
        return F.linear(x, weight, out=out) if out is not None else F.linear(x, weight)
    if x2.stride(-1) != 1 or x2.stride(0) % 8:
        x2 = x2.contiguous()
    if packed is None and (weight.stride(-1) != 1 or weight.stride(0) % 8):
        weight = weight.contiguous()
    lib = _lib.load()
    if defer_reduce and out is None:
        ks, rp = ctypes.c_int(0), ctypes.c_int(0)
        _lib.check(lib.coopt_linear_split(M, N, K, ctypes.byref(ks), ctypes.byref(rp)),
                   "coopt_linear_split")
        ws = _WS.get(ks.value * rp.value * N * 4, x.device)
        if packed is None:
            _lib.check(lib.coopt_linear_partials(
                _lib.ptr(x2), x2.stride(0), _lib.ptr(weight), weight.stride(0), M, N, K,
                _lib.ptr(ws), ws.numel(), _lib.stream_handle(x.device)), "coopt_linear_partials")
        else:
            _lib.check(lib.coopt_linear_partials_packed(
                _lib.ptr(x2), x2.stride(0), _lib.ptr(packed), M, N, K, _lib.ptr(ws), ws.numel(),
                _lib.stream_handle(x.device)), "coopt_linear_partials_packed")
        return LinearPartials(ws, ks.value, M, rp.value, N, x.shape[:-1] + (N,), x.device)
    if out is None:
        out = torch.empty(x.shape[:-1] + (N,), dtype=torch.bfloat16, device=x.device)
    y2 = out.view(-1, N)
    need = int(lib.coopt_linear_workspace(M, N, K))
    ws = _WS.get(need, x.device) if need else None
    if packed is None:
        _lib.check(lib.coopt_linear(
            _lib.ptr(x2), x2.stride(0), _lib.ptr(weight), weight.stride(0), M, N, K, _lib.ptr(y2),
            y2.stride(0), _lib.ptr(ws), 0 if ws is None else ws.numel(),
            _lib.stream_handle(x.device)), "coopt_linear")
    else:
        _lib.check(lib.coopt_linear_packed(
            _lib.ptr(x2), x2.stride(0), _lib.ptr(packed), M, N, K, _lib.ptr(y2), y2.stride(0),
            _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_handle(x.device)),
            "coopt_linear_packed")
    return out
