"""GPU: coopt_linear (weight-streaming projections at decode / verify row counts) against an
fp32 reference of the same op, y = x w^T.

Bar: |y - ref| <= 2^-8 |ref| + 2 K 2^-24 sum_k |x_k w_k| per element -- one bf16 rounding
(unit roundoff 2^-8)
of the output plus fp32 summation error -- written below as `bound`.  Repeated calls and HIP
graph replays are bit-identical (fixed-order split-K reduction).
"""
import pytest
import torch
import torch.nn.functional as F

from iitj_llm_coopt_amd import _lib, fused

pytestmark = pytest.mark.gpu


def ref_and_bound(x, w):
    xf, wf = x.float(), w.float()
    ref = xf @ wf.t()
    mag = xf.abs() @ wf.abs().t()
    K = x.shape[-1]
    return ref, 2.0 ** -8 * ref.abs() + 2 * K * 2.0 ** -24 * mag + 1e-30


def check(y, x, w, label):
    ref, bound = ref_and_bound(x, w)
    err = (y.float() - ref).abs()
    worst = (err / bound).max().item()
    print(f"[linear {label}] max err/bound {worst:.3f}", flush=True)
    assert worst <= 1.0, label


@pytest.mark.parametrize("M,N,K", [
    (160, 6144, 4096), (160, 4096, 4096), (160, 4096, 14336), (32, 3072, 2048),
    (32, 2048, 8192), (64, 16384, 2048), (1, 256, 128), (17, 100, 384), (200, 64, 640),
    (256, 520, 1152), (5, 4, 128),
])
def test_linear_matches_fp32_reference(dev, M, N, K):
    g = torch.Generator(device=dev).manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    ws = int(_lib.load().coopt_linear_workspace(M, N, K))
    print(f"[linear] M={M} N={N} K={K} workspace {ws} B", flush=True)
    y = fused.linear(x, w)
    check(y, x, w, f"{M}x{N}x{K}")
    assert torch.equal(y, fused.linear(x, w))          # deterministic


def test_linear_strided_rows_and_out(dev):
    M, N, K = 40, 272, 1024
    g = torch.Generator(device=dev).manual_seed(3)
    xb = torch.randn(M, K + 64, generator=g, device=dev).to(torch.bfloat16)
    x = xb[:, 32:32 + K]                                  # row stride K + 64, offset 64 B
    w = (torch.randn(N, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    yb = torch.full((M, N + 12), 7.0, device=dev, dtype=torch.bfloat16)
    y = yb[:, :N]
    fused.linear(x, w, out=y)
    check(y, x, w, "strided")
    assert torch.all(yb[:, N:] == 7.0)                    # nothing written past N


def test_linear_large_rows_use_torch(dev):
    x = torch.randn(300, 256, device=dev).to(torch.bfloat16)
    w = torch.randn(64, 256, device=dev).to(torch.bfloat16)
    assert torch.equal(fused.linear(x, w), F.linear(x, w))


def test_linear_graph_replay_equals_eager(dev):
    M, N, K = 160, 4096, 4096
    g = torch.Generator(device=dev).manual_seed(11)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager = fused.linear(x, w)
        out = torch.empty_like(eager)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            fused.linear(x, w, out=out)
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        x2 = fused.linear(x, w)                           # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(x2, eager)


def test_linear_argument_errors(dev):
    x = torch.randn(4, 128, device=dev).to(torch.bfloat16)
    w = torch.randn(8, 128, device=dev).to(torch.bfloat16)
    y = torch.empty(4, 8, device=dev, dtype=torch.bfloat16)
    L = _lib.load()
    st = _lib.stream_handle(dev)
    assert L.coopt_linear(_lib.ptr(x), 128, _lib.ptr(w), 128, 4, 8, 100, _lib.ptr(y), 8, None, 0, st) != 0
    assert "multiple of 128" in _lib.last_error()
    assert L.coopt_linear(_lib.ptr(x), 128, _lib.ptr(w), 128, 300, 8, 128, _lib.ptr(y), 8, None, 0, st) != 0
    need = int(L.coopt_linear_workspace(160, 4096, 4096))
    assert need > 0
    xx = torch.empty(160, 4096, device=dev, dtype=torch.bfloat16)
    ww = torch.empty(4096, 4096, device=dev, dtype=torch.bfloat16)
    yy = torch.empty(160, 4096, device=dev, dtype=torch.bfloat16)
    assert L.coopt_linear(_lib.ptr(xx), 4096, _lib.ptr(ww), 4096, 160, 4096, 4096, _lib.ptr(yy), 4096,
                          None, 0, st) != 0
    assert "workspace" in _lib.last_error()


# (160, 4096, 4352) splits K 7 ways: a slice count that is not a power of two, so the
# consumers' compile-time-bounded loaders (bound 8) repeat the last slice without adding it.
@pytest.mark.parametrize("M,N,K", [(160, 4096, 4096), (160, 4096, 14336), (32, 2048, 2048),
                                   (32, 2048, 8192), (17, 264, 256), (64, 2048, 128),
                                   (160, 4096, 4352)])
def test_deferred_reduction_into_rms_norm_is_bit_exact(dev, M, N, K):
    """linear(defer_reduce=True) + rms_norm(partials) == linear() + rms_norm(), bit for bit,
    with and without the fused residual add (the reduction order is the same)."""
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    ln = (1 + 0.1 * torch.randn(N, generator=g, device=dev)).to(torch.bfloat16)
    res = torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16)
    y = fused.linear(x, w)
    part = fused.linear(x, w, defer_reduce=True)
    assert isinstance(part, fused.LinearPartials)
    print(f"[defer] M={M} N={N} K={K}: {part.ks} slice(s) of {part.rows_padded} rows", flush=True)
    assert torch.equal(part.reduce(), y)
    want = fused.rms_norm(y, ln, 1e-5)
    got = fused.rms_norm(part, ln, 1e-5)
    assert torch.equal(got, want)
    r1, r2 = res.clone(), res.clone()
    want = fused.rms_norm(y, ln, 1e-5, residual=r1)
    part = fused.linear(x, w, defer_reduce=True)
    got = fused.rms_norm(part, ln, 1e-5, residual=r2)
    assert torch.equal(got, want) and torch.equal(r2, r1)


@pytest.mark.parametrize("M,F,K", [(32, 8192, 2048), (64, 8192, 2048), (5, 64, 256),
                                   (32, 512, 4224)])   # the last splits K 7 ways
def test_deferred_reduction_into_silu_mul_is_bit_exact(dev, M, F, K):
    """linear(defer_reduce=True) + silu_and_mul(partials) == linear() + silu_and_mul()."""
    g = torch.Generator(device=dev).manual_seed(M + F + K)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(2 * F, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    want = fused.silu_and_mul(fused.linear(x, w))
    part = fused.linear(x, w, defer_reduce=True)
    print(f"[defer silu] M={M} F={F} K={K}: {part.ks} slice(s)", flush=True)
    assert torch.equal(fused.silu_and_mul(part), want)


# ---- tile-packed weights (coopt_linear_pack_weight, coopt_linear_packed) ----

def packed_layout(w):
    """The documented packed layout as torch views: tile (t, u) of 16 rows x 128 K, 16-byte
    chunk j * 64 + l = w[16 t + l % 16][128 u + 32 j + 8 (l // 16), +8)."""
    N, K = w.shape
    return w.reshape(N // 16, 16, K // 128, 4, 4, 8).permute(0, 2, 3, 4, 1, 5).reshape(-1)


@pytest.mark.parametrize("N,K,pad", [(16, 128, 0), (48, 256, 0), (4096, 4096, 0), (96, 384, 64)])
def test_pack_weight_layout(dev, N, K, pad):
    g = torch.Generator(device=dev).manual_seed(N + K + pad)
    wb = torch.randn(N, K + pad, generator=g, device=dev).to(torch.bfloat16)
    w = wb[:, :K]                                         # row stride K + pad
    p = fused.pack_linear_weight(w)
    torch.cuda.synchronize()
    assert p.packed.numel() == N * K
    assert torch.equal(p.packed.view(torch.int16), packed_layout(w.contiguous()).view(torch.int16))
    # one spot by hand: tile (1, 0), chunk j = 2, lane 37 -> row 16 + 5, K 64 + 16
    if N >= 32:
        off = ((1 * (K // 128) + 0) * 256 + 2 * 64 + 37) * 8
        assert torch.equal(p.packed[off:off + 8], w[21, 80:88])


# shapes of every launch plan: 160 rows (10 row tiles, split K), the draft's 32 / 64 rows,
# lm_head widths (4 tiles per wave row-major, 1 packed), a K split 7 ways, tails in M, one row
@pytest.mark.parametrize("M,N,K", [
    (160, 6144, 4096), (160, 4096, 14336), (160, 4096, 4352), (32, 3072, 2048), (64, 2048, 8192),
    (32, 128256, 2048), (64, 128256, 2048), (1, 256, 128), (17, 96, 384), (200, 64, 640),
    (256, 528, 1152),
])
def test_packed_linear_is_bit_identical_to_row_major(dev, M, N, K):
    g = torch.Generator(device=dev).manual_seed(M * 3 + N + K)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    pw = fused.pack_linear_weight(w)
    y = fused.linear(x, w)
    yp = fused.linear(x, pw)
    print(f"[packed] M={M} N={N} K={K}", flush=True)
    assert torch.equal(yp.view(torch.int16), y.view(torch.int16))
    check(yp, x, w, f"packed {M}x{N}x{K}")
    part = fused.linear(x, w, defer_reduce=True)
    n = part.ks * part.rows_padded * part.n * 4
    want = part.buf[:n].clone()
    part_p = fused.linear(x, pw, defer_reduce=True)
    assert (part_p.ks, part_p.rows_padded) == (part.ks, part.rows_padded)
    assert torch.equal(part_p.buf[:n], want)


def test_packed_weight_on_the_torch_path(dev):
    """Row counts above the kernel's range use the PackedWeight's row-major copy."""
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(300, 256, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(64, 256, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    assert torch.equal(fused.linear(x, fused.pack_linear_weight(w)), F.linear(x, w))


def test_pack_weight_errors(dev):
    w = torch.randn(40, 128, device=dev).to(torch.bfloat16)
    with pytest.raises(ValueError):
        fused.pack_linear_weight(w)
    out = torch.empty(40 * 128, device=dev, dtype=torch.bfloat16)
    L = _lib.load()
    assert L.coopt_linear_pack_weight(_lib.ptr(w), 128, 40, 128, _lib.ptr(out), _lib.stream_handle(dev)) != 0
    assert "multiple of 16" in _lib.last_error()
    x = torch.randn(4, 128, device=dev).to(torch.bfloat16)
    y = torch.empty(4, 40, device=dev, dtype=torch.bfloat16)
    assert L.coopt_linear_packed(_lib.ptr(x), 128, _lib.ptr(out), 4, 40, 128, _lib.ptr(y), 40, None, 0,
                                 _lib.stream_handle(dev)) != 0
    assert "multiple of 16" in _lib.last_error()


# ---- gate_up fused with SiLU-and-mul (coopt_linear_pack_gate_up, coopt_linear_silu_packed) ----

def test_pack_gate_up_interleaves_gate_and_up_tiles(dev):
    F, K = 48, 256
    g = torch.Generator(device=dev).manual_seed(5)
    w = torch.randn(2 * F, K, generator=g, device=dev).to(torch.bfloat16)
    p = fused.pack_gate_up_weight(w)
    order = torch.cat([torch.stack([w[16 * s:16 * s + 16], w[F + 16 * s:F + 16 * s + 16]])
                       for s in range(F // 16)]).reshape(2 * F, K)     # gate 0, up 0, gate 1, ...
    assert torch.equal(p.packed.view(torch.int16), packed_layout(order).view(torch.int16))


@pytest.mark.parametrize("M,F,K", [(32, 8192, 2048), (64, 8192, 2048), (1, 512, 256), (17, 48, 384),
                                   (64, 16, 128), (160, 14336, 4096), (131, 14336, 4096)])
def test_linear_silu_is_bit_identical_to_linear_then_silu(dev, M, F, K):
    g = torch.Generator(device=dev).manual_seed(M + F + K)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(2 * F, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    assert _lib.load().coopt_linear_silu_supported(M, F, K) == 1    # the fused launch runs
    want = fused.silu_and_mul(fused.linear(x, w))
    got = fused.linear_silu(x, fused.pack_gate_up_weight(w))
    print(f"[linear_silu] M={M} F={F} K={K}", flush=True)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_linear_silu_falls_back_outside_the_fused_shapes(dev):
    """160 rows (a split K and 8 waves) and torch-sized row counts take the two-step path."""
    g = torch.Generator(device=dev).manual_seed(2)
    for M, F, K in [(160, 2048, 2048), (300, 64, 256)]:
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        w = (torch.randn(2 * F, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
        assert _lib.load().coopt_linear_silu_supported(M, F, K) == 0
        want = fused.silu_and_mul(fused.linear(x, w))
        assert torch.equal(fused.linear_silu(x, fused.pack_gate_up_weight(w)), want)
