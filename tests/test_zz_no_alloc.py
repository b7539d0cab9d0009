"""GPU: coopt_accept_sample_noalloc (the accept entry point that allocates nothing: its
workspace is the library's file-scope device array) against coopt_accept_sample with a
caller workspace, both through the C ABI: bit-identical accepted lengths, tokens and margins
on two calls in a row, the second smaller than the first (the array keeps the first call's
contents), for fp32 and bf16 logits, sampling and greedy, ragged gamma with row offsets."""
import numpy as np
import pytest
import torch

from iitj_llm_coopt_amd import _lib

pytestmark = pytest.mark.gpu


def report(msg):
    print(msg, flush=True)


def inputs(dev, B, g, V, seed, dtype, ragged=False):
    gen = torch.Generator(device=dev).manual_seed(seed)
    tl = (torch.randn(B, g + 1, V, generator=gen, device=dev) * 2).to(dtype).contiguous()
    dl = (tl[:, :g].float() + torch.randn(B, g, V, generator=gen, device=dev) * 0.5).to(dtype).contiguous()
    dt = torch.randint(0, V, (B, g), generator=gen, device=dev, dtype=torch.int32)
    dt[:, 0] = tl[:, 0].float().argmax(-1).to(torch.int32)      # some acceptances
    ua = torch.rand(B, g, generator=gen, device=dev)
    ur = torch.rand(B, generator=gen, device=dev)
    gam = (torch.arange(B, device=dev, dtype=torch.int32) % (g + 1)) if ragged else None
    t0 = (torch.arange(B, device=dev, dtype=torch.int32) * (g + 1)) if ragged else None
    d0 = (torch.arange(B, device=dev, dtype=torch.int32) * g) if ragged else None
    return tl, dl, dt, ua, ur, gam, t0, d0


def call(lib, noalloc, x, T, B, g, V, dev):
    tl, dl, dt, ua, ur, gam, t0, d0 = x
    acc = torch.full((B,), -7, dtype=torch.int32, device=dev)
    tok = torch.full((B, g + 1), -7, dtype=torch.int32, device=dev)
    marg = torch.full((B,), -7.0, dtype=torch.float32, device=dev)
    P = _lib.ptr
    common = (_lib.dt_code(tl.dtype), P(tl), V, P(t0), 0, P(dl), V, P(d0), P(dt), P(gam), P(ua),
              P(ur), float(T), B, g, V, P(acc), P(tok), P(marg))
    if noalloc:
        rc = lib.coopt_accept_sample_noalloc(*common, _lib.stream_handle(dev))
    else:
        need = lib.coopt_accept_sample_workspace(B, g, V)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        rc = lib.coopt_accept_sample(*common, P(ws), need, _lib.stream_handle(dev))
    assert rc == _lib.COOPT_OK, _lib.last_error()
    torch.cuda.synchronize(dev)
    return acc.cpu(), tok.cpu(), marg.cpu()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T", [1.0, 0.0])
def test_noalloc_matches_the_workspace_entry_point(dev, dtype, T):
    lib = _lib.load()
    shapes = [(32, 4, 128256, False), (3, 2, 5000, True)]   # the second call is smaller
    for i, (B, g, V, ragged) in enumerate(shapes):
        x = inputs(dev, B, g, V, 40 + i, dtype, ragged)
        report(f"[noalloc] call {i}: B={B} gamma={g} V={V} {dtype} T={T} ragged={ragged}")
        a = call(lib, True, x, T, B, g, V, dev)
        b = call(lib, False, x, T, B, g, V, dev)
        for u, v, name in zip(a, b, ("accepted_len", "tokens", "margin")):
            assert torch.equal(u, v), f"call {i}: {name} differs"
        assert int(a[0].min()) >= 0 and int((a[1][:, 0] >= 0).sum()) == B


def test_noalloc_python_path_in_a_graph(dev):
    """spec_decode.accept(workspace="static") recorded into a HIP graph and replayed with new
    inputs between replays, against eager calls with a caller workspace."""
    import iitj_llm_coopt_amd as M
    B, g, V = 16, 4, 32000
    x = inputs(dev, B, g, V, 50, torch.float32)
    tl, dl, dt, ua, ur, _, _, _ = x
    out = M.AcceptResult(torch.empty(B, dtype=torch.int32, device=dev),
                         torch.empty((B, g + 1), dtype=torch.int32, device=dev),
                         torch.empty(B, dtype=torch.float32, device=dev))
    M.accept(tl, dl, dt, 1.0, ua, ur, out=out, workspace="static")   # warm-up
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        M.accept(tl, dl, dt, 1.0, ua, ur, out=out, workspace="static")
    for i in range(3):
        y = inputs(dev, B, g, V, 60 + i, torch.float32)
        for dst, src in zip((tl, dl, dt, ua, ur), y[:5]):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize(dev)
        ref = M.accept(tl, dl, dt, 1.0, ua, ur)
        assert torch.equal(out.accepted_len, ref.accepted_len), i
        assert torch.equal(out.tokens, ref.tokens), i
