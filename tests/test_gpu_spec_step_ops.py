"""GPU: the step bookkeeping kernels (coopt_spec_step_begin / _verify_tokens / _commit) against
the reference's per-sequence rules restated on the host (engine/engine.py:354-389 lag and
catch-up, 380-389 proposals, 414-417 verify rows, 444-446 counters, 455 append, 463-470
rollback), on random states with speculating, lagging, plain-decode and dummy slots, catch-up
strides 2 and 5, and histories at their length limit.  Bar: every output exact.  The whole
step is compared with the oracle step in test_gpu_spec_step_parity.py."""
import numpy as np
import pytest
import torch

from iitj_llm_coopt_amd import _lib

pytestmark = pytest.mark.gpu


def host_begin(live, gamma, n, dc, hist, max_len, Bc, G, S_c):
    out = {k: [] for k in ("geff", "cu_start", "cu_nreal", "cu_tok", "cu_keep", "pr_start",
                           "pr_nreal", "v_start", "v_nreal", "v_tok0", "dc_final")}
    pr_s = np.zeros((max(G - 1, 0), Bc), np.int64)
    pr_n = np.zeros((max(G - 1, 0), Bc), np.int64)
    for b in range(Bc):
        lv, gq, nn, d = bool(live[b]), int(gamma[b]), int(n[b]), int(dc[b])
        lag = nn - d
        want = lv and gq > 0
        spec, lagging = want and lag <= 2, want and lag > 2
        ge = gq if spec else 0
        m = lag if spec else (min(lag - 1, S_c) if lagging else 0)
        out["geff"].append(ge)
        dc1 = d
        if G > 0:
            st = d if lv else 0
            out["cu_start"].append(st)
            out["cu_nreal"].append(m)
            out["cu_tok"].append([hist[b, min(st + j, max_len - 1)] for j in range(S_c)])
            out["cu_keep"].append(b * S_c + max(m - 1, 0))
            dc1 = d + m
            for i in range(1, G):
                act = 1 if (spec and ge > i) else 0
                pr_s[i - 1, b] = dc1 if lv else 0
                pr_n[i - 1, b] = act
                dc1 += act
        vs = nn - 1 if lv else 0
        out["v_start"].append(vs)
        out["v_nreal"].append(ge + 1 if lv else 0)
        out["v_tok0"].append(hist[b, vs])
        out["dc_final"].append(dc1)
    out["pr_start"], out["pr_nreal"] = pr_s, pr_n
    return out


@pytest.mark.parametrize("S_c", [2, 5])
@pytest.mark.parametrize("seed", [0, 1])
def test_begin_verify_tokens_commit_match_host_rules(dev, S_c, seed):
    rng = np.random.default_rng(seed + 10 * S_c)
    Bcap, Bc, gmax, S_t, max_len, V = 48, 37, 4, 5, 64, 1000
    G = gmax
    print(f"[step ops] seed {seed} S_c {S_c} Bc {Bc}", flush=True)
    live = np.zeros(Bcap, np.uint8)
    live[:30] = 1                                   # slots 30.. are dummies
    gamma = rng.integers(0, gmax + 1, Bcap).astype(np.int64)
    gamma[30:] = 0
    n = rng.integers(10, max_len - 2, Bcap).astype(np.int64)
    n[:4] = max_len - 1                              # histories at their limit
    lag = rng.choice([1, 1, 2, 2, 3, 4, 7, 12], Bcap)
    dc = np.maximum(n - lag, 0).astype(np.int64)
    hist = rng.integers(0, V, (Bcap, max_len)).astype(np.int64)
    nu, u_rows = Bcap * (2 * gmax + 1), 5
    u_table = rng.random((u_rows, nu)).astype(np.float32)
    ctr0 = 7

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    d_live, d_gamma, d_n, d_dc, d_hist = t(live), t(gamma), t(n), t(dc), t(hist)
    d_ut, d_ctr = t(u_table), torch.tensor(ctr0, dtype=torch.int64, device=dev)
    i64 = dict(dtype=torch.int64, device=dev)
    d_u = torch.zeros(nu, dtype=torch.float32, device=dev)
    geff = torch.zeros(Bcap, dtype=torch.int32, device=dev)
    cu_start, cu_nreal, cu_keep = (torch.full((Bcap,), -9, **i64) for _ in range(3))
    cu_tok = torch.full((Bcap * S_c,), -9, **i64)
    pr_start = torch.full((gmax, Bcap), -9, **i64)
    pr_nreal = torch.full((gmax, Bcap), -9, **i64)
    v_start, v_nreal, dc_final = (torch.full((Bcap,), -9, **i64) for _ in range(3))
    vt = torch.full((Bcap, S_t), -9, dtype=torch.int32, device=dev)
    lib, P = _lib.load(), _lib.ptr
    stream = _lib.stream_handle(dev)
    _lib.check(lib.coopt_spec_step_begin(
        P(d_ut), u_rows, nu, P(d_ctr), P(d_u), P(d_live), P(d_gamma), P(d_n), P(d_dc), P(d_hist),
        max_len, max_len, Bc, G, S_c, S_t, P(geff), P(cu_start), P(cu_nreal), P(cu_tok),
        P(cu_keep), P(pr_start), P(pr_nreal), pr_start.stride(0), P(v_start), P(v_nreal), P(vt),
        P(dc_final), stream), "begin")
    torch.cuda.synchronize()
    ref = host_begin(live, gamma, n, dc, hist, max_len, Bc, G, S_c)
    assert int(d_ctr) == ctr0 + 1
    assert np.array_equal(d_u.cpu().numpy(), u_table[ctr0 % u_rows])
    assert geff[:Bc].cpu().tolist() == ref["geff"]
    assert cu_start[:Bc].cpu().tolist() == ref["cu_start"]
    assert cu_nreal[:Bc].cpu().tolist() == ref["cu_nreal"]
    assert cu_tok[: Bc * S_c].view(Bc, S_c).cpu().tolist() == [[int(x) for x in r] for r in ref["cu_tok"]]
    assert cu_keep[:Bc].cpu().tolist() == ref["cu_keep"]
    assert np.array_equal(pr_start[: G - 1, :Bc].cpu().numpy(), ref["pr_start"])
    assert np.array_equal(pr_nreal[: G - 1, :Bc].cpu().numpy(), ref["pr_nreal"])
    assert v_start[:Bc].cpu().tolist() == ref["v_start"]
    assert v_nreal[:Bc].cpu().tolist() == ref["v_nreal"]
    assert vt[:Bc, 0].cpu().tolist() == [int(x) for x in ref["v_tok0"]]
    assert dc_final[:Bc].cpu().tolist() == ref["dc_final"]
    # nothing written past the batch
    assert int(cu_start[Bc]) == -9 and int(v_start[Bc]) == -9

    # verify rows: proposals (proposal-major) into [b][1 + i] and the accept's [b][i]
    prop = torch.from_numpy(rng.integers(0, V, (S_t - 1, Bcap)).astype(np.int32)).to(dev)
    dt = torch.full((Bc, S_t - 1), -9, dtype=torch.int32, device=dev)
    _lib.check(lib.coopt_spec_step_verify_tokens(P(prop), prop.stride(0), Bc, S_t, P(vt), P(dt),
                                                 stream), "verify_tokens")
    torch.cuda.synchronize()
    assert torch.equal(vt[:Bc, 1:], prop[:, :Bc].t())
    assert torch.equal(dt, prop[:, :Bc].t())
    assert vt[:Bc, 0].cpu().tolist() == [int(x) for x in ref["v_tok0"]]

    # commit: accepted lengths within each sequence's gamma_eff, tokens random
    ge = np.array(ref["geff"])
    acc = np.array([rng.integers(0, g + 1) for g in ge], np.int32)
    acc[~live[:Bc].astype(bool)] = rng.integers(0, S_t, int((~live[:Bc].astype(bool)).sum()))
    toks = rng.integers(0, V, (Bc, S_t)).astype(np.int32)
    emitted, drafted, accepted = (torch.tensor(v, dtype=torch.int64, device=dev) for v in (5, 6, 7))
    d_acc, d_toks = t(acc), t(toks)   # held until the launch has run
    _lib.check(lib.coopt_spec_step_commit(
        P(d_live), P(d_acc), P(d_toks), S_t, P(geff), P(dc_final), P(d_n), P(d_dc), P(d_hist),
        max_len, max_len, P(emitted), P(drafted), P(accepted), Bc, stream), "commit")
    torch.cuda.synchronize()
    h_hist, h_n, h_dc = hist.copy(), n.copy(), dc.copy()
    e = dr = ac = 0
    for b in range(Bc):
        if live[b]:
            k = int(acc[b])
            for j in range(k + 1):
                if n[b] + j < max_len:
                    h_hist[b, n[b] + j] = toks[b, j]
            h_n[b] = n[b] + k + 1
            h_dc[b] = min(ref["dc_final"][b], h_n[b] - 1)
            e += k + 1
            ac += k
        dr += ref["geff"][b]
    assert np.array_equal(d_hist.cpu().numpy(), h_hist)
    assert np.array_equal(d_n.cpu().numpy(), h_n)
    assert np.array_equal(d_dc.cpu().numpy(), h_dc)
    assert (int(emitted), int(drafted), int(accepted)) == (5 + e, 6 + dr, 7 + ac)


def test_argument_errors_are_reported(dev):
    lib = _lib.load()
    rc = lib.coopt_spec_step_commit(None, None, None, 1, None, None, None, None, None, 4, 8,
                                    None, None, None, 0, None)
    assert rc != 0 and b"hist_stride" in lib.coopt_last_error()
    rc = lib.coopt_spec_step_verify_tokens(None, 1, 4, 3, None, None, None)
    assert rc != 0 and b"null" in lib.coopt_last_error()
