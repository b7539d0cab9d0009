"""Benchmark: verified tokens/s of the speculative step at gamma=4, B=32 on one MI355X, with the
verification-attention kernel's HBM roofline and the CPU path timed on the same host.

    python bench.py [--steps 128] [--warmup 3] [--batch 32] [--gamma 4] [--prompt 1024]

Workload (BASELINE.json config 5 at the metric's B=32): random-init Llama-3.1-8B-shaped target
(32 layers, hidden 4096, 32/8 heads, head_dim 128, FFN 14336, RoPE theta 5e5, vocab 128256) with a
paged INT8 KV cache, Llama-3.2-1B-shaped draft (16 layers, hidden 2048, head_dim 64, FFN 8192,
tied embeddings) with a paged bf16 KV cache; B prompts of 1024 seeded uniform-random ids are
prefilled, then each timed step is one HIP-graph replay of: draft catch-up + gamma draft
proposals (temperature 1.0, draws from the decoder's seeded uniform table), one (gamma+1)-row
target verify forward, the fused accept kernel and the length/history update.  value = tokens
emitted by the accept step (sum of k_b + 1) per second over the timed steps; also reported:
scored positions/s (B (gamma+1) per step) and config 5's stated B=16.

Printed: one JSON line (the driver's contract) with `roofline` for the verify-attention kernel
(40 back-to-back launches between HIP events on torch's current stream, the stream the kernels
run on, averaged per launch) and `cpu_baseline`: the reference's step restated on the host
(oracle.spec_step) from the GPU run's state, at every core and at 8 threads, each step checked
against the GPU step it shadows.  The kernel cases of configs 1-4 carry `cpu` legs: the
reference's verify loop, quantize + index_put and textbook paged attention on the host.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s

METRIC = "verified tokens/s at γ=4 B=32 on 1 MI355X; verify-attn HBM GB/s as % of peak"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--gamma", type=int, default=4)
    ap.add_argument("--prompt", type=int, default=1024)
    ap.add_argument("--temperature", type=float, default=1.0)
    ap.add_argument("--cpu-steps", type=int, default=4,
                    help="steps of the CPU baseline (half at all threads, half at 8)")
    ap.add_argument("--b16-steps", type=int, default=20,
                    help="timed steps of config 5's stated B=16 (0: skip)")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline leg and the configs' CPU legs")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-tune-gemm", action="store_true",
                    help="skip PyTorch TunableOp selection of the decode-shape GEMMs")
    ap.add_argument("--no-kernel-cases", action="store_true",
                    help="skip the per-kernel cases (roofline is then null); for profiling the step")
    ap.add_argument("--kernels-only", action="store_true",
                    help="run only the per-kernel cases (no model step), for profiling")
    ap.add_argument("--case", action="append", choices=sorted(KERNEL_CASES),
                    help="with --kernels-only: the case(s) to run (default: all)")
    ap.add_argument("--summarize", metavar="DIR", nargs="+",
                    help="print a text summary of the rocprofv3 CSV output under DIR(s) and exit")
    return ap.parse_args()


def head_start(torch, dev):
    """Queues ~10 ms of GPU work so the host enqueues the timed launches ahead of the GPU and
    the events bracket kernel time, not host latency."""
    a = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
    for _ in range(8):
        a = a @ a * 1e-3
    return a


def time_launches(torch, dev, fn, n=40):
    """(average, median) duration of fn().  The average is n back-to-back calls between two
    HIP events divided by n: the sustained per-call time, launch gaps included, which is what
    a kernel-trace average plus the gap between kernels measures.  The median is over n calls
    each bracketed by its own pair of events (each pair's marker packets add a little)."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize(dev)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    keep = head_start(torch, dev)
    t0.record()
    for _ in range(n):
        fn()
    t1.record()
    torch.cuda.synchronize(dev)
    del keep
    avg = t0.elapsed_time(t1) * 1e-3 / n
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    keep = head_start(torch, dev)
    for s, e in ev:
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize(dev)
    del keep
    d = sorted(s.elapsed_time(e) * 1e-3 for s, e in ev)
    return avg, d[n // 2]


def rate(res, nbytes, avg, med):
    res.update({"bytes": nbytes, "avg_us": avg * 1e6, "median_us": med * 1e6,
                "GB_s": nbytes / avg / 1e9, "frac": nbytes / avg / HBM_PEAK})
    return res


CPU_LEGS = {"on": True}   # main() turns the configs' CPU legs off with --no-cpu


def cpu_legs(torch, fn, reps=3):
    """Median wall time of fn() on the host cores, at torch's default thread count (every
    core this process may use) and at 8 threads (the reference's OMP_NUM_THREADS,
    runpod/setup.sh:23).  One untimed call first."""
    out = {}
    n_all = torch.get_num_threads()
    for label, n in (("all_cores", n_all), ("threads_8", 8)):
        torch.set_num_threads(n)
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        out[label] = {"seconds": sorted(ts)[len(ts) // 2], "threads": n}
    torch.set_num_threads(n_all)
    out["affinity_cores"] = len(os.sched_getaffinity(0))
    return out


def cpu_attention(torch, q, kc, vc, ks, vs, table, seq, qlen, seqs, D):
    """Textbook paged attention on the host (FlashAttention has no CPU path): per sequence,
    gather its pages, dequantise INT8 to bf16 (dequantize(), engine/kv_tier_manager.py:34-41),
    softmax(scale * q K^T + bottom-right causal mask) V in fp32."""
    import math

    out = torch.empty(len(seqs) * qlen, q.shape[1], D, dtype=torch.bfloat16)
    Hkv = kc.shape[2]
    G = q.shape[1] // Hkv
    for i, b in enumerate(seqs):
        L = int(seq[b])
        pos = torch.arange(L)
        blk, off = table[b].long()[pos // 16], pos % 16
        if ks is None:
            K, V = kc[blk, off].float(), vc[blk, off].float()
        else:
            K = (kc[blk, off].float() * ks[blk, off].float().unsqueeze(-1)).to(torch.bfloat16).float()
            V = (vc[blk, off].float() * vs[blk, off].float().unsqueeze(-1)).to(torch.bfloat16).float()
        Q = q[b * qlen:(b + 1) * qlen].float().view(qlen, Hkv, G, D).permute(1, 0, 2, 3).reshape(Hkv, qlen * G, D)
        sc = torch.matmul(Q, K.permute(1, 2, 0)) / math.sqrt(D)
        lim = torch.repeat_interleave(L - qlen + torch.arange(qlen), G)
        sc = sc.masked_fill(torch.arange(L)[None, None, :] > lim[None, :, None], float("-inf"))
        o = torch.matmul(torch.softmax(sc, -1), V.permute(1, 0, 2))
        out[i * qlen:(i + 1) * qlen] = o.view(Hkv, qlen, G, D).permute(1, 0, 2, 3).reshape(qlen, -1, D)
    return out


def attention_setup(torch, M, dev, ctx, qlen, kv_dtype, seed, D=128, outlier=0.01,
                    layout="head"):
    """The paged cache of an attention case: len(ctx) sequences with ctx[b] cached tokens and
    q_len new rows each (seq_len = ctx + q_len), Hq 32 / Hkv 8, head size D, block size 16,
    block tables a seeded permutation of a shared pool.  K/V are N(0,1), each element x20
    with probability `outlier` (configs 2 and 4; config 3 is plain N(0,1)), quantised on write
    for INT8.  layout: the caches' storage --
      "head"   allocate_kv_cache: [NB, bs, Hkv, D] views of head-major storage (a head's 16
               tokens of a block contiguous), scales likewise;
      "token"  the reference's own per-layer caches, token-major [NB, bs, Hkv, D]
               (engine/model.py:148-155), INT8 scales [NB, bs, Hkv] as quantize(cache[blocks])
               lays them out (engine/kv_tier_manager.py:99);
      "block"  a per-layer view buf[:, l, 0/1] of the elastic block-major buffer
               [NB, 32, 2, bs, Hkv, D] (engine/elastic.py:74-77; bf16 only, as there)."""
    import numpy as np

    Hq, Hkv, bs = 32, 8, 16
    ctx = np.asarray(ctx, np.int64)
    B = len(ctx)
    seq = ctx + qlen
    W = -(-seq // bs)
    nblk = int(W.sum()) + 1
    perm = np.random.default_rng(seed).permutation(nblk)
    table_np = np.zeros((B, int(W.max())), np.int32)
    o = 0
    for b in range(B):
        table_np[b, :W[b]] = perm[o:o + W[b]]
        o += int(W[b])
    table = torch.from_numpy(table_np).to(dev)
    buf = None
    if layout == "head":
        kc, vc, ks, vs = M.allocate_kv_cache(nblk, bs, Hkv, D, kv_dtype, device=dev)
    elif layout == "token":
        cdt = torch.int8 if kv_dtype == "int8" else torch.bfloat16
        kc = torch.zeros(nblk, bs, Hkv, D, dtype=cdt, device=dev)
        vc = torch.zeros_like(kc)
        ks = torch.zeros(nblk, bs, Hkv, dtype=torch.float16, device=dev) if kv_dtype == "int8" else None
        vs = None if ks is None else torch.zeros_like(ks)
    elif layout == "block" and kv_dtype == "auto":
        buf, kl, vl = M.allocate_block_major_kv(nblk, 32, bs, Hkv, D, device=dev)
        kc, vc, ks, vs = kl[13], vl[13], None, None     # one layer's strided views
    else:
        raise ValueError(f"no {layout} layout for {kv_dtype} caches")
    g = torch.Generator(device=dev).manual_seed(seed)
    slots = torch.arange(nblk * bs, device=dev)
    for lo in range(0, nblk * bs, 1 << 18):   # fill the pool in chunks
        hi = min(nblk * bs, lo + (1 << 18))
        kv = torch.randn(2, hi - lo, Hkv, D, generator=g, device=dev)
        if outlier:
            kv = torch.where(torch.rand(kv.shape, generator=g, device=dev) < outlier, kv * 20, kv)
        kv = kv.to(torch.bfloat16)
        M.reshape_and_cache_flash(kv[0], kv[1], kc, vc, slots[lo:hi], kv_dtype, ks, vs)
        del kv
    cu = torch.arange(B + 1, dtype=torch.int32, device=dev) * qlen
    sl = torch.from_numpy(seq.astype(np.int32)).to(dev)
    per_tok = Hkv * D * 2 * 2 if kv_dtype == "auto" else Hkv * (2 * D + 2 * 2)
    return dict(Hq=Hq, Hkv=Hkv, bs=bs, ctx=ctx, B=B, seq=seq, table_np=table_np, table=table,
                caches=(kc, vc, ks, vs), gen=g, cu=cu, sl=sl, max_k=int(seq.max()),
                per_tok=per_tok, buf=buf)


# MI355X's Infinity Cache (256 MB) holds a call's whole working set when it is small and the
# same call repeats back to back; in the step, a layer's cache was last read a whole forward
# earlier.  Cases rotate over enough copies of their cache to exceed twice that size.
INFINITY_CACHE_BYTES = 256 << 20


def cache_copies(nbytes):
    return max(1, -(-2 * INFINITY_CACHE_BYTES // max(int(nbytes), 1)))


def attention_case(torch, M, dev, ctx, qlen, kv_dtype, seed, D=128, cpu_sample=0, outlier=0.01,
                   layout="head"):
    """Verify attention (coopt_verify_attention) over the cache of attention_setup, the calls
    rotating over cache_copies() copies of it (one at the roofline shape)."""
    st = attention_setup(torch, M, dev, ctx, qlen, kv_dtype, seed, D, outlier, layout)
    Hq, Hkv, B, seq, ctx = st["Hq"], st["Hkv"], st["B"], st["seq"], st["ctx"]
    kc, vc, ks, vs = st["caches"]
    table, cu, sl, max_k, g = st["table"], st["cu"], st["sl"], st["max_k"], st["gen"]
    q = torch.randn(B * qlen, Hq, D, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    ws = torch.empty(M.attention.workspace_bytes(B, Hq, Hkv, D, qlen, max_k), dtype=torch.uint8,
                     device=dev)
    nbytes = int(seq.sum()) * st["per_tok"] + 2 * B * qlen * Hq * D * 2
    sets = [(kc, vc, ks, vs, table, st["buf"])]
    for i in range(1, cache_copies(nbytes)):
        o = attention_setup(torch, M, dev, ctx.tolist(), qlen, kv_dtype, seed + 1000 * i, D,
                            outlier, layout)
        sets.append((*o["caches"], o["table"], o["buf"]))
    turn = [0]

    def fn():
        c = sets[turn[0] % len(sets)]
        turn[0] += 1
        M.paged_attention(q, c[0], c[1], cu, sl, c[4], qlen, max_k, D ** -0.5, c[2], c[3], out, ws)

    cpu_sample = cpu_sample if CPU_LEGS["on"] else 0

    res = {"kv": kv_dtype, "head_dim": D, "batch": B, "q_len": qlen, "ctx_min": int(ctx.min()),
           "ctx_max": int(ctx.max()), "ctx_mean": float(ctx.mean()), "cache_copies": len(sets),
           "cache_layout": layout, "outliers": outlier}
    res = rate(res, nbytes, *time_launches(torch, dev, fn))
    M.paged_attention(q, kc, vc, cu, sl, table, qlen, max_k, D ** -0.5, ks, vs, out, ws)
    if cpu_sample:
        # the same call on the host cores over the first cpu_sample sequences, scaled to the
        # batch by their share of the keys
        seqs = list(range(min(cpu_sample, B)))
        hc = [None if t is None else t.cpu() for t in (kc, vc, ks, vs)]
        hq, ht = q.cpu(), table.cpu()
        legs = cpu_legs(torch, lambda: cpu_attention(torch, hq, *hc, ht, seq, qlen, seqs, D), reps=1)
        share = float(seq[seqs].sum()) / float(seq.sum())
        for k in ("all_cores", "threads_8"):
            legs[k]["us_per_call"] = legs[k]["seconds"] / share * 1e6
        got = cpu_attention(torch, hq, *hc, ht, seq, qlen, seqs[:2], D).float()
        legs["max_abs_vs_gpu_first_2_seqs"] = float((got - out[: 2 * qlen].float().cpu()).abs().max())
        legs["sample"] = f"{len(seqs)} of {B} sequences ({share:.1%} of the keys), fp32 torch on the host"
        res["cpu"] = legs
    return res


def attention_qkv_case(torch, M, dev, ctx, qlen, kv_dtype, seed, D=128, hidden=4096):
    """The step's form of the call: coopt_verify_attention_qkv, the qkv projection's split-K
    partials in (coopt_linear_packed with defer_reduce, as the step runs it: hidden -> (Hq +
    2 Hkv) D over B q_len rows), RoPE, the new rows' K/V written at key positions ctx ..
    ctx + q_len - 1, and the attention over the cache of attention_setup.  Algorithmic bytes:
    the K/V of every key (the new ones read back after their write), the partials once, the
    new rows' K/V written, the RoPE table rows and the output.  The calls rotate over
    cache_copies() copies of the cache (the partials, as in the step, stay warm)."""
    import numpy as np

    st = attention_setup(torch, M, dev, ctx, qlen, kv_dtype, seed, D)
    Hq, Hkv, bs, B, seq, ctx = st["Hq"], st["Hkv"], st["bs"], st["B"], st["seq"], st["ctx"]
    g = st["gen"]
    T, width = B * qlen, (Hq + 2 * Hkv) * D
    x = torch.randn(T, hidden, generator=g, device=dev).to(torch.bfloat16)
    w = M.fused.pack_linear_weight((torch.randn(width, hidden, generator=g, device=dev) * 0.02)
                                   .to(torch.bfloat16))
    part = M.fused.linear(x, w, defer_reduce=True)
    if not isinstance(part, M.fused.LinearPartials):
        raise RuntimeError("expected split-K partials from the qkv projection")
    pos_np = np.concatenate([np.arange(c, c + qlen) for c in ctx]).astype(np.int64)
    pos = torch.from_numpy(pos_np).to(dev)

    def cache_set(o):  # caches, table and the new rows' slots of one copy
        tb = o["table_np"]
        slot_np = np.concatenate([tb[b][np.arange(c, c + qlen) // bs] * bs + np.arange(c, c + qlen) % bs
                                  for b, c in enumerate(ctx)]).astype(np.int64)
        return (*o["caches"], o["table"], torch.from_numpy(slot_np).to(dev))
    max_pos = st["max_k"] + 8
    inv = 500000.0 ** (-torch.arange(0, D // 2, dtype=torch.float64) * 2 / D)
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None, :]
    cos, sin = ang.cos().to(dev, torch.bfloat16), ang.sin().to(dev, torch.bfloat16)
    if not M.qkv_attention_supported(kv_dtype, B, Hq, Hkv, D, qlen, st["max_k"]):
        raise RuntimeError("shape not taken by the fused call")
    out = torch.empty(T, Hq, D, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(M.attention.workspace_bytes(B, Hq, Hkv, D, qlen, st["max_k"]),
                     dtype=torch.uint8, device=dev)

    nbytes = (int(seq.sum()) * st["per_tok"] + part.ks * T * width * 4 + T * st["per_tok"]
              + T * D * 2 + T * Hq * D * 2)
    sets = [cache_set(st)]
    for i in range(1, cache_copies(nbytes)):
        sets.append(cache_set(attention_setup(torch, M, dev, ctx.tolist(), qlen, kv_dtype,
                                              seed + 1000 * i, D)))
    turn = [0]

    def fn():
        kc, vc, ks, vs, table, slots = sets[turn[0] % len(sets)]
        turn[0] += 1
        M.paged_attention_qkv(part, pos, cos, sin, slots, kc, vc, st["cu"], st["sl"], table,
                              qlen, st["max_k"], Hq, D ** -0.5, kv_dtype, ks, vs, out, ws)

    res = {"kv": kv_dtype, "head_dim": D, "batch": B, "q_len": qlen, "ctx": int(ctx.max()),
           "qkv_partials": part.ks, "hidden": hidden, "cache_copies": len(sets)}
    return rate(res, nbytes, *time_launches(torch, dev, fn))


def accept_case(torch, M, dev, B, gamma, V, seed):
    """Config 1: target N(0, 2^2), draft = target + N(0, 0.5^2), fp32 logits; the draft tokens
    sampled from the draft softmax at T = 1 (sample(), inverse CDF on seeded uniforms), so the
    accept positions, and with them the rows decide reads, follow the config's mix."""
    g = torch.Generator(device=dev).manual_seed(seed)
    tl = torch.randn(B, gamma + 1, V, generator=g, device=dev) * 2
    dl = (tl[:, :gamma] + torch.randn(B, gamma, V, generator=g, device=dev) * 0.5).contiguous()
    ud = torch.rand(B * gamma, generator=g, device=dev)
    dt = M.sample(dl.view(B * gamma, V), 1.0, uniforms=ud)[0].view(B, gamma).long()
    ua = torch.rand(B, gamma, generator=g, device=dev)
    ur = torch.rand(B, generator=g, device=dev)
    res = M.accept(tl, dl, dt, 1.0, ua, ur)
    ws = torch.empty(M._lib.load().coopt_accept_sample_workspace(B, gamma, V), dtype=torch.uint8,
                     device=dev)
    dt32 = dt.to(torch.int32)

    def fn():
        M.accept(tl, dl, dt32, 1.0, ua, ur, out=res, workspace=ws)

    nbytes = B * (2 * gamma + 1) * V * 4 + B * 2 * V * 4
    res = rate({"batch": B, "gamma": gamma, "vocab": V}, nbytes, *time_launches(torch, dev, fn))
    if CPU_LEGS["on"]:
        # engine/engine.py:437-446 on the host: per sequence, the draft softmax the engine
        # keeps from sample() and the reference's verify lines (engine/spec_decode.py:37-49)
        # executed by torch-CPU with the same uniforms
        from oracle import accept as OA
        htl, hdl, hdt, hua, hur = (t.cpu() for t in (tl, dl, dt, ua, ur))

        def loop():
            return [OA.verify_torch(htl[b], hdt[b].tolist(), torch.softmax(hdl[b], -1), 1.0,
                                    hua[b], float(hur[b])) for b in range(B)]
        legs = cpu_legs(torch, loop)
        for k in ("all_cores", "threads_8"):
            legs[k]["us_per_call"] = legs[k]["seconds"] * 1e6
        got = M.accept(tl, dl, dt32, 1.0, ua, ur).to_lists()
        ref = loop()
        legs["sequences_equal_to_gpu"] = sum(a == b for a, b in zip(got, ref))
        legs["sample"] = f"the whole batch: {B} sequences, torch-CPU"
        res["cpu"] = legs
    return res


def kv_write_case(torch, M, dev, T, seed):
    """Config 2: 256 sequences append T / 256 new tokens each (5 at config 2's T = 1280; 256
    in the T = 65,536 sweep) at existing lengths U[0, 4096), with block tables from a seeded
    permutation of a 65,536-block pool (BlockManager's free list), so each sequence's new
    tokens fill consecutive slots of its blocks; Hkv 8, D 128, INT8 quantise on write; N(0,1)
    with 1% x20 outliers."""
    import numpy as np

    NB, bs, Hkv, D, nseq = 65536, 16, 8, 128, 256
    new = T // nseq
    kc, vc, ks, vs = M.allocate_kv_cache(NB, bs, Hkv, D, "int8", device=dev)
    rng = np.random.default_rng(seed)
    bm = M.BlockManager(NB, bs, free_order=rng.permutation(NB))
    existing = rng.integers(0, 4096, nseq)
    parts = []
    for sq in range(nseq):
        bm.ensure(sq, int(existing[sq]) + new)
        parts.append(bm.slot_mapping(sq, int(existing[sq]), int(existing[sq]) + new).numpy())
    slots = torch.from_numpy(np.concatenate(parts).astype(np.int64)).to(dev)
    T = int(slots.numel())
    g = torch.Generator(device=dev).manual_seed(seed)
    kv = torch.randn(2, T, Hkv, D, generator=g, device=dev)
    kv = torch.where(torch.rand(kv.shape, generator=g, device=dev) < 0.01, kv * 20, kv)
    k, v = kv.to(torch.bfloat16).unbind(0)

    def fn():
        M.reshape_and_cache_flash(k, v, kc, vc, slots, "int8", ks, vs)

    nbytes = T * Hkv * D * (2 * 2 + 2 * 1) + T * Hkv * 2 * 2 + T * 8
    res = rate({"tokens": T}, nbytes, *time_launches(torch, dev, fn))
    if CPU_LEGS["on"] and T <= 4096:
        # the reference's quantize lines (engine/kv_tier_manager.py:21-31) on torch-CPU and
        # the index_put write (engine/model.py:201-203) into host caches of the same pool
        from oracle import codec as OC
        hk, hv, hs = k.cpu(), v.cpu(), slots.cpu()
        ck = torch.zeros(NB, bs, Hkv, D, dtype=torch.int8)
        cv = torch.zeros_like(ck)
        sk = torch.zeros(NB, bs, Hkv, dtype=torch.float16)
        sv = torch.zeros_like(sk)
        blk, off = hs // bs, hs % bs

        def write():
            for x, c, sc in ((hk, ck, sk), (hv, cv, sv)):
                qx, s_ = OC.quantize_torch_cpu(x, 8)
                c[blk, off] = qx
                sc[blk, off] = s_
        legs = cpu_legs(torch, write)
        for kk in ("all_cores", "threads_8"):
            legs[kk]["us_per_call"] = legs[kk]["seconds"] * 1e6
        write()
        # torch-CPU divides by 127 exactly; on the GPU the reference's "/ 127" is a multiply by
        # fp32(1/127) (what the kernel restates), so a few near-tie elements round apart.
        # Reported: how many codes the two differ in, and whether the GPU's codes equal the
        # oracle codec's GPU-division mode on every element.
        ndiff, total, dev_equal = 0, 0, True
        for x, c, gc in ((hk, ck, kc), (hv, cv, vc)):
            gpu = gc[slots // bs, slots % bs].cpu()
            ndiff += int((c[blk, off] != gpu).sum())
            total += gpu.numel()
            dq, _ = OC.quantize(x.float().numpy(), 8, mode="device")
            dev_equal &= bool(np.array_equal(dq, gpu.numpy()))
        legs["codes_differing_from_gpu"] = f"{ndiff} of {total} (torch-CPU true division)"
        legs["gpu_codes_equal_to_oracle_gpu_division"] = dev_equal
        legs["sample"] = f"the whole call: {T} tokens, torch-CPU"
        res["cpu"] = legs
    return res


def kv_swap_case(torch, M, dev, seed, tokens=4096, bits=8):
    """Swap codec, one launch: gather + INT8-quantise one layer's K blocks of a `tokens`-token
    sequence (bf16 cache, head-major storage, blocks a seeded permutation of a 4096-block
    pool) into the contiguous swap format."""
    import numpy as np

    NB, bs, Hkv, D = 4096, 16, 8, 128
    cache, _, _, _ = M.allocate_kv_cache(NB, bs, Hkv, D, "auto", device=dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    cache.copy_(torch.randn(cache.shape, generator=g, device=dev).to(torch.bfloat16))
    nb = tokens // bs
    blocks = torch.from_numpy(np.random.default_rng(seed).permutation(NB)[:nb].astype(np.int64)).to(dev)
    q, sc = M.swap_out_blocks(cache, blocks, bits)

    def fn():
        M.swap_out_blocks(cache, blocks, bits, out=q, out_scale=sc)

    nbytes = nb * bs * Hkv * (D * 2 + D * bits // 8 + 2) + nb * 8
    return rate({"tokens": tokens, "bits": bits}, nbytes, *time_launches(torch, dev, fn))


def kv_swap_all_case(torch, M, dev, seed, tokens=4096, layers=32, bits=8):
    """Swap codec over a whole sequence, one launch: gather + INT8-quantise the K and V blocks
    of a `tokens`-token sequence in all `layers` layers (bf16 caches, head-major, blocks a
    seeded permutation of the pool) into the contiguous [2 L, ...] swap format."""
    import numpy as np

    NB, bs, Hkv, D = 2 * tokens // 16, 16, 8, 128
    g = torch.Generator(device=dev).manual_seed(seed)
    caches = []
    for _ in range(2 * layers):
        c, _, _, _ = M.allocate_kv_cache(NB, bs, Hkv, D, "auto", device=dev)
        c.copy_(torch.randn(c.shape, generator=g, device=dev).to(torch.bfloat16))
        caches.append(c)
    nb = tokens // bs
    blocks = torch.from_numpy(np.random.default_rng(seed).permutation(NB)[:nb].astype(np.int64)).to(dev)
    q, sc = M.swap_out_caches(caches, blocks, bits)

    def fn():
        M.swap_out_caches(caches, blocks, bits, out=q, out_scale=sc)

    nbytes = 2 * layers * (nb * bs * Hkv * (D * 2 + D * bits // 8 + 2)) + nb * 8
    return rate({"tokens": tokens, "layers": layers, "caches": 2 * layers, "bits": bits}, nbytes,
                *time_launches(torch, dev, fn))


def kv_swap_in_all_case(torch, M, dev, seed, tokens=4096, layers=32, bits=8):
    """Swap codec back, one launch: dequantise a `tokens`-token sequence's INT8 swap rows of
    all `layers` layers' K and V and scatter them into the bf16 caches' blocks (head-major
    storage, blocks a seeded permutation of the pool)."""
    import numpy as np

    NB, bs, Hkv, D = 2 * tokens // 16, 16, 8, 128
    g = torch.Generator(device=dev).manual_seed(seed)
    caches = []
    for _ in range(2 * layers):
        c, _, _, _ = M.allocate_kv_cache(NB, bs, Hkv, D, "auto", device=dev)
        c.copy_(torch.randn(c.shape, generator=g, device=dev).to(torch.bfloat16))
        caches.append(c)
    nb = tokens // bs
    blocks = torch.from_numpy(np.random.default_rng(seed).permutation(NB)[:nb].astype(np.int64)).to(dev)
    q, sc = M.swap_out_caches(caches, blocks, bits)

    def fn():
        M.swap_in_caches(q, sc, bits, blocks, caches)

    nbytes = 2 * layers * (nb * bs * Hkv * (D * 2 + D * bits // 8 + 2)) + nb * 8
    return rate({"tokens": tokens, "layers": layers, "caches": 2 * layers, "bits": bits}, nbytes,
                *time_launches(torch, dev, fn))


def sample_case(torch, M, dev, seed, B=32, V=128256, probs=True):
    """The sample() drop-in (engine/spec_decode.py:12-17) at config 1's draft shape: fp32
    logits [B, V] at T = 1 -> one token per row by inverse CDF and the probability rows.
    Algorithmic bytes: the logits read once and the probabilities written once.  probs=False:
    tokens only, as the step draws its draft tokens (bf16 logits there), logits read once."""
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(B, V, generator=g, device=dev) * 2.0
    u = torch.rand(B, generator=g, device=dev)

    def fn():
        M.sample(x, 1.0, uniforms=u, return_probs=probs)

    return rate({"B": B, "V": V, "probs": probs}, (2 if probs else 1) * B * V * 4,
                *time_launches(torch, dev, fn))


def codec_case(torch, M, dev, seed, direction, rows=262144, D=128, bits=8):
    """The standalone codec (kv_tier_manager.quantize / dequantize): bf16 [rows, D] <-> INT8
    codes + fp16 scales per row; rows = 32768 tokens x 8 heads (64 MiB of bf16)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(rows, D, generator=g, device=dev).to(torch.bfloat16)
    q, sc = M.quantize(x, bits)
    if direction == "quantize":
        def fn():
            M.quantize(x, bits)
    else:
        def fn():
            M.dequantize(q, sc, bits, torch.bfloat16)
    nbytes = rows * (D * 2 + D * bits // 8 + 2)
    return rate({"rows": rows, "D": D, "bits": bits}, nbytes, *time_launches(torch, dev, fn))


def kv_tier_case(torch, M, dev, seed, tokens=4096, layers=32):
    """KVTierManager swap_out + swap_in of one `tokens`-token sequence of a Llama-3.1-8B-shaped
    target (32 layers, bf16 caches, INT8 tier): codec launches plus the PCIe copies to and from
    pinned host memory, host-timed around synchronisation (PCIe-inclusive)."""
    import types

    import numpy as np

    NB, bs, Hkv, D = 2 * tokens // 16, 16, 8, 128
    kc, vc = [], []
    g = torch.Generator(device=dev).manual_seed(seed)
    for _ in range(layers):
        a, b, _, _ = M.allocate_kv_cache(NB, bs, Hkv, D, "auto", device=dev)
        a.copy_(torch.randn(a.shape, generator=g, device=dev).to(torch.bfloat16))
        b.copy_(torch.randn(b.shape, generator=g, device=dev).to(torch.bfloat16))
        kc.append(a)
        vc.append(b)
    cfg = types.SimpleNamespace(num_hidden_layers=layers, num_key_value_heads=Hkv, head_dim=D)
    eng = types.SimpleNamespace(target=types.SimpleNamespace(k_cache=kc, v_cache=vc, cfg=cfg),
                                bm=M.BlockManager(NB, bs, free_order=np.random.default_rng(seed).permutation(NB)),
                                counters={})
    tm = M.KVTierManager(eng, cpu_gb=64.0, bits=8)
    seq = types.SimpleNamespace(seq_id=0, num_computed=tokens)
    times = []
    for it in range(4):
        eng.bm.ensure(0, tokens)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        tm.swap_out(seq)
        eng.bm.free(0)
        tm.swap_in(seq)
        torch.cuda.synchronize(dev)
        if it:
            times.append(time.perf_counter() - t0)
        eng.bm.free(0)
    avg = sum(times) / len(times)
    host_bytes = 2 * tm.estimate_bytes(tokens, 8)   # out and back over PCIe
    return {"tokens": tokens, "layers": layers, "bits": 8, "host_bytes": host_bytes,
            "avg_us": avg * 1e6, "median_us": sorted(times)[len(times) // 2] * 1e6,
            "GB_s": host_bytes / avg / 1e9, "frac": None,
            "note": "PCIe-inclusive: swap_out (one codec launch over the 64 K/V caches, one D2H "
                    "copy) + swap_in (one H2D copy, one codec launch), host-timed"}


def migrate_case(torch, M, dev, seed, pairs=256):
    """Block migration copy: `pairs` blocks of the block-major elastic buffer of a
    Llama-3.1-8B-shaped target (32 layers x K/V x 16 tokens x 8 heads x 128, bf16: 2 MiB a
    block) move to free blocks, one coopt_kv_copy_blocks launch.  Also timed: the same pairs
    as one torch copy per block, the reference's copy_fn (engine/elastic.py:131)."""
    import numpy as np

    nb = 4 * pairs
    buf, _, _ = M.allocate_block_major_kv(nb, 32, 16, 8, 128, device=dev)
    buf.view(torch.int16).random_(generator=torch.Generator(device=dev).manual_seed(seed))
    perm = np.random.default_rng(seed).permutation(nb)
    src, dst = perm[:pairs], perm[pairs:2 * pairs]
    s_t = torch.from_numpy(src.astype(np.int64)).to(dev)
    d_t = torch.from_numpy(dst.astype(np.int64)).to(dev)
    M.copy_blocks(buf, src, dst)             # host checks once; the timed calls pass device ids

    def fn():
        M.copy_blocks(buf, s_t, d_t)

    res = rate({"pairs": pairs, "block_bytes": buf[0].numel() * 2},
               2 * pairs * buf[0].numel() * 2, *time_launches(torch, dev, fn, n=20))
    sl, dl = src.tolist(), dst.tolist()

    def per_block():
        for a, b in zip(sl, dl):
            buf[b].copy_(buf[a])

    avg, _ = time_launches(torch, dev, per_block, n=5)
    res["per_block_torch_copy_us"] = avg * 1e6
    return res


def linear_case(torch, M, dev, rows, n, k, seed, packed=False):
    """One projection of the step through fused.linear (coopt_linear, or coopt_linear_packed
    with the tile-packed weight the step's qkv / o / down use: split-K partials plus the
    reduction launch at these shapes): x [rows, k] @ w[n, k]^T, bf16, N(0,1) x, N(0, 0.02^2)
    weights.  Algorithmic bytes: the weight, x and y once each."""
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(rows, k, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    if packed:
        w = M.fused.pack_linear_weight(w)
    y = torch.empty(rows, n, dtype=torch.bfloat16, device=dev)

    def fn():
        M.fused.linear(x, w, out=y)

    res = rate({"rows": rows, "n": n, "k": k, "packed_weight": packed, "flops": 2 * rows * n * k},
               n * k * 2 + rows * k * 2 + rows * n * 2, *time_launches(torch, dev, fn))
    res["TFLOP_s"] = 2 * rows * n * k / (res["avg_us"] * 1e-6) / 1e12
    return res


def copy_case(torch, M, dev, seed):
    """A plain streaming kernel of known size (torch.neg over 1 GiB of bf16: 1 GiB read,
    1 GiB written): the calibration for FETCH_SIZE / WRITE_SIZE and a practical HBM ceiling."""
    n = 1 << 29
    a = torch.empty(n, dtype=torch.bfloat16, device=dev).fill_(1.0)
    b = torch.empty_like(a)

    def fn():
        torch.neg(a, out=b)

    return rate({"elements": n, "read_bytes": 2 * n, "write_bytes": 2 * n}, 4 * n,
                *time_launches(torch, dev, fn, n=20))


def config_ctx(seed, B, lo, hi):
    import numpy as np

    return np.random.default_rng(seed).integers(lo, hi + 1, B)


KERNEL_CASES = {
    # the roofline case: the metric's gamma=4, B=32, 8k context, INT8 KV (config 5's target)
    "attention_int8": lambda t, M, d, s: attention_case(t, M, d, [8192] * 32, 5, "int8", s),
    "attention_bf16": lambda t, M, d, s: attention_case(t, M, d, [8192] * 32, 5, "auto", s),
    # config 3: bf16, B=32, ctx U[512, 4096], q_len 5
    "attention_config3": lambda t, M, d, s: attention_case(t, M, d, config_ctx(s, 32, 512, 4096), 5, "auto", s, cpu_sample=32, outlier=0.0),
    # the roofline shape on the reference's own cache layouts: token-major per-layer caches
    # (engine/model.py:148-155) and a layer view of the block-major elastic buffer
    # (engine/elastic.py:74-77, bf16)
    "attention_int8_token_major": lambda t, M, d, s: attention_case(t, M, d, [8192] * 32, 5, "int8", s, layout="token"),
    "attention_bf16_token_major": lambda t, M, d, s: attention_case(t, M, d, [8192] * 32, 5, "auto", s, layout="token"),
    "attention_bf16_block_major": lambda t, M, d, s: attention_case(t, M, d, [8192] * 32, 5, "auto", s, layout="block"),
    # config 4: INT8, B=64, ctx U[4096, 16384], gamma 2 / 4 / 8
    "attention_config4_g2": lambda t, M, d, s: attention_case(t, M, d, config_ctx(s, 64, 4096, 16384), 3, "int8", s, cpu_sample=8),
    "attention_config4_g4": lambda t, M, d, s: attention_case(t, M, d, config_ctx(s, 64, 4096, 16384), 5, "int8", s, cpu_sample=8),
    "attention_config4_g8": lambda t, M, d, s: attention_case(t, M, d, config_ctx(s, 64, 4096, 16384), 9, "int8", s, cpu_sample=8),
    # the bench step's own attention launches (prompt 1024 + the tokens of the timed steps):
    # target verify (INT8, q_len 5), draft proposals (bf16, D 64, 1 row) and catch-up (2 rows)
    "attention_step_target": lambda t, M, d, s: attention_case(t, M, d, [1100] * 32, 5, "int8", s),
    "attention_step_draft": lambda t, M, d, s: attention_case(t, M, d, [1100] * 32, 1, "auto", s, D=64),
    "attention_step_draft_q2": lambda t, M, d, s: attention_case(t, M, d, [1100] * 32, 2, "auto", s, D=64),
    # the same launches as the step makes them: the qkv epilogue inside the attention launch
    "attention_qkv_step_target": lambda t, M, d, s: attention_qkv_case(t, M, d, [1100] * 32, 5, "int8", s),
    "attention_qkv_step_draft": lambda t, M, d, s: attention_qkv_case(t, M, d, [1100] * 32, 1, "auto", s, D=64, hidden=2048),
    # config 1 (B=8) and the metric's B=32
    "accept_b8": lambda t, M, d, s: accept_case(t, M, d, 8, 4, 128256, s),
    "accept_b32": lambda t, M, d, s: accept_case(t, M, d, 32, 4, 128256, s),
    # config 2 (T=1280) and a sustained-bandwidth size
    "kv_write_t1280": lambda t, M, d, s: kv_write_case(t, M, d, 1280, s),
    "kv_write_t65536": lambda t, M, d, s: kv_write_case(t, M, d, 65536, s),
    "kv_swap_out_4096tok": lambda t, M, d, s: kv_swap_case(t, M, d, s),
    "kv_swap_out_4096tok_32layers": lambda t, M, d, s: kv_swap_all_case(t, M, d, s),
    "kv_swap_in_4096tok_32layers": lambda t, M, d, s: kv_swap_in_all_case(t, M, d, s),
    "kv_tier_roundtrip": lambda t, M, d, s: kv_tier_case(t, M, d, s),
    "sample_b32": lambda t, M, d, s: sample_case(t, M, d, s),
    "sample_tokens_b32": lambda t, M, d, s: sample_case(t, M, d, s, probs=False),
    "codec_quantize_64MiB": lambda t, M, d, s: codec_case(t, M, d, s, "quantize"),
    "codec_dequantize_64MiB": lambda t, M, d, s: codec_case(t, M, d, s, "dequantize"),
    "kv_migrate_256x2MiB": lambda t, M, d, s: migrate_case(t, M, d, s),
    # the step's weight-streaming projections, tile-packed as in the step: target qkv / down
    # at the verify rows (B (gamma+1) = 160), draft lm_head at the draft rows (B = 32)
    "linear_m160_qkv": lambda t, M, d, s: linear_case(t, M, d, 160, 6144, 4096, s, packed=True),
    "linear_m160_down": lambda t, M, d, s: linear_case(t, M, d, 160, 4096, 14336, s, packed=True),
    "linear_m32_lm_head": lambda t, M, d, s: linear_case(t, M, d, 32, 128256, 2048, s, packed=True),
    "copy": lambda t, M, d, s: copy_case(t, M, d, s),
}


def layout_fracs(kern):
    """The roofline call's fraction of 8 TB/s on each cache layout (allocate_kv_cache's
    head-major storage, the reference's token-major caches, the elastic block-major view)."""
    names = {"int8": {"head_major": "attention_int8", "token_major": "attention_int8_token_major"},
             "bf16": {"head_major": "attention_bf16", "token_major": "attention_bf16_token_major",
                      "block_major_view": "attention_bf16_block_major"}}
    return {kv: {lay: round(kern[n]["frac"], 4) for lay, n in d.items() if n in kern}
            for kv, d in names.items()}


def run_kernel_cases(torch, M, dev, names, seed):
    out = {}
    for name in names:
        out[name] = KERNEL_CASES[name](torch, M, dev, seed)
        r = out[name]
        frac = "" if r["frac"] is None else f" ({r['frac'] * 100:.1f}% of 8 TB/s)"
        log(f"{name}: {r['avg_us']:.1f} us/call, {r['GB_s']:.0f} GB/s{frac}")
        torch.cuda.empty_cache()
    return out


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "verify_attention_int8_b32_ctx8192.md")


def committed_traffic():
    """HBM bytes per roofline call from the committed FETCH_SIZE / WRITE_SIZE profile (the
    `traffic_bytes_per_call:` line), or None."""
    import re

    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                m = re.match(r"\s*traffic_bytes_per_call:\s*([0-9.eE+]+)", line)
                if m:
                    return float(m.group(1))
    except OSError:
        pass
    return None


def _short(name):
    """Kernel name without `void`, anonymous namespaces and the argument list."""
    name = name.replace("(anonymous namespace)::", "").replace("void ", "")
    depth = 0
    for i, c in enumerate(name):
        if c == "<":
            depth += 1
        elif c == ">":
            depth -= 1
        elif c == "(" and depth == 0:
            return name[:i][:100]
    return name[:100]


# The roofline call's kernels (the PMC passes run only the attention_int8 case and the copy
# calibration, so every verify-attention or merge dispatch in them belongs to that call), and
# the copy calibration kernel.
ROOFLINE_KERNELS = ("verify_attn_kernel", "merge_kernel")
COPY_KERNEL = ("neg_kernel_cuda", 67108864, 1 << 30, 1 << 30)   # name part, grid, read, write


def summarize(paths):
    """Text summary of rocprofv3 CSV output under `paths`: per-(kernel, grid) durations
    (*kernel_trace.csv) and mean counter values per dispatch (*counter_collection.csv); with
    FETCH_SIZE and WRITE_SIZE for the copy calibration kernel and the roofline call's kernels,
    also the calibrated HBM bytes per roofline call (`traffic_bytes_per_call:`)."""
    import csv

    def rows(suffix):
        for path in paths:
            for dp, _, files in os.walk(path):
                for f in sorted(files):
                    if f.endswith(suffix):
                        with open(os.path.join(dp, f), newline="") as fh:
                            yield from csv.DictReader(fh)

    trace_rows = list(rows("kernel_trace.csv"))
    marks = sorted(int(r["Start_Timestamp"]) for r in trace_rows if "spin_kernel" in r["Kernel_Name"])
    if len(marks) >= 2:
        # the timed steps of a full bench.py run lie between its two marker kernels
        lo, hi = marks[0], marks[1]
        win = [r for r in trace_rows if lo < int(r["Start_Timestamp"]) < hi and "spin_kernel" not in r["Kernel_Name"]]
        fam = {}
        for r in win:
            n = _short(r["Kernel_Name"])
            k = "GEMM (hipBLASLt / rocBLAS)" if n.startswith(("Cijk", "Custom_Cijk")) else n.split("<")[0]
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            c, t = fam.get(k, (0, 0.0))
            fam[k] = (c + 1, t + d)
        busy = sum(t for _, t in fam.values())
        print(f"timed steps window: {(hi - lo) / 1e6:.2f} ms wall, {busy / 1e3:.2f} ms of kernel time, "
              f"{len(win)} kernels")
        print("| kernel family | launches | total us | share |")
        print("|---|---|---|---|")
        for k, (c, t) in sorted(fam.items(), key=lambda kv: -kv[1][1]):
            print(f"| `{k}` | {c} | {t:.0f} | {t / busy * 100:.1f}% |")
        shapes = {}
        for r in win:
            key = (_short(r["Kernel_Name"]), f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}x{r['Grid_Size_Z']}")
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            shapes.setdefault(key, []).append(d)
        print("\nsame window by launch shape (top 30 by total time):")
        print("| kernel | grid (threads) | launches | avg us | total us | share |")
        print("|---|---|---|---|---|---|")
        for (k, g), ds in sorted(shapes.items(), key=lambda kv: -sum(kv[1]))[:30]:
            print(f"| `{k}` | {g} | {len(ds)} | {sum(ds) / len(ds):.1f} | {sum(ds):.0f} | "
                  f"{sum(ds) / busy * 100:.1f}% |")
        print()
    trace = {}
    for r in trace_rows:
        grid = f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}x{r['Grid_Size_Z']}"
        key = (_short(r["Kernel_Name"]), grid, r["Workgroup_Size_X"])
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        trace.setdefault(key, []).append(d)
    if trace:
        # every launch shape of the library's kernels and the GEMMs; torch's own set-up kernels
        # (fills, copies, random draws) only among the first ten by total time
        ranked = sorted(trace.items(), key=lambda kv: -sum(kv[1]))
        shown = [kv for i, kv in enumerate(ranked)
                 if i < 10 or not kv[0][0].startswith(("at::", "__amd_rocclr", "elementwise_kernel",
                                                       "c10::", "std::"))]
        print("| kernel | grid (threads) | wg | calls | avg us | min us | max us | total ms |")
        print("|---|---|---|---|---|---|---|---|")
        for (k, grid, wg), ds in shown:
            print(f"| `{k}` | {grid} | {wg} | {len(ds)} | {sum(ds) / len(ds):.1f} | "
                  f"{min(ds):.1f} | {max(ds):.1f} | {sum(ds) / 1e3:.2f} |")
    agg = {}
    for r in rows("counter_collection.csv"):
        key = (_short(r["Kernel_Name"]), int(r["Grid_Size"]), r["Counter_Name"])
        n, tot = agg.get(key, (0, 0.0))
        agg[key] = (n + 1, tot + float(r["Counter_Value"]))
    if not agg:
        return
    mean = {k: tot / n for k, (n, tot) in agg.items()}
    print("\n| kernel | grid (threads) | counter | dispatches | mean per dispatch (FETCH_SIZE / WRITE_SIZE in KiB) |")
    print("|---|---|---|---|---|")
    for (k, grid, c), (n, tot) in sorted(agg.items()):
        print(f"| `{k}` | {grid} | {c} | {n} | {tot / n:.1f} |")
    scale = {}
    for (k, grid, c), v in mean.items():
        if COPY_KERNEL[0] in k and grid == COPY_KERNEL[1] and v > 0:
            known = COPY_KERNEL[2] if c == "FETCH_SIZE" else COPY_KERNEL[3]
            scale[c] = known / (v * 1024)
    for c, f in sorted(scale.items()):
        print(f"\ncalibration {c}: x{f:.4f} (copy kernel moving 1 GiB each way)")
    sized = sorted({(k, g) for (k, g, c) in agg if c in scale})
    if sized:
        print("\n| kernel | grid (threads) | calibrated read MB / dispatch | calibrated write MB / dispatch |")
        print("|---|---|---|---|")
        for k, g in sized:
            cols = []
            for c in ("FETCH_SIZE", "WRITE_SIZE"):
                v = mean.get((k, g, c))
                cols.append("-" if v is None or c not in scale else f"{v * 1024 * scale[c] / 1e6:.2f}")
            print(f"| `{k}` | {g} | {cols[0]} | {cols[1]} |")
    mops = [key for key in agg if key[2].startswith("SQ_INSTS_VALU_MFMA_MOPS_")]
    if mops:
        # MOPS counters count MFMA multiply/add operations / 512, summed over the chip
        print("\n| kernel | grid (threads) | counter | MFMA GFLOP / dispatch |")
        print("|---|---|---|---|")
        for k, g, c in sorted(mops):
            print(f"| `{k}` | {g} | {c} | {mean[(k, g, c)] * 512 / 1e9:.3f} |")
    util = sorted(key for key in agg if key[2] == "MfmaUtil")
    if util:
        print("\n| kernel | grid (threads) | MfmaUtil % (MFMA busy cycles / (GPU active cycles x SIMDs)) |")
        print("|---|---|---|")
        for k, g, c in util:
            print(f"| `{k}` | {g} | {mean[(k, g, c)]:.2f} |")
    if set(scale) == {"FETCH_SIZE", "WRITE_SIZE"}:
        # calls = dispatches of the main kernel; merge dispatches (if any) add to the same calls
        main = [(k, g) for (k, g, c) in agg if k.startswith(ROOFLINE_KERNELS[0]) and c == "FETCH_SIZE"]
        if not main:
            return
        calls = sum(agg[(k, g, "FETCH_SIZE")][0] for k, g in main)
        total = 0.0
        for (k, g, c), (n, tot) in sorted(agg.items()):
            if k.startswith(ROOFLINE_KERNELS) and c in scale:
                b = tot * 1024 * scale[c] / calls
                print(f"{k} (grid {g}) {c}: {b / 1e6:.1f} MB per call (calibrated, {n} dispatches)")
                total += b
        print(f"traffic_bytes_per_call: {total:.0f}")


def cpu_baseline(torch, dec, steps):
    """The reference's step on the host cores, checked against the GPU step it shadows.

    For each of `steps` steps (the first half at torch's default thread count, i.e. every core
    this process may use, the rest at 8 threads, the reference's OMP_NUM_THREADS), the GPU runs
    one eager step from the decoder's state and oracle.spec_step runs the same step on the
    host from a copy of that state and the same row of the uniform table: the reference's
    engine step (engine/engine.py:338-470) with a bf16 torch-CPU Llama, INT8 KV quantised on
    write, fp32 paged attention and explicit-uniform sampling, teacher-forced on the GPU's
    logits so that every decision is compared (oracle.step_check).  Reported: tokens emitted
    per second of oracle step time at each thread count, and the agreement counts."""
    from oracle.step_check import StepChecker

    t0 = time.perf_counter()
    chk = StepChecker(dec, logit_tol=None, kv_tol=None)   # differences reported
    log(f"cpu baseline: weights copied to host in {time.perf_counter() - t0:.1f}s")
    n_all = torch.get_num_threads()
    legs = {"all_cores": [0, 0.0, n_all], "threads_8": [0, 0.0, 8]}
    for i in range(steps):
        leg = "all_cores" if i < (steps + 1) // 2 else "threads_8"
        torch.set_num_threads(legs[leg][2])
        chk.before()
        dec.step()
        torch.cuda.synchronize()
        e0 = sum(len(s.tokens) for s in chk.seqs)
        secs = chk.after()
        legs[leg][0] += sum(len(s.tokens) for s in chk.seqs) - e0
        legs[leg][1] += secs
        log(f"cpu baseline step {i} ({legs[leg][2]} threads): {secs:.2f}s")
    torch.set_num_threads(n_all)
    agree = chk.summary()
    v = {k: (toks / secs if secs else None) for k, (toks, secs, _) in legs.items()}
    return {"value": v["all_cores"], "unit": "tokens/s", "cores": n_all, "kind": "port",
            "sample": f"{steps} speculative steps of the same B={dec.B}, gamma={dec.g} batch "
                      f"from the GPU run's state ({(steps + 1) // 2} at {n_all} threads, the rest "
                      f"at 8): oracle.spec_step on the host (bf16 torch-CPU Llama, INT8 KV "
                      f"quantised on write, fp32 paged attention, explicit-uniform sampling), "
                      f"each step checked against the GPU step from the same state",
            "seconds": legs["all_cores"][1], "affinity_cores": len(os.sched_getaffinity(0)),
            "threads_8": {"value": v["threads_8"], "seconds": legs["threads_8"][1]},
            "agreement": agree}


def run_step_bench(torch, dec, steps, warmup, tune):
    """Prefilled decoder -> (seconds over `steps` graph replays, emitted, drafted, accepted)."""
    dev = dec.hist.device
    if tune:
        # Pick the hipBLASLt/rocBLAS solution of each decode-shape GEMM by timing (PyTorch
        # TunableOp), during an eager step, i.e. after prefill and before capture.
        t0 = time.perf_counter()
        torch.cuda.tunable.enable(True)
        torch.cuda.tunable.tuning_enable(True)
        torch.cuda.tunable.set_max_tuning_duration(50)
        torch.cuda.tunable.set_filename(os.path.join(os.environ.get("TMPDIR", "/tmp"),
                                                     "coopt_tunableop_%d.csv"))
        dec.step()
        torch.cuda.synchronize(dev)
        torch.cuda.tunable.tuning_enable(False)
        log(f"GEMM tuning step in {time.perf_counter() - t0:.1f}s")
    dec.step()                       # eager warm-up (allocates workspaces)
    dec.capture()                    # one HIP graph for the step's bucket
    for _ in range(warmup):
        dec.replay()
    torch.cuda.synchronize(dev)
    e0, d0, a0 = int(dec.emitted), int(dec.drafted), int(dec.accepted)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1)  # marker kernel (spin_kernel) bracketing the timed steps in traces
    start.record()
    for _ in range(steps):
        dec.replay()
    end.record()
    torch.cuda._sleep(1)
    torch.cuda.synchronize(dev)
    secs = start.elapsed_time(end) * 1e-3
    return secs, int(dec.emitted) - e0, int(dec.drafted) - d0, int(dec.accepted) - a0


def main():
    args = parse()
    if args.summarize:
        summarize(args.summarize)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported in this "
              "build (the path runs on a single MI355X; see DESIGN.md for how it would shard)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import iitj_llm_coopt_amd as M
    from iitj_llm_coopt_amd.spec_engine import (DRAFT_LLAMA32_1B, TARGET_LLAMA31_8B, RandomLlama,
                                                SpecDecoder)

    dev = torch.device("cuda:0")
    torch.manual_seed(args.seed)
    CPU_LEGS["on"] = not args.no_cpu
    if args.kernels_only:
        names = args.case or sorted(KERNEL_CASES)
        print(json.dumps(run_kernel_cases(torch, M, dev, names, args.seed)), flush=True)
        return
    B, g, P = args.batch, args.gamma, args.prompt
    t0 = time.perf_counter()
    target = RandomLlama(TARGET_LLAMA31_8B, dev, seed=args.seed + 1)
    draft = RandomLlama(DRAFT_LLAMA32_1B, dev, seed=args.seed + 2,
                        packed=("qkv", "o", "gate_up", "down", "lm_head"))  # 32 / 64 rows only
    log(f"weights ready in {time.perf_counter() - t0:.1f}s")
    dec = SpecDecoder(target, draft, B, g, P, max_steps=args.warmup + args.steps + 2 + args.cpu_steps,
                      temperature=args.temperature, seed=args.seed)
    gen = torch.Generator(device=dev).manual_seed(args.seed + 3)
    prompts = torch.randint(0, TARGET_LLAMA31_8B.vocab, (B, P), generator=gen, device=dev)
    t0 = time.perf_counter()
    dec.prefill(prompts, torch.rand(B, generator=gen, device=dev))
    log(f"prefill of {B}x{P} tokens in {time.perf_counter() - t0:.1f}s")

    tuned = not args.no_tune_gemm
    secs, emitted, drafted, accepted = run_step_bench(torch, dec, args.steps, args.warmup, tuned)
    acc_rate = accepted / max(1, drafted)
    log(f"{args.steps} steps in {secs * 1e3:.1f} ms: {emitted} tokens, acceptance {acc_rate:.3f}")

    b16 = None
    if args.b16_steps and B != 16:
        # config 5 as stated (B=16): a second decoder over the same weights
        d16 = SpecDecoder(target, draft, 16, g, P, max_steps=args.warmup + args.b16_steps + 2,
                          temperature=args.temperature, seed=args.seed)
        d16.prefill(prompts[:16], torch.rand(16, generator=gen, device=dev))
        s16, e16, dr16, a16 = run_step_bench(torch, d16, args.b16_steps, args.warmup, False)
        b16 = {"batch": 16, "steps": args.b16_steps, "ms_per_step": s16 / args.b16_steps * 1e3,
               "tokens_per_s": e16 / s16, "scored_positions_per_s": 16 * (g + 1) * args.b16_steps / s16,
               "acceptance_rate": a16 / max(1, dr16)}
        log(f"B=16: {b16['ms_per_step']:.2f} ms/step, {b16['tokens_per_s']:.0f} tokens/s")
        del d16
        torch.cuda.empty_cache()

    # kernel-level measurements (HIP events per call, torch's current stream)
    kern, att_i8 = {}, None
    if not args.no_kernel_cases:
        kern = run_kernel_cases(torch, M, dev, sorted(KERNEL_CASES), args.seed)
        att_i8 = kern["attention_int8"]

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, dec, args.cpu_steps)
        log(f"cpu baseline {cpu['value']:.2f} tokens/s on {cpu['cores']} threads, "
            f"{cpu['threads_8']['value']:.2f} on 8; agreement {cpu['agreement']}")

    out = {
        "metric": METRIC,
        "value": emitted / secs,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": secs / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights (N(0, 0.02^2)), seeded uniform prompt ids",
        "config": {"workload": "config 5 speculative step at the metric's B: draft Llama-3.2-1B "
                               "shape (bf16 paged KV) proposes gamma, target Llama-3.1-8B shape "
                               "(INT8 paged KV) verifies gamma+1, fused accept; one HIP graph "
                               "per step",
                   "global_batch": B, "seq_len": P, "gamma": g,
                   "temperature": args.temperature, "block_size": 16,
                   "gemm_selection": "PyTorch TunableOp" if tuned else "default",
                   "parallelism": "single GPU"},
        "roofline": None if att_i8 is None else {"bound": "hbm", "achieved": att_i8["GB_s"], "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": att_i8["frac"], "traffic": committed_traffic(),
                     "kernel": "coopt_verify_attention, INT8 KV, B=32, q_len 5, 8192 cached "
                               "tokens (one block per sequence and KV head at this shape, so "
                               "no split-merge launch)",
                     "bytes_per_launch": att_i8["bytes"], "avg_launch_us": att_i8["avg_us"],
                     "traffic_source": "profiles/verify_attention_int8_b32_ctx8192.md "
                                       "(rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
                     "frac_by_cache_layout": layout_fracs(kern)},
        "cpu_baseline": cpu,
        "acceptance_rate": acc_rate,
        "tokens_per_step": emitted / args.steps,
        "scored_positions_per_s": B * (g + 1) * args.steps / secs,
        "config5_b16": b16,
        "kernels": kern,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
