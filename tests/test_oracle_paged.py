"""CPU: host-side paged-KV contract (product BlockManager / build_batch) and oracle.paged.

The block-manager tests port tests/test_units.py:19-37 of the reference; the attention tests
pin the oracle with closed forms and a brute-force loop.
"""
import numpy as np
import pytest
import torch

from iitj_llm_coopt_amd import BlockManager, OutOfBlocks, WorkItem, build_batch, build_padded_batch
from oracle import paged


# ---- reference known-answer tests (tests/test_units.py:19-37) ---------------------------------
def test_alloc_slots_truncate_free():
    bm = BlockManager(num_blocks=8, block_size=16)
    bm.ensure(1, 20)
    assert len(bm.tables[1]) == 2 and bm.num_free == 6
    b0, b1 = bm.tables[1]
    assert bm.slot_mapping(1, 14, 18).tolist() == [b0 * 16 + 14, b0 * 16 + 15, b1 * 16, b1 * 16 + 1]
    bm.ensure(1, 33)
    bm.truncate(1, 16)
    assert len(bm.tables[1]) == 1 and bm.num_free == 7
    assert bm.free(1) == 1 and bm.num_free == 8


def test_out_of_blocks():
    bm = BlockManager(num_blocks=2, block_size=16)
    bm.ensure(1, 32)
    assert not bm.can_fit(2, 1)
    with pytest.raises(OutOfBlocks):
        bm.ensure(2, 1)


# ---- slot mapping / block tables vs the closed form -------------------------------------------
def test_slot_mapping_matches_closed_form_on_permuted_pool():
    rng = np.random.default_rng(0)
    order = rng.permutation(4096)
    bm = BlockManager(4096, 16, free_order=order)
    lens = rng.integers(1, 900, size=40)
    for s, n in enumerate(lens):
        bm.ensure(s, int(n))
    for s, n in enumerate(lens):
        a, b = sorted(rng.integers(0, int(n) + 1, size=2))
        got = bm.slot_mapping(s, int(a), int(b)).numpy()
        assert np.array_equal(got, paged.slot_mapping(bm.tables[s], int(a), int(b), 16))
    # blocks come out in the given order and no block is handed out twice
    flat = [b for s in range(len(lens)) for b in bm.tables[s]]
    assert flat == list(order[:len(flat)]) and len(set(flat)) == len(flat)
    bt = bm.block_table_tensor(list(range(len(lens)))).numpy()
    assert np.array_equal(bt, paged.block_table([bm.tables[s] for s in range(len(lens))]))


def test_free_order_must_be_a_permutation():
    with pytest.raises(ValueError):
        BlockManager(4, 16, free_order=[0, 1, 1, 2])


def test_build_batch_layout_for_verify_items():
    bm = BlockManager(64, 16)
    items = [WorkItem(0, [5, 6, 7], 30, all_logits=True), WorkItem(1, [9], 3),
             WorkItem(2, list(range(20)), 0)]
    batch, spans = build_batch(items, bm, device="cpu")
    assert batch.cu_seqlens_q.tolist() == [0, 3, 4, 24]
    assert batch.seq_lens.tolist() == [33, 4, 20]
    assert batch.positions[:4].tolist() == [30, 31, 32, 3]
    assert batch.logits_indices.tolist() == [0, 1, 2, 3, 23]
    assert spans == [(0, 3), (3, 1), (4, 1)]
    assert batch.max_seqlen_q == 20 and batch.max_seqlen_k == 33
    exp = np.concatenate([paged.slot_mapping(bm.tables[0], 30, 33, 16),
                          paged.slot_mapping(bm.tables[1], 3, 4, 16),
                          paged.slot_mapping(bm.tables[2], 0, 20, 16)])
    assert np.array_equal(batch.slot_mapping.numpy(), exp)
    assert batch.block_table.dtype == torch.int32 and batch.cu_seqlens_q.dtype == torch.int32


def test_padded_layout_semantics():
    """engine/cuda_graphs.py:7-16: rows i*S.., seq_len = start + S, padding -> scratch slot."""
    bm = BlockManager(64, 16)
    scratch = 63 * 16
    items = [WorkItem(0, [1, 2], 10, all_logits=True), WorkItem(1, [3], 40)]
    batch, spans = build_padded_batch(items, bm, stride=5, batch_size=4, width=8,
                                      scratch_slot=scratch, device="cpu")
    assert batch.cu_seqlens_q.tolist() == [0, 5, 10, 15, 20]
    assert batch.seq_lens.tolist() == [15, 45, 5, 5]
    sm = batch.slot_mapping.numpy()
    assert (sm[2:5] == scratch).all() and (sm[6:] == scratch).all()
    assert sm[0] == paged.slot_mapping(bm.tables[0], 10, 11, 16)[0]
    assert batch.positions[:5].tolist() == [10, 11, 12, 13, 14]
    assert spans == [(0, 2), (5, 1)]


# ---- oracle attention -------------------------------------------------------------------------
def _random_paged(rng, B, Hq, Hkv, D, lens, qlens, bs=16, nb=None):
    nb = nb or sum(-(-L // bs) for L in lens) + 3
    kc = rng.standard_normal((nb, bs, Hkv, D)).astype(np.float32)
    vc = rng.standard_normal((nb, bs, Hkv, D)).astype(np.float32)
    perm = rng.permutation(nb)
    tables, o = [], 0
    for L in lens:
        nbk = -(-L // bs)
        tables.append(list(perm[o:o + nbk]))
        o += nbk
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    q = rng.standard_normal((int(cu[-1]), Hq, D)).astype(np.float32)
    return q, kc, vc, cu, np.asarray(lens, np.int32), paged.block_table(tables)


def test_attention_matches_brute_force_loop():
    rng = np.random.default_rng(3)
    Hq, Hkv, D = 8, 2, 16
    lens, qlens = [37, 5, 70], [1, 3, 5]
    q, kc, vc, cu, sl, bt = _random_paged(rng, 3, Hq, Hkv, D, lens, qlens)
    out = paged.attention(q, kc, vc, cu, sl, bt, 16, scale=0.3)
    for b in range(3):
        n, L = qlens[b], lens[b]
        K = paged.gather(kc, bt[b], L, 16)
        V = paged.gather(vc, bt[b], L, 16)
        for j in range(n):
            t = cu[b] + j
            for h in range(Hq):
                kv = h // (Hq // Hkv)
                vis = L - n + j + 1
                s = [0.3 * float(np.dot(q[t, h].astype(np.float64), K[i, kv].astype(np.float64)))
                     for i in range(vis)]
                m = max(s)
                w = [np.exp(x - m) for x in s]
                ref = sum(wi * V[i, kv].astype(np.float64) for i, wi in enumerate(w)) / sum(w)
                assert np.allclose(out[t, h], ref, atol=1e-9)


def test_attention_single_visible_key_returns_that_value():
    rng = np.random.default_rng(4)
    q, kc, vc, cu, sl, bt = _random_paged(rng, 1, 4, 1, 8, [1], [1])
    out = paged.attention(q, kc, vc, cu, sl, bt, 16)
    assert np.allclose(out[0, :], vc[bt[0][0], 0, 0][None, :])


def test_attention_equal_scores_average_the_visible_values():
    rng = np.random.default_rng(5)
    q, kc, vc, cu, sl, bt = _random_paged(rng, 1, 2, 1, 8, [20], [4])
    q[:] = 0.0  # all scores equal -> uniform weights over the causal window
    out = paged.attention(q, kc, vc, cu, sl, bt, 16)
    V = paged.gather(vc, bt[0], 20, 16)[:, 0]
    for j in range(4):
        assert np.allclose(out[j, 0], V[: 20 - 4 + j + 1].mean(0))


def test_strided_block_major_view_equals_contiguous():
    """tests/strided_kv_check.py: a per-layer view of [NB, L, 2, bs, H, D] reads the same."""
    rng = np.random.default_rng(6)
    NB, Lyr, bs, Hkv, Hq, D = 64, 4, 16, 8, 32, 32
    buf = rng.standard_normal((NB, Lyr, 2, bs, Hkv, D)).astype(np.float32)
    ks, vs = buf[:, 2, 0], buf[:, 2, 1]
    lens, qlens = [37, 200, 5], [1, 3, 5]
    cu = np.array([0, 1, 4, 9], np.int32)
    bt = rng.permutation(NB)[:48].reshape(3, 16).astype(np.int32)
    q = rng.standard_normal((9, Hq, D)).astype(np.float32)
    a = paged.attention(q, np.ascontiguousarray(ks), np.ascontiguousarray(vs), cu, lens, bt, bs)
    b = paged.attention(q, ks, vs, cu, lens, bt, bs)
    assert np.array_equal(a, b)


def test_kv_write_index_put_and_no_leak_into_other_layers():
    rng = np.random.default_rng(7)
    NB, Lyr, bs, H, D, T = 64, 4, 16, 8, 16, 37
    buf = np.zeros((NB, Lyr, 2, bs, H, D), np.float32)
    kc, vc = buf[:, 2, 0], buf[:, 2, 1]
    slots = rng.permutation(NB * bs)[:T]
    k = rng.standard_normal((T, H, D)).astype(np.float32)
    v = rng.standard_normal((T, H, D)).astype(np.float32)
    paged.kv_write(kc, vc, k, v, slots, bs)
    assert np.array_equal(kc[slots // bs, slots % bs], k)
    assert np.array_equal(vc[slots // bs, slots % bs], v)
    others = np.concatenate([buf[:, l] for l in range(Lyr) if l != 2])
    assert (others == 0).all()


def test_tier_manager_accounting_matches_reference_formula():
    """engine/kv_tier_manager.py:67-82 without a GPU: estimate_bytes for the Llama-3.1-8B
    geometry (32 layers, 8 KV heads, head_dim 128), capacity, hit rate, and the early
    refusals of swap_out (nothing computed; does not fit)."""
    import types

    torch = pytest.importorskip("torch")
    from iitj_llm_coopt_amd.kv_tier import KVTierManager

    cfg = types.SimpleNamespace(num_hidden_layers=32, num_key_value_heads=8, head_dim=128)
    e = types.SimpleNamespace(target=types.SimpleNamespace(cfg=cfg, k_cache=[], v_cache=[]), bm=None)
    tm = KVTierManager(e, cpu_gb=1.0, bits=8)
    assert e.kv_tiers is tm
    per_tok8 = 2 * 32 * 8 * 128          # bytes of codes per token at 8 bits
    assert tm.estimate_bytes(1000, 8) == int(per_tok8 * 1000 * (1 + 2 / 128))
    assert tm.estimate_bytes(1000, 16) == 2 * per_tok8 * 1000
    assert tm.estimate_bytes(1000, 4) == int(per_tok8 / 2 * 1000 * (1 + 2 / 128))
    assert tm.cpu_usage == 0.0 and tm.hit_rate == 0.0
    tm.note_recompute()
    assert tm.hit_rate == 0.0 and tm.recomputes == 1
    seq = types.SimpleNamespace(seq_id=1, num_computed=0)
    assert tm.swap_out(seq) is False      # nothing computed
    tm.capacity = 10
    seq.num_computed = 5
    assert tm.swap_out(seq) is False      # does not fit (checked before touching the GPU)
    tm.drop(99)                           # unknown ids are ignored
    with pytest.raises(ValueError):
        KVTierManager(e, bits=3)


def test_swap_oracle_is_gather_then_codec():
    rng = np.random.default_rng(4)
    cache = rng.standard_normal((6, 16, 2, 32)).astype(np.float32)
    blocks = np.array([4, -1, 0])
    q, s = paged.swap_out(cache, blocks, 8)
    from oracle import codec as OC
    q0, s0 = OC.quantize(cache[4], 8)
    assert np.array_equal(q[0], q0) and np.array_equal(s[0], s0)
    assert np.all(q[1] == 0) and np.all(s[1] == 0)
    x, none = paged.swap_out(cache, blocks, 16)
    assert none is None and np.array_equal(x[2], cache[0])
    back = paged.swap_in(q, s, 8)
    assert np.allclose(back[0], cache[4], atol=np.abs(cache[4]).max() / 127)


# ---- elastic pool: add / migrate / withdraw (engine/block_manager.py:159-213) ---------------
def _tail_scenario():
    bm = BlockManager(num_blocks=4, block_size=16)
    bm.add_blocks([4, 5])
    bm.ensure(1, 48)
    bm.ensure(2, 32)
    bm.free(1)
    return bm


def test_migrate_known_answer():
    # free [5, 0, 1, 2], tables {2: [3, 4]}: block 4 moves to the first free block outside
    # {4, 5}, i.e. 0; the source joins the end of the free list; 5 and 4 are then withdrawn.
    bm = _tail_scenario()
    assert bm.num_blocks == 6 and list(bm.free_blocks) == [5, 0, 1, 2] and bm.tables == {2: [3, 4]}
    pairs = []
    assert bm.migrate_out_of({4, 5}, lambda s, d: pairs.append((s, d))) == 1
    assert pairs == [(4, 0)] and bm.tables == {2: [3, 0]} and list(bm.free_blocks) == [5, 1, 2, 4]
    bm.withdraw_free({4, 5})
    assert bm.num_blocks == 4 and list(bm.free_blocks) == [1, 2]
    got = paged.migrate({2: [3, 4]}, [5, 0, 1, 2], {4, 5})
    assert got == ([(4, 0)], {2: [3, 0]}, [5, 1, 2, 4])


def test_migrate_without_room_changes_nothing():
    bm = BlockManager(num_blocks=4, block_size=16)
    bm.add_blocks([4, 5])
    bm.ensure(1, 96)                       # all six blocks, two of them in {4, 5}
    before = (dict((k, list(v)) for k, v in bm.tables.items()), list(bm.free_blocks))
    assert bm.migrate_out_of({4, 5}, lambda s, d: pytest.fail("no copy expected")) == -1
    assert (bm.tables, list(bm.free_blocks)) == before
    assert paged.migrate(bm.tables, bm.free_blocks, {4, 5}) is None
    with pytest.raises(OutOfBlocks):
        bm.withdraw_free({4, 5})
    assert (bm.tables, list(bm.free_blocks), bm.num_blocks) == (before[0], before[1], 6)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_migrate_invariants_and_oracle_agree(seed):
    """Random pools: the product and the restatement agree, and both keep every table reading
    the same KV (content[dst] = content[src]) with no table left in the migrated set."""
    rng = np.random.default_rng(seed)
    base, tail = 64, 24
    bm = BlockManager(base, 16, free_order=rng.permutation(base))
    bm.add_blocks(rng.permutation(np.arange(base, base + tail)).tolist())
    for sid in range(12):
        bm.ensure(sid, int(rng.integers(1, 7 * 16)))
    for sid in rng.choice(12, 5, replace=False):
        bm.free(int(sid))
    ids = set(range(base, base + tail))
    tables0 = {k: list(v) for k, v in bm.tables.items()}
    free0 = list(bm.free_blocks)
    content = np.arange(base + tail) * 7 + 3          # a distinct payload per block
    pairs = []

    def copy(s, d):
        pairs.append((s, d))
        content[d] = content[s]

    moved = bm.migrate_out_of(ids, copy)
    want = paged.migrate(tables0, free0, ids)
    if want is None:
        assert moved == -1
        return
    assert moved == len(want[0]) and pairs == want[0]
    assert bm.tables == want[1] and list(bm.free_blocks) == want[2]
    assert all(s in ids and d not in ids for s, d in pairs)
    assert len({d for _, d in pairs}) == len(pairs)
    assert not any(b in ids for t in bm.tables.values() for b in t)
    for sid, t in bm.tables.items():
        assert [content[b] for b in t] == [(b * 7 + 3) for b in tables0[sid]]
    n_before = bm.num_blocks
    bm.withdraw_free(ids)
    assert bm.num_blocks == n_before - tail and bm.num_free + sum(map(len, bm.tables.values())) == base


def test_copy_blocks_oracle_is_fancy_indexing_for_disjoint_pairs():
    rng = np.random.default_rng(5)
    a = rng.standard_normal((40, 3, 4)).astype(np.float32)
    b = rng.integers(-128, 127, size=(40, 6)).astype(np.int8)
    src = rng.choice(20, 9, replace=False)
    dst = 20 + rng.choice(20, 9, replace=False)
    got = paged.copy_blocks([a, b], list(zip(src, dst)))
    for x, y in zip([a, b], got):
        want = x.copy()
        want[dst] = x[src]
        assert np.array_equal(y, want)


def test_block_region_of_cache_layouts():
    from iitj_llm_coopt_amd.kv_blocks import block_region

    NB, L, bs, H, D = 6, 3, 16, 8, 128
    buf = torch.empty((NB, L, 2, bs, H, D), dtype=torch.bfloat16)
    base, stride, per = block_region(buf)
    assert (stride, per) == (L * 2 * bs * H * D * 2,) * 2
    base, stride, per = block_region(buf[:, 1, 0])
    assert base == buf.data_ptr() + (2 * bs * H * D) * 2 and stride == L * 2 * bs * H * D * 2
    assert per == bs * H * D * 2
    hm = torch.empty((NB, H, bs, D), dtype=torch.int8).permute(0, 2, 1, 3)   # head-major view
    assert block_region(hm)[1:] == (H * bs * D, H * bs * D)
    sc = torch.empty((NB, H, bs), dtype=torch.float16).permute(0, 2, 1)
    assert block_region(sc)[1:] == (H * bs * 2, H * bs * 2)
    with pytest.raises(ValueError):
        block_region(buf[:, :, 0, :8])                # half the tokens of each block
