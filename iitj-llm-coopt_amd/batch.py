"""Varlen batch packing: the layout contract between the scheduler and the kernels.

Mirrors engine/batch.py:15-55 and the Batch record of engine/model.py:54-65
(mohsinmubarak/iitj-llm-coopt).  A work item appends `tokens` to sequence `seq_id` at positions
[start, start + len(tokens)); verification items ([last token] + drafts) ask for logits at
every new position, decode/prefill items only at the last one.

`build_padded_batch` is the fixed-shape layout of engine/cuda_graphs.py:7-16, 76-104: item i
owns rows [i*S, (i+1)*S), its real tokens first; seq_len = start + S; padding rows write to a
scratch slot, so with the bottom-right causal mask real query j still sees keys
[0, start + j] and padding never changes real outputs.
"""
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .block_manager import BlockManager

__all__ = ["WorkItem", "Batch", "build_batch", "build_padded_batch", "row_slots"]


@dataclass
class WorkItem:
    seq_id: int
    tokens: list
    start: int
    all_logits: bool = False


@dataclass
class Batch:
    """Flattened inputs of one forward step (device tensors)."""
    input_ids: torch.Tensor       # [T] int64, new tokens back to back
    positions: torch.Tensor       # [T] int64
    cu_seqlens_q: torch.Tensor    # [B+1] int32, row offsets of each sequence
    seq_lens: torch.Tensor        # [B] int32, cached + new tokens per sequence
    block_table: torch.Tensor     # [B, W] int32
    slot_mapping: torch.Tensor    # [T] int64, cache slot of each new token
    logits_indices: torch.Tensor  # [N] int64, rows that need logits
    max_seqlen_q: int
    max_seqlen_k: int


def _to(x: np.ndarray, dtype, device):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dtype)
    if torch.device(device).type == "cuda":
        t = t.pin_memory().to(device, non_blocking=True)
    return t


def build_batch(items, bm: BlockManager, device="cuda", block_table_width=None):
    """Allocates blocks for the new tokens; returns (Batch, [(first logits row, rows)])."""
    ids, pos, slots, rows, spans, cu, lens = [], [], [], [], [], [0], []
    for it in items:
        n = len(it.tokens)
        end = it.start + n
        bm.ensure(it.seq_id, end)
        ids.extend(int(t) for t in it.tokens)
        pos.append(np.arange(it.start, end, dtype=np.int64))
        slots.append(bm.slot_mapping(it.seq_id, it.start, end).numpy())
        off = cu[-1]
        if it.all_logits:
            spans.append((len(rows), n))
            rows.extend(range(off, off + n))
        else:
            spans.append((len(rows), 1))
            rows.append(off + n - 1)
        cu.append(off + n)
        lens.append(end)
    table = bm.block_table_tensor([it.seq_id for it in items], block_table_width).numpy()
    batch = Batch(
        input_ids=_to(np.asarray(ids, np.int64), torch.int64, device),
        positions=_to(np.concatenate(pos) if pos else np.zeros(0, np.int64), torch.int64, device),
        cu_seqlens_q=_to(np.asarray(cu, np.int32), torch.int32, device),
        seq_lens=_to(np.asarray(lens, np.int32), torch.int32, device),
        block_table=_to(table, torch.int32, device),
        slot_mapping=_to(np.concatenate(slots) if slots else np.zeros(0, np.int64), torch.int64,
                         device),
        logits_indices=_to(np.asarray(rows, np.int64), torch.int64, device),
        max_seqlen_q=max((len(it.tokens) for it in items), default=0),
        max_seqlen_k=max(lens, default=0),
    )
    return batch, spans


def build_padded_batch(items, bm: BlockManager, stride: int, batch_size: int, width: int,
                       scratch_slot: int, device="cuda"):
    """Fixed-shape layout for graph replay (engine/cuda_graphs.py:76-104 semantics).

    `batch_size` >= len(items) rows of `stride` >= every item's token count; dummy sequences
    have seq_len = stride and scratch slots.  Returns (Batch, spans) with spans like
    build_batch's: verification items get logits rows [i*S, i*S + n).
    """
    S, Bp, bs = stride, batch_size, bm.block_size
    if len(items) > Bp or any(len(it.tokens) > S for it in items):
        raise ValueError("items do not fit the padded shape")
    T = Bp * S
    ids = np.zeros(T, np.int64)
    pos = np.tile(np.arange(S, dtype=np.int64), Bp)
    slots = np.full(T, scratch_slot, np.int64)
    lens = np.full(Bp, S, np.int32)
    table = np.zeros((Bp, width), np.int32)
    spans = []
    for i, it in enumerate(items):
        n, base = len(it.tokens), i * S
        bm.ensure(it.seq_id, it.start + n)
        t = bm.tables[it.seq_id]
        table[i, :len(t)] = t
        ids[base:base + n] = it.tokens
        pos[base:base + S] += it.start
        p = np.arange(it.start, it.start + n)
        slots[base:base + n] = table[i, p // bs].astype(np.int64) * bs + p % bs
        lens[i] = it.start + S
        spans.append((base, n) if it.all_logits else (base + n - 1, 1))
    batch = Batch(
        input_ids=_to(ids, torch.int64, device), positions=_to(pos, torch.int64, device),
        cu_seqlens_q=_to(np.arange(Bp + 1, dtype=np.int32) * S, torch.int32, device),
        seq_lens=_to(lens, torch.int32, device), block_table=_to(table, torch.int32, device),
        slot_mapping=_to(slots, torch.int64, device),
        logits_indices=_to(np.arange(T, dtype=np.int64), torch.int64, device),
        max_seqlen_q=S, max_seqlen_k=int(lens.max()) if Bp else 0)
    return batch, spans


def row_slots(block_table, start, S: int, block_size: int, n_real=None):
    """Device-side paged addressing of S rows per sequence at positions start[b] + j
    (coopt_row_slots): returns positions [B, S] int64, slots [B*S] int64 -- the
    BlockManager.slot_mapping formula (engine/block_manager.py:216-220), -1 for rows
    j >= n_real[b] and for positions past the table -- and seq_lens [B] int32 = start + S.
    block_table [B, W] int32 and start / n_real [B] int64 on the GPU; one launch."""
    _lib.require_cuda(block_table, start, n_real)
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(-1) != 1:
        raise ValueError("block_table must be an int32 [B, W] tensor with contiguous rows")
    B = start.numel()
    if start.dtype != torch.int64 or not start.is_contiguous() or block_table.shape[0] < B:
        raise ValueError("start must be a contiguous int64 [B] tensor, B <= block_table rows")
    if n_real is not None and (n_real.dtype != torch.int64 or not n_real.is_contiguous()
                               or n_real.numel() != B):
        raise ValueError("n_real must be a contiguous int64 [B] tensor")
    dev = start.device
    pos = torch.empty((B, S), dtype=torch.int64, device=dev)
    slots = torch.empty(B * S, dtype=torch.int64, device=dev)
    seq_lens = torch.empty(B, dtype=torch.int32, device=dev)
    _lib.check(_lib.load().coopt_row_slots(
        _lib.ptr(block_table), block_table.stride(0), block_table.shape[1], _lib.ptr(start),
        None if n_real is None else _lib.ptr(n_real), B, S, block_size, _lib.ptr(pos),
        _lib.ptr(slots), _lib.ptr(seq_lens), _lib.stream_handle(dev)), "coopt_row_slots")
    return pos, slots, seq_lens
