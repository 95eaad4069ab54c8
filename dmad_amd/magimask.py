"""Block-sparse attention masks as range tables (MagiMask) for the masked JVP forward.

Host-side construction of what the block-sparse kernel reads, with the
reference's names and semantics:

* ``BlockPattern`` / ``AttnMaskSpec`` -- the block schedule of a causal video
  student: block 0 holds ``first_chunk_frames`` frames, every later block
  ``chunk_frames`` frames of ``frame_tokens`` tokens
  (train/wan/rcm/utils/blockmask.py:71-189).
* ``make_magi_ranges_full`` -- the mask as a list of full rectangles
  ``(q_range, k_range)`` for the "block_causal" and "teacher_forcing" modes
  (magimask.py:10-124).
* ``merge_k_ranges`` -- rows with the same query range: key ranges clipped,
  sorted and merged (magimask.py:127-184).
* ``group_q_ranges_csr`` -- consecutive equal query ranges -> CSR
  ``(q_unique, k_flat, qk_map)`` (magimask.py:187-213).
* ``build_qtile_tasks`` -- one task per (group, BLOCK_M-query tile) pair that
  intersect (magimask.py:216-245).
* ``MagiMask`` / ``prepare_magi_csr_and_tasks`` -- the bundle the op takes
  (magimask.py:248-283).

The kernels' query tile is ``BLOCK_M = 128`` rows: masks built with another
``BLOCK_M`` (the reference picks 64 on some GPUs) still work, their tasks are
rebuilt once per mask for 128-row tiles (``tasks_for_kernel``).

This is index bookkeeping on the host (numpy); the tables end up as int32
tensors on the device of the inputs.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import List, Literal, Sequence, Tuple

import numpy as np
import torch

KERNEL_BLOCK_M = 128  # query rows per task of the block-sparse kernels


@dataclass(frozen=True)
class BlockPattern:
    """Block schedule in frames: [first_chunk_frames] [chunk_frames] [chunk_frames] ...

    (train/wan/rcm/utils/blockmask.py:71-155)
    """

    frame_tokens: int = 0
    first_chunk_frames: int = 1
    chunk_frames: int = 1

    def get_block_tokens(self, block_idx: int) -> int:
        return self.block_size(block_idx) * self.frame_tokens

    def blocks_to_frames(self, num_blocks: int) -> int:
        if num_blocks <= 0:
            return 0
        return self.first_chunk_frames + (num_blocks - 1) * self.chunk_frames

    def blocks_to_tokens(self, num_blocks: int) -> int:
        return self.blocks_to_frames(num_blocks) * self.frame_tokens

    def block_size(self, block_idx: int) -> int:
        return self.first_chunk_frames if block_idx == 0 else self.chunk_frames

    def token_to_rel_block(self, token_idx: torch.Tensor, use_first_block: bool) -> torch.Tensor:
        """Block of each token; without the first block every block is chunk_frames long."""
        frame = token_idx // self.frame_tokens
        if not use_first_block:
            return frame // self.chunk_frames
        later = 1 + (frame - self.first_chunk_frames) // self.chunk_frames
        return torch.where(frame < self.first_chunk_frames, torch.zeros_like(frame), later)

    def spans(self, num_blocks: int, block_offset: int, count_tokens: bool = False) -> Tuple[List[Tuple[int, int]], int]:
        """[start, end) of num_blocks consecutive blocks from block_offset, and their total length."""
        unit = self.frame_tokens if count_tokens else 1
        out: List[Tuple[int, int]] = []
        pos = 0
        for i in range(num_blocks):
            first = block_offset == 0 and i == 0
            n = (self.first_chunk_frames if first else self.chunk_frames) * unit
            out.append((pos, pos + n))
            pos += n
        return out, pos

    def block_bounds(self, q_bo: int, Q: int) -> List[int]:
        """Token boundaries [0, ..., Q] of the query blocks from block q_bo on (the last one cut at Q)."""
        bounds = [0]
        if q_bo == 0:
            bounds.append(min(Q, self.first_chunk_frames * self.frame_tokens))
        step = self.chunk_frames * self.frame_tokens
        while bounds[-1] < Q:
            bounds.append(min(Q, bounds[-1] + step))
        return bounds


@dataclass(frozen=True)
class AttnMaskSpec:
    """Block mask spec (train/wan/rcm/utils/blockmask.py:158-186).

    mode "block_causal": key blocks <= the query block (full inside a block);
    mode "teacher_forcing": packed [clean][noisy] sequence, clean queries see
    clean blocks <= theirs, noisy queries see earlier clean blocks and their
    own noisy block. local_attn_blocks > 0 keeps only that many latest blocks
    (the query's included); sink_blocks always admits the first blocks.
    """

    mode: Literal["none", "block_causal", "teacher_forcing"] = "none"
    pattern: BlockPattern = None
    local_attn_blocks: int = 0
    sink_blocks: int = 0
    q_block_offset: int = 0
    clean_blocks: int = 0


def _block_causal_rects(spec: AttnMaskSpec, Q: int, KV: int):
    pat, q_bo = spec.pattern, spec.q_block_offset
    window = spec.local_attn_blocks - 1  # < 0: no sliding window
    bounds = pat.block_bounds(q_bo=q_bo, Q=Q)
    nblk = len(bounds) - 1
    assert bounds[-1] == Q
    assert KV == pat.blocks_to_tokens(q_bo + nblk)
    sink_end = min(KV, pat.blocks_to_tokens(spec.sink_blocks)) if spec.sink_blocks > 0 else 0
    for i in range(nblk):
        blk = q_bo + i
        hi = min(KV, pat.blocks_to_tokens(blk + 1))
        lo = pat.blocks_to_tokens(max(0, blk - window)) if window >= 0 else 0
        yield bounds[i], bounds[i + 1], lo, hi
        if sink_end > 0 and lo > 0:
            yield bounds[i], bounds[i + 1], 0, min(sink_end, hi)


def _teacher_forcing_rects(spec: AttnMaskSpec, Q: int, KV: int):
    pat, nclean = spec.pattern, spec.clean_blocks
    assert nclean > 0
    clean = pat.blocks_to_tokens(nclean)
    assert Q == 2 * clean and KV == 2 * clean, (
        f"teacher forcing packs a clean and a noisy copy: query and key lengths must both be "
        f"{2 * clean} (twice the {clean} clean tokens), got {Q} and {KV}")
    window = spec.local_attn_blocks - 1
    hb = pat.block_bounds(q_bo=0, Q=clean)
    for i in range(nclean):
        q0, q1 = hb[i], hb[i + 1]
        sink_end = min(clean, pat.blocks_to_tokens(min(spec.sink_blocks, i))) if spec.sink_blocks > 0 else 0
        lo = hb[max(0, i - window)] if window >= 0 else 0
        # clean block i: clean keys of blocks <= i
        yield q0, q1, lo, q1
        if sink_end > 0 and lo > 0:
            yield q0, q1, 0, sink_end
        # noisy block i: clean keys of blocks < i, then its own noisy block
        n0, n1 = q0 + clean, q1 + clean
        if q0 > lo:
            yield n0, n1, lo, q0
            if sink_end > 0 and lo > 0:
                yield n0, n1, 0, sink_end
        yield n0, n1, n0, n1


def make_magi_ranges_full(spec: AttnMaskSpec, Q_real: int, KV_real: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """(q_ranges, k_ranges) [R, 2] int32: the mask as a union of full rectangles
    (train/wan/rcm/utils/magimask.py:10-124)."""
    assert spec.pattern is not None
    if spec.mode == "block_causal":
        rects = list(_block_causal_rects(spec, Q_real, KV_real))
    elif spec.mode == "teacher_forcing":
        rects = list(_teacher_forcing_rects(spec, Q_real, KV_real))
    else:
        raise ValueError(f"Unsupported mode: {spec.mode}")
    arr = np.asarray(rects, dtype=np.int64).reshape(-1, 4)
    return (torch.tensor(arr[:, :2], device=device, dtype=torch.int32),
            torch.tensor(arr[:, 2:], device=device, dtype=torch.int32))


def _host(t) -> np.ndarray:
    return (t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)).astype(np.int64).reshape(-1, 2)


def merge_k_ranges(q_ranges: torch.Tensor, k_ranges: torch.Tensor, KV_real: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rows sorted by query range; per query range the key ranges clipped to
    [0, KV_real], empty ones dropped, sorted by start and merged where they
    overlap or touch (train/wan/rcm/utils/magimask.py:127-184)."""
    assert q_ranges.shape == k_ranges.shape and q_ranges.ndim == 2 and q_ranges.shape[1] == 2
    qs, ks = _host(q_ranges), _host(k_ranges)
    order = np.lexsort((qs[:, 1], qs[:, 0]))  # stable: by q0, then q1
    qs, ks = qs[order], ks[order]
    out: List[Tuple[int, int, int, int]] = []
    i = 0
    while i < len(qs):
        q0, q1 = int(qs[i, 0]), int(qs[i, 1])
        assert q0 < q1, f"query range [{q0}, {q1}) is empty or reversed"
        j = i
        while j < len(qs) and qs[j, 0] == q0 and qs[j, 1] == q1:
            j += 1
        clipped = np.clip(ks[i:j], 0, KV_real)
        segs = sorted((int(a), int(b)) for a, b in clipped if b > a)
        assert segs, f"query rows [{q0}, {q1}) have no key range inside [0, {KV_real})"
        lo, hi = segs[0]
        for a, b in segs[1:]:
            if a <= hi:
                hi = max(hi, b)
            else:
                out.append((q0, q1, lo, hi))
                lo, hi = a, b
        out.append((q0, q1, lo, hi))
        i = j
    arr = np.asarray(out, dtype=np.int64).reshape(-1, 4)
    dev = q_ranges.device
    return (torch.tensor(arr[:, :2], device=dev, dtype=torch.int32),
            torch.tensor(arr[:, 2:], device=dev, dtype=torch.int32))


def group_q_ranges_csr(q_ranges: torch.Tensor, k_ranges: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Runs of equal consecutive query ranges -> (q_unique [G,2], k_flat [R,2], qk_map [G+1])
    (train/wan/rcm/utils/magimask.py:187-213)."""
    assert q_ranges.ndim == 2 and q_ranges.shape[1] == 2 and k_ranges.shape == q_ranges.shape
    qs = _host(q_ranges)
    starts = [0] + [i for i in range(1, len(qs)) if (qs[i] != qs[i - 1]).any()]
    qk_map = np.asarray(starts + [len(qs)], dtype=np.int64)
    dev = q_ranges.device
    return (q_ranges.contiguous()[torch.as_tensor(starts, dtype=torch.long, device=dev)].contiguous(),
            k_ranges.contiguous(),
            torch.tensor(qk_map, device=dev, dtype=torch.int32))


def _tasks(qu: np.ndarray, Q_real: int, block_m: int) -> Tuple[np.ndarray, np.ndarray]:
    q0 = np.clip(qu[:, 0], 0, Q_real)
    q1 = np.clip(qu[:, 1], 0, Q_real)
    t0 = q0 // block_m
    n = np.maximum((q1 + block_m - 1) // block_m - t0, 0)
    group = np.repeat(np.arange(len(qu), dtype=np.int64), n)
    first = np.cumsum(n) - n
    qtile = np.repeat(t0, n) + (np.arange(int(n.sum()), dtype=np.int64) - np.repeat(first, n))
    return group.astype(np.int32), qtile.astype(np.int32)


def build_qtile_tasks(q_unique: torch.Tensor, Q_real: int, BLOCK_M: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(task_group, task_qtile) [T] int32: every BLOCK_M-row query tile that meets
    a group's (clipped) query range, groups in order (magimask.py:216-245)."""
    g, t = _tasks(_host(q_unique), Q_real, BLOCK_M)
    dev = q_unique.device
    return torch.tensor(g, device=dev), torch.tensor(t, device=dev)


@dataclass(frozen=True)
class MagiMask:
    """CSR range tables plus the task list (train/wan/rcm/utils/magimask.py:248-262)."""

    q_unique: torch.Tensor  # [G,2] int32
    k_flat: torch.Tensor  # [K,2] int32
    qk_map: torch.Tensor  # [G+1] int32
    task_group: torch.Tensor  # [T] int32
    task_qtile: torch.Tensor  # [T] int32
    G: int
    T: int
    BLOCK_M: int


def prepare_magi_csr_and_tasks(q_ranges: torch.Tensor, k_ranges: torch.Tensor, Q_real: int, KV_real: int,
                               BLOCK_M: int = KERNEL_BLOCK_M) -> MagiMask:
    """Merge, group, check that the query groups partition [0, Q_real), build tasks
    (train/wan/rcm/utils/magimask.py:265-283). BLOCK_M defaults to the kernels' 128."""
    q_ranges, k_ranges = merge_k_ranges(q_ranges, k_ranges, KV_real=KV_real)
    q_unique, k_flat, qk_map = group_q_ranges_csr(q_ranges, k_ranges)
    qu = _host(q_unique)
    assert len(qu) > 0 and qu[0, 0] == 0 and qu[-1, 1] == Q_real, \
        f"the query groups must start at row 0 and end at row {Q_real} (Q_real)"
    for i in range(len(qu) - 1):
        assert qu[i, 1] == qu[i + 1, 0], \
            f"query groups {i} and {i + 1} do not meet: {qu[i].tolist()} then {qu[i + 1].tolist()}"
    task_group, task_qtile = build_qtile_tasks(q_unique, Q_real=Q_real, BLOCK_M=BLOCK_M)
    return MagiMask(q_unique=q_unique.contiguous(), k_flat=k_flat.contiguous(), qk_map=qk_map.contiguous(),
                    task_group=task_group, task_qtile=task_qtile, G=int(qu.shape[0]), T=int(task_group.numel()),
                    BLOCK_M=int(BLOCK_M))


def csr_to_dense(q_unique, k_flat, qk_map, Q: int, KV: int) -> torch.Tensor:
    """[Q, KV] bool mask the tables describe (for inspection and tests)."""
    qu, kf = _host(q_unique), _host(k_flat)
    qm = (qk_map.detach().cpu().numpy() if isinstance(qk_map, torch.Tensor) else np.asarray(qk_map)).astype(np.int64)
    m = np.zeros((Q, KV), dtype=bool)
    for g in range(len(qu)):
        q0, q1 = max(int(qu[g, 0]), 0), min(int(qu[g, 1]), Q)
        for r in range(int(qm[g]), int(qm[g + 1])):
            k0, k1 = max(int(kf[r, 0]), 0), min(int(kf[r, 1]), KV)
            if q1 > q0 and k1 > k0:
                m[q0:q1, k0:k1] = True
    return torch.from_numpy(m)


# tasks rebuilt for the kernels' tile, per mask object
_TASK_CACHE: dict = {}


def tasks_for_kernel(mask, Lq: int, device: torch.device) -> Tuple[torch.Tensor, torch.Tensor, int]:
    """(task_group, task_qtile, T) for 128-row query tiles on `device`.

    A mask built with BLOCK_M = 128 is used as is; another BLOCK_M costs one
    device-to-host copy of q_unique on the first call with that mask object.
    """
    if int(mask.BLOCK_M) == KERNEL_BLOCK_M:
        tg = mask.task_group.to(device=device, dtype=torch.int32).contiguous()
        tq = mask.task_qtile.to(device=device, dtype=torch.int32).contiguous()
        return tg, tq, int(tg.numel())
    key = (id(mask), Lq, str(device))
    hit = _TASK_CACHE.get(key)
    if hit is not None and hit[0]() is mask:
        return hit[1], hit[2], int(hit[1].numel())
    g, t = _tasks(_host(mask.q_unique), Lq, KERNEL_BLOCK_M)
    tg = torch.tensor(g, device=device)
    tq = torch.tensor(t, device=device)
    try:
        ref = weakref.ref(mask, lambda _r, k=key: _TASK_CACHE.pop(k, None))
        _TASK_CACHE[key] = (ref, tg, tq)
    except TypeError:  # objects without weak references are not cached
        pass
    return tg, tq, int(tg.numel())


def as_int32(t: torch.Tensor, device: torch.device, shape: Sequence[int] = None) -> torch.Tensor:
    out = t.to(device=device, dtype=torch.int32).contiguous()
    return out if shape is None else out.view(*shape)
