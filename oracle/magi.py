"""CPU oracle for the block-sparse (MagiMask) JVP forward (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this module, and only as the checker.

* ``allowed_mask``      -- the [Q, KV] boolean mask of a block schedule, written
  from the rules the reference tests state (``_build_bool_mask_from_spec``,
  train/wan/rcm/utils/flash_attention_jvp_triton.py:806-868): blocks of frames
  (first block ``first_chunk_frames`` frames, the rest ``chunk_frames``),
  block-causal with an optional sliding window and sink, or teacher forcing on
  a packed [clean][noisy] sequence. It does not use the range tables, so it
  checks them. ``as_range_builder=True`` switches the one rule where the
  reference's range builder differs from its test mask (teacher forcing,
  1-block window, sink: noisy queries get no sink).
* ``masked_jvp``        -- (O, Od, LSE, mu) of attention restricted to a boolean
  mask, closed form in float64: P = softmax over the allowed keys,
  Sd = s (Qd K^T + Q Kd^T), mu = rowsum(P Sd), Od = P Vd + (P (Sd - mu)) V.
  A row with no allowed key gets O = Od = 0, LSE = -inf, mu = 0 (what
  ``_attn_fwd_magi``'s epilogue gives for l_i == 0, :386-400).
* ``masked_jvp_rows``   -- the same for a subset of query rows.
* ``random_rectangles`` -- a seeded random mask as the reference's builder takes
  it (``prepare_magi_csr_and_tasks``, train/wan/rcm/utils/magimask.py:265-283):
  the query axis cut into groups, each with 1-4 key ranges that may overlap,
  touch or reach outside [0, KV), rows shuffled; the [Q, KV] mask is the union
  of the clipped rectangles, painted straight from the raw ranges.
* ``magi_fwd_emulator`` -- the numerics of ``_attn_fwd_magi`` (:242-409): per
  query group, key tiles of BLOCK_N walking each range from the tile boundary
  below its start, keys outside the range at -inf (tangent scores at 0),
  log2-domain online softmax with the -inf-safe max, p~ and H~ rounded to the
  input type before the PV dots; rows outside every group are NaN.

How each is pinned (tests/test_magi_oracle.py): ``allowed_mask`` by
hand-written matrices of small schedules and by agreement with the mask the
range tables describe for a sweep of schedules; ``masked_jvp`` by
``torch.func.jvp`` of masked math attention, by the dense closed form when
everything is allowed, by per-row brute force and the empty-row case;
``magi_fwd_emulator`` by ``masked_jvp`` in float64 without rounding, for
several BLOCK_N; ``random_rectangles`` by hand-painted masks of small draws
(every row's rectangle, and nothing else, is set).
"""
from __future__ import annotations

import math

import numpy as np
import torch

LN2 = math.log(2.0)
LOG2E = 1.0 / LN2


def _block_of(tok: np.ndarray, ft: int, first: int, chunk: int, use_first: bool) -> np.ndarray:
    frame = tok // ft
    if not use_first:
        return frame // chunk
    return np.where(frame < first, 0, 1 + (frame - first) // chunk)


def allowed_mask(mode: str, frame_tokens: int, Q: int, KV: int, first_chunk_frames: int = 1, chunk_frames: int = 1,
                 q_block_offset: int = 0, local_attn_blocks: int = 0, sink_blocks: int = 0,
                 clean_blocks: int = 0, as_range_builder: bool = False) -> torch.Tensor:
    """[Q, KV] bool: which keys each query may attend to.

    The reference states teacher forcing twice, and the two differ in one case:
    with ``local_attn_blocks == 1`` and a sink, its boolean test mask
    (flash_attention_jvp_triton.py:850-853) lets noisy queries see the sink
    blocks, while its range builder (train/wan/rcm/utils/magimask.py:98-104)
    adds a noisy block's sink only together with a non-empty window of earlier
    clean blocks, which a 1-block window never has. The kernels run on the range
    builder's tables, so ``as_range_builder=True`` gives that rule."""
    ft, first, chunk = frame_tokens, first_chunk_frames, chunk_frames
    q = np.arange(Q)[:, None]
    kv = np.arange(KV)[None, :]
    window = local_attn_blocks - 1
    if mode == "block_causal":
        qb = q_block_offset + _block_of(q, ft, first, chunk, use_first=q_block_offset == 0)
        kb = _block_of(kv, ft, first, chunk, use_first=True)
        ok = kb <= qb
        if window >= 0:
            ok &= kb >= qb - window
        if sink_blocks > 0:
            ok |= (kb < sink_blocks) & (kb <= qb)
        return torch.from_numpy(np.broadcast_to(ok, (Q, KV)).copy())
    if mode == "teacher_forcing":
        clean = (first + (clean_blocks - 1) * chunk) * ft
        q_clean, k_clean = q < clean, kv < clean
        qb_c = _block_of(q, ft, first, chunk, True)
        qb_n = _block_of(np.maximum(q - clean, 0), ft, first, chunk, True)
        kb_c = _block_of(kv, ft, first, chunk, True)
        kb_n = _block_of(np.maximum(kv - clean, 0), ft, first, chunk, True)
        clean_ok = q_clean & k_clean & (kb_c <= qb_c)
        noisy_prev = ~q_clean & k_clean & (kb_c < qb_n)
        if window >= 0:
            clean_ok &= kb_c >= qb_c - window
            noisy_prev &= kb_c >= qb_n - window
        noisy_own = ~q_clean & ~k_clean & (kb_n == qb_n)
        ok = clean_ok | noisy_prev | noisy_own
        if sink_blocks > 0:
            if not (as_range_builder and window == 0):
                ok |= ~q_clean & k_clean & (kb_c < sink_blocks) & (kb_c < qb_n)
            ok |= q_clean & k_clean & (kb_c < sink_blocks) & (kb_c < qb_c)
        ok = ok | (q == kv)
        return torch.from_numpy(np.broadcast_to(ok, (Q, KV)).copy())
    raise ValueError(f"Unknown mode: {mode}")


def masked_jvp(q, k, v, tq, tk, tv, allow, sm_scale):
    """(O, Od, LSE, mu) of attention over the allowed keys (float64 closed form)."""
    q, k, v, tq, tk, tv = (x.double() for x in (q, k, v, tq, tk, tv))
    allow = allow.to(torch.bool)
    S = torch.matmul(q, k.transpose(-1, -2)) * sm_scale
    S = S.masked_fill(~allow, -math.inf)
    lse = torch.logsumexp(S, dim=-1)
    empty = torch.isinf(lse)
    P = torch.exp(S - torch.where(empty, torch.zeros_like(lse), lse)[..., None])
    P = P.masked_fill(~allow, 0.0)
    Sd = (torch.matmul(tq, k.transpose(-1, -2)) + torch.matmul(q, tk.transpose(-1, -2))) * sm_scale
    mu = (P * Sd).sum(-1)
    o = torch.matmul(P, v)
    to = torch.matmul(P, tv) + torch.matmul(P * (Sd - mu[..., None]), v)
    return o, to, lse, mu


def masked_jvp_rows(q, k, v, tq, tk, tv, allow, rows, sm_scale):
    """masked_jvp for the query rows `rows` only (float64)."""
    idx = torch.as_tensor(rows, dtype=torch.long)
    return masked_jvp(q[..., idx, :], k, v, tq[..., idx, :], tk, tv, allow[idx], sm_scale)


def random_rectangles(seed: int, Q: int, KV: int, max_groups: int = 6):
    """(q_ranges [R,2], k_ranges [R,2] int32, allow [Q,KV] bool) of a random mask
    whose query groups partition [0, Q) and each have at least one key in range."""
    rng = np.random.default_rng(seed)
    n_groups = int(rng.integers(1, min(max_groups, Q) + 1))
    cuts = np.sort(rng.choice(np.arange(1, Q), size=n_groups - 1, replace=False)) if n_groups > 1 else np.array([], int)
    bounds = [0] + [int(c) for c in cuts] + [Q]
    rows = []
    allow = np.zeros((Q, KV), dtype=bool)
    for q0, q1 in zip(bounds[:-1], bounds[1:]):
        a = int(rng.integers(0, KV))
        spans = [(a, int(rng.integers(a + 1, KV + 1)))]  # one range inside [0, KV)
        for _ in range(int(rng.integers(0, 4))):
            kind = int(rng.integers(0, 3))
            if kind == 0 and spans:  # touching the previous range
                b0 = spans[-1][1]
                spans.append((b0, b0 + int(rng.integers(1, KV // 3 + 2))))
            else:  # anywhere, possibly before 0 or past KV
                a = int(rng.integers(-KV // 4 - 1, KV + KV // 4 + 1))
                spans.append((a, a + int(rng.integers(1, KV // 2 + 2))))
        for a, b in spans:
            rows.append((q0, q1, a, b))
            if max(a, 0) < min(b, KV):  # a range wholly outside [0, KV) adds nothing
                allow[q0:q1, max(a, 0):min(b, KV)] = True
    rows = [rows[i] for i in rng.permutation(len(rows))]
    arr = torch.tensor(rows, dtype=torch.int32).reshape(-1, 4)
    return arr[:, :2].contiguous(), arr[:, 2:].contiguous(), torch.from_numpy(allow)


def _round(x, dtype):
    return x if dtype is None else x.to(dtype).to(x.dtype)


def magi_fwd_emulator(q, k, v, tq, tk, tv, q_unique, k_flat, qk_map, sm_scale, block_n=64, round_dtype=torch.bfloat16):
    """Numerics of `_attn_fwd_magi`; returns (O, Od, LSE) in float32 (float64 for
    float64 inputs), NaN on rows no group covers."""
    f = torch.float64 if q.dtype == torch.float64 else torch.float32
    q, k, v, tq, tk, tv = (x.to(f) for x in (q, k, v, tq, tk, tv))
    B, H, Lq, _ = q.shape
    Lk, Dv = v.shape[-2], v.shape[-1]
    qk_scale = sm_scale * LOG2E
    qu = np.asarray(q_unique.cpu()).reshape(-1, 2)
    kf = np.asarray(k_flat.cpu()).reshape(-1, 2)
    qm = np.asarray(qk_map.cpu()).reshape(-1)
    O = torch.full((B, H, Lq, Dv), math.nan, dtype=f)
    tO = torch.full_like(O, math.nan)
    LSE = torch.full((B, H, Lq), math.nan, dtype=f)
    for g in range(len(qu)):
        r0, r1 = max(int(qu[g, 0]), 0), min(int(qu[g, 1]), Lq)
        if r1 <= r0:
            continue
        qq, tqq = q[..., r0:r1, :], tq[..., r0:r1, :]
        n = r1 - r0
        m_i = torch.full((B, H, n), -math.inf, dtype=f)
        l_i = torch.zeros((B, H, n), dtype=f)
        r_i = torch.zeros_like(l_i)
        o_i = torch.zeros((B, H, n, Dv), dtype=f)
        a_i = torch.zeros_like(o_i)
        b_i = torch.zeros_like(o_i)
        for r in range(int(qm[g]), int(qm[g + 1])):
            k0, k1 = max(int(kf[r, 0]), 0), min(int(kf[r, 1]), Lk)
            start = (k0 // block_n) * block_n
            while start < k1:
                idx = torch.arange(start, start + block_n)
                keep = (idx >= k0) & (idx < k1) & (idx < Lk)
                sel = idx.clamp(max=Lk - 1)
                z = keep.to(f)[:, None]
                kk, tkk = k[..., sel, :] * z, tk[..., sel, :] * z
                vv, tvv = v[..., sel, :] * z, tv[..., sel, :] * z
                qk = torch.matmul(qq, kk.transpose(-1, -2)) * qk_scale
                qk = qk.masked_fill(~keep, -math.inf)
                m_ij = torch.maximum(m_i, qk.amax(-1))
                m_safe = torch.where(torch.isinf(m_ij), torch.zeros_like(m_ij), m_ij)
                p = torch.exp2(qk - m_safe[..., None])
                alpha = torch.exp2(m_i - m_safe)
                l_i = l_i * alpha + p.sum(-1)
                o_i, a_i, b_i = o_i * alpha[..., None], a_i * alpha[..., None], b_i * alpha[..., None]
                r_i = r_i * alpha
                m_i = m_ij
                ts = (torch.matmul(tqq, kk.transpose(-1, -2)) + torch.matmul(qq, tkk.transpose(-1, -2))) * sm_scale
                ts = ts.masked_fill(~keep, 0.0)
                ht = p * ts
                r_i = r_i + ht.sum(-1)
                p_r, ht_r = _round(p, round_dtype), _round(ht, round_dtype)
                o_i = o_i + torch.matmul(p_r, vv)
                a_i = a_i + torch.matmul(p_r, tvv)
                b_i = b_i + torch.matmul(ht_r, vv)
                start += block_n
        l_safe = torch.where(l_i == 0, torch.ones_like(l_i), l_i)
        inv = 1.0 / l_safe
        o = o_i * inv[..., None]
        mu = r_i * inv
        O[..., r0:r1, :] = o
        tO[..., r0:r1, :] = a_i * inv[..., None] + b_i * inv[..., None] - mu[..., None] * o
        LSE[..., r0:r1] = (m_i + torch.log2(l_safe)) * LN2
    return O, tO, LSE
