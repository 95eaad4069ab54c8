"""CPU oracle for the flash-attention JVP path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this module, and only as the checker. The product path
(``dmad_amd``) never calls it.

Restates, in plain PyTorch on the CPU (float64 by default), what the reference
computes on this path:

* ``math_attention``          -- softmax attention, O and natural-log LSE
  (the semantics of ``_attn_fwd``, train/wan/rcm/utils/flash_attention_jvp_triton.py:107-232,
  and of the math oracles :637-645 / :778-783).
* ``jvp_attention_autodiff``  -- ``torch.func.jvp`` of math attention, the oracle of
  the reference's ``_test_jvp`` / ``_test_jvp_ca`` (:627-658, :768-803).
* ``jvp_closed_form``         -- the closed form the kernel evaluates:
  Od = P Vd + (P*(Sd - mu)) V, mu = rowsum(P*Sd) (:193-223).
* ``grads_dout_only``         -- the dO-only gradients the reference backward
  returns (flash-attn FA2 backward called at :540-578, cotangent of ``to``
  discarded at :535).
* ``grads_full``              -- the full derivative of (O, Od) w.r.t. all six inputs.
* ``triton_fwd_emulator``     -- the numerics of ``_attn_fwd`` (log2-domain online
  softmax over BLOCK_N tiles, bf16/fp16 rounding of P~ and H~ before the PV dots,
  fp32 accumulators, the :216-223 epilogue), used to measure the reference
  kernel's own error floor.
* ``naive_attention_in_dtype`` -- the reference tests' oracle: matmul in the input
  dtype, softmax in fp32 cast back to the dtype (:596-605, :637-645).
* ``fa2_bwd_emulator``        -- the numerics of the standard FA2 backward the reference
  calls (P and dS rounded to the input type before the gradient products), used to
  measure the reference backward's own error floor.

How each function is pinned (tests/test_oracle.py):
  math_attention            brute-force loops on tiny inputs; LSE >= max S;
                            Lk = 1 gives O = V.
  jvp_closed_form           torch.func.jvp (autodiff) and central differences
                            in float64; invariants (linearity in the tangents,
                            zero tangents -> 0, Vd-only tangent -> attention(Q,K,Vd),
                            joint key permutation, Lk = 1 -> Od = Vd).
  grads_dout_only           torch.autograd of math_attention.
  grads_full                torch.autograd through torch.func.jvp, and float64
                            central differences of <dO,O> + <dOd,Od>.
  triton_fwd_emulator       equals math attention in float64 with no rounding
                            for every BLOCK_N; bf16 error within the reference
                            tests' tolerances.
  naive_attention_in_dtype  reduces to math_attention in float64.
  fa2_bwd_emulator          equals grads_dout_only in float64 with no rounding;
                            bf16 error within the reference tests' tolerances.
Tensors are [B, H, L, D] (BHSD).
"""
from __future__ import annotations

import math

import torch

LN2 = math.log(2.0)
LOG2E = 1.0 / LN2


def _scale(q, sm_scale):
    return q.shape[-1] ** (-0.5) if sm_scale is None else sm_scale


def math_attention(q, k, v, sm_scale=None):
    """O = softmax(s Q K^T) V and LSE = logsumexp(s Q K^T) (natural log)."""
    s = _scale(q, sm_scale)
    S = torch.matmul(q, k.transpose(-1, -2)) * s
    lse = torch.logsumexp(S, dim=-1)
    P = torch.exp(S - lse[..., None])
    return torch.matmul(P, v), lse


def jvp_closed_form(q, k, v, tq, tk, tv, sm_scale=None):
    """(O, Od, LSE, mu) with Sd = s(Qd K^T + Q Kd^T), mu = rowsum(P*Sd),
    Od = P Vd + (P*(Sd - mu)) V  (flash_attention_jvp_triton.py:193-223)."""
    s = _scale(q, sm_scale)
    S = torch.matmul(q, k.transpose(-1, -2)) * s
    lse = torch.logsumexp(S, dim=-1)
    P = torch.exp(S - lse[..., None])
    Sd = (torch.matmul(tq, k.transpose(-1, -2)) + torch.matmul(q, tk.transpose(-1, -2))) * s
    mu = (P * Sd).sum(-1)
    Pd = P * (Sd - mu[..., None])
    o = torch.matmul(P, v)
    to = torch.matmul(P, tv) + torch.matmul(Pd, v)
    return o, to, lse, mu


def jvp_attention_autodiff(q, k, v, tq, tk, tv, sm_scale=None):
    """(O, Od) by forward-mode autodiff of math attention."""
    fn = lambda a, b, c: math_attention(a, b, c, sm_scale)[0]  # noqa: E731
    return torch.func.jvp(fn, (q, k, v), (tq, tk, tv))


def grads_dout_only(q, k, v, dout, sm_scale=None):
    """FA2 backward restated: D = rowsum(dO*O), dP = dO V^T, dS = P*(dP - D),
    dQ = s dS K, dK = s dS^T Q, dV = P^T dO."""
    s = _scale(q, sm_scale)
    S = torch.matmul(q, k.transpose(-1, -2)) * s
    lse = torch.logsumexp(S, dim=-1)
    P = torch.exp(S - lse[..., None])
    o = torch.matmul(P, v)
    Dr = (dout * o).sum(-1)
    dP = torch.matmul(dout, v.transpose(-1, -2))
    dS = P * (dP - Dr[..., None])
    dq = torch.matmul(dS, k) * s
    dk = torch.matmul(dS.transpose(-1, -2), q) * s
    dv = torch.matmul(P.transpose(-1, -2), dout)
    return dq, dk, dv


def grads_full(q, k, v, tq, tk, tv, dout, dto, sm_scale=None):
    """Closed-form vector-Jacobian product of (O, Od) w.r.t. (Q, K, V, Qd, Kd, Vd).

    rho = rowsum(dOd*O), D' = rowsum(dO*O) + rowsum(dOd*Od) - mu*rho,
    dPd = dOd V^T, dP = dO V^T + dOd Vd^T + dPd*(Sd - mu) - Sd*rho,
    dS = P*(dP - D'), dSd = P*(dPd - rho),
    dQ = s(dS K + dSd Kd), dK = s(dS^T Q + dSd^T Qd), dV = P^T dO + Pd^T dOd,
    dQd = s dSd K, dKd = s dSd^T Q, dVd = P^T dOd.
    """
    s = _scale(q, sm_scale)
    S = torch.matmul(q, k.transpose(-1, -2)) * s
    lse = torch.logsumexp(S, dim=-1)
    P = torch.exp(S - lse[..., None])
    Sd = (torch.matmul(tq, k.transpose(-1, -2)) + torch.matmul(q, tk.transpose(-1, -2))) * s
    mu = (P * Sd).sum(-1)
    Pd = P * (Sd - mu[..., None])
    o = torch.matmul(P, v)
    to = torch.matmul(P, tv) + torch.matmul(Pd, v)
    rho = (dto * o).sum(-1)
    Dp = (dout * o).sum(-1) + (dto * to).sum(-1) - mu * rho
    dPd = torch.matmul(dto, v.transpose(-1, -2))
    dP = (torch.matmul(dout, v.transpose(-1, -2)) + torch.matmul(dto, tv.transpose(-1, -2))
          + dPd * (Sd - mu[..., None]) - Sd * rho[..., None])
    dS = P * (dP - Dp[..., None])
    dSd = P * (dPd - rho[..., None])
    dq = s * (torch.matmul(dS, k) + torch.matmul(dSd, tk))
    dk = s * (torch.matmul(dS.transpose(-1, -2), q) + torch.matmul(dSd.transpose(-1, -2), tq))
    dv = torch.matmul(P.transpose(-1, -2), dout) + torch.matmul(Pd.transpose(-1, -2), dto)
    dtq = s * torch.matmul(dSd, k)
    dtk = s * torch.matmul(dSd.transpose(-1, -2), q)
    dtv = torch.matmul(P.transpose(-1, -2), dto)
    return dq, dk, dv, dtq, dtk, dtv


def grads_full_autodiff(q, k, v, tq, tk, tv, dout, dto, sm_scale=None):
    """Same VJP by reverse-mode autograd through torch.func.jvp."""
    leaves = [x.detach().clone().requires_grad_(True) for x in (q, k, v, tq, tk, tv)]
    o, to = jvp_attention_autodiff(*leaves, sm_scale=sm_scale)
    loss = (o * dout).sum() + (to * dto).sum()
    return torch.autograd.grad(loss, leaves)


def naive_attention_in_dtype(q, k, v, sm_scale, dtype):
    """The reference tests' oracle: matmul in `dtype`, softmax in fp32, P cast back."""
    p = torch.matmul(q, k.transpose(2, 3)) * sm_scale
    p = torch.softmax(p.float(), dim=-1).to(dtype)
    return torch.matmul(p, v)


def _round(x, dtype):
    return x if dtype is None else x.to(dtype).to(x.dtype)


def triton_fwd_emulator(q, k, v, tq, tk, tv, sm_scale=None, block_n=64, round_dtype=torch.bfloat16):
    """Numerics of `_attn_fwd` (flash_attention_jvp_triton.py:150-232) in float32.

    Inputs are the (already rounded) operands in any float dtype; arithmetic is
    float32; p and H~ are rounded to `round_dtype` before the PV dots (:204-205),
    outputs are returned in float32 (before the final store rounding).
    `round_dtype=None` keeps every step in float32 (and, with float64 inputs,
    float64) -- then the result equals math attention up to summation order.
    """
    f = torch.float64 if q.dtype == torch.float64 else torch.float32
    q, k, v, tq, tk, tv = (x.to(f) for x in (q, k, v, tq, tk, tv))
    s = _scale(q, sm_scale)
    qk_scale = s * LOG2E
    B, H, Lq, _ = q.shape
    Lk, Dv = v.shape[-2], v.shape[-1]
    m_i = torch.full((B, H, Lq), -math.inf, dtype=f)
    l_i = torch.zeros((B, H, Lq), dtype=f)
    r_i = torch.zeros((B, H, Lq), dtype=f)
    o_i = torch.zeros((B, H, Lq, Dv), dtype=f)
    a_i = torch.zeros_like(o_i)
    b_i = torch.zeros_like(o_i)
    for start in range(0, Lk, block_n):
        kk, tkk = k[..., start:start + block_n, :], tk[..., start:start + block_n, :]
        vv, tvv = v[..., start:start + block_n, :], tv[..., start:start + block_n, :]
        qk = torch.matmul(q, kk.transpose(-1, -2)) * qk_scale
        m_ij = torch.maximum(m_i, qk.amax(-1))
        p = torch.exp2(qk - m_ij[..., None])
        alpha = torch.exp2(m_i - m_ij)
        l_i = l_i * alpha + p.sum(-1)
        o_i = o_i * alpha[..., None]
        a_i = a_i * alpha[..., None]
        b_i = b_i * alpha[..., None]
        r_i = r_i * alpha
        ts = (torch.matmul(tq, kk.transpose(-1, -2)) + torch.matmul(q, tkk.transpose(-1, -2))) * s
        ht = p * ts
        r_i = r_i + ht.sum(-1)
        p_r, ht_r = _round(p, round_dtype), _round(ht, round_dtype)
        o_i = o_i + torch.matmul(p_r, vv)
        a_i = a_i + torch.matmul(p_r, tvv)
        b_i = b_i + torch.matmul(ht_r, vv)
        m_i = m_ij
    inv_l = 1.0 / l_i
    o = o_i * inv_l[..., None]
    mu = r_i * inv_l
    to = a_i * inv_l[..., None] + b_i * inv_l[..., None] - mu[..., None] * o
    lse = (m_i + torch.log2(l_i)) * LN2
    return o, to, lse


def fa2_bwd_emulator(q, k, v, do, sm_scale=None, round_dtype=torch.bfloat16):
    """Numerics of the standard FlashAttention-2 backward the reference calls
    (flash-attn, flash_attention_jvp_triton.py:540-578; the published FA2
    backward: P recomputed from the forward's LSE, D = rowsum(dO * O) from the
    stored O, dP = dO V^T and dS = P * (dP - D) in float32, P and dS rounded to
    the input type before the dV = P^T dO, dK = s dS^T Q, dQ = s dS K products,
    float32 accumulation). Inputs are the (already rounded) operands; returns
    float32 (float64 for float64 inputs) dq, dk, dv before their final store
    rounding. `round_dtype=None` rounds nothing, so float64 inputs give the
    exact dO-only gradients.
    """
    f = torch.float64 if q.dtype == torch.float64 else torch.float32
    q, k, v, do = (x.to(f) for x in (q, k, v, do))
    s = _scale(q, sm_scale)
    S = torch.matmul(q, k.transpose(-1, -2)) * s
    lse = torch.logsumexp(S, dim=-1)
    P = torch.exp(S - lse[..., None])
    o = torch.matmul(_round(P, round_dtype), v)
    o = _round(o, round_dtype)  # the forward stores O in the input type
    Dr = (do * o).sum(-1)
    dP = torch.matmul(do, v.transpose(-1, -2))
    dS = P * (dP - Dr[..., None])
    P_r, dS_r = _round(P, round_dtype), _round(dS, round_dtype)
    dv = torch.matmul(P_r.transpose(-1, -2), do)
    dk = s * torch.matmul(dS_r.transpose(-1, -2), q)
    dq = s * torch.matmul(dS_r, k)
    return dq, dk, dv


def rel_l2(x, ref):
    """||x - ref||_2 / ||ref||_2 in float64."""
    x = x.detach().to(torch.float64).cpu()
    ref = ref.detach().to(torch.float64).cpu()
    den = torch.linalg.vector_norm(ref)
    return float(torch.linalg.vector_norm(x - ref) / (den if den > 0 else 1.0))


def jvp_rows(q, k, v, tq, tk, tv, rows, sm_scale=None, dtype=torch.float64):
    """Closed-form (O, Od, LSE, mu) for a subset of query rows at full Lk."""
    idx = torch.as_tensor(rows, dtype=torch.long)
    qs, tqs = q[..., idx, :], tq[..., idx, :]
    return jvp_closed_form(*(x.to(dtype) for x in (qs, k, v, tqs, tk, tv)), sm_scale=sm_scale)
