"""Writes the golden fixtures of this directory from the float64 oracle.

Run from the repository root: ``python tests/golden/make_golden.py``. Each
``.pt`` file holds plain tensors (load with ``torch.load(..., weights_only=True)``):
the inputs exactly as the tests feed them and the oracle's outputs in float32.

Cases
  plumbing   B=1, H=2, L=256, D=64, float32 inputs, Q,K,V ~ N(0,1), tangents
             ~ N(0, 0.1^2), seed 0, scale 1/8: O and Od by torch.func.jvp of math
             attention (the reference's CPU plumbing configuration), plus LSE, mu.
  ragged     B=1, H=1, Lq=Lk=515, D=64, bf16, N(0, 0.5^2), seed 20, scale 0.5 (the
             value distribution of the reference's op tests): O, Od, LSE, mu and the
             dO-only gradients for dO ~ N(0, 1).
  cross      B=1, H=1, Lq=700, Lk=15, Dqk=128, Dv=32, bf16, seed 20, scale 0.5:
             O, Od, LSE, mu (Lq != Lk, Dqk != Dv, ragged key tile).
  full_bwd   B=1, H=1, Lq=300, Lk=200, D=64, bf16, seed 7: the full derivative of
             (O, Od) for dO ~ N(0,1), dOd ~ N(0, 0.1^2), all six gradients.
"""
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention as orc  # noqa: E402


def _draw(g, shape, std, dtype):
    return (torch.randn(shape, generator=g, dtype=torch.float64) * std).to(dtype)


def plumbing():
    g = torch.Generator().manual_seed(0)
    shp = (1, 2, 256, 64)
    q, k, v = (_draw(g, shp, 1.0, torch.float32) for _ in range(3))
    tq, tk, tv = (_draw(g, shp, 0.1, torch.float32) for _ in range(3))
    o, to = orc.jvp_attention_autodiff(*(x.double() for x in (q, k, v, tq, tk, tv)), sm_scale=0.125)
    _, _, lse, mu = orc.jvp_closed_form(*(x.double() for x in (q, k, v, tq, tk, tv)), sm_scale=0.125)
    return dict(q=q, k=k, v=v, tq=tq, tk=tk, tv=tv, sm_scale=torch.tensor(0.125),
                o=o.float(), to=to.float(), lse=lse.float(), mu=mu.float())


def _fwd_case(B, H, Lq, Lk, Dqk, Dv, seed, sm_scale, grads):
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    q, k, v = _draw(g, (B, H, Lq, Dqk), 0.5, bf), _draw(g, (B, H, Lk, Dqk), 0.5, bf), _draw(g, (B, H, Lk, Dv), 0.5, bf)
    tq, tk, tv = _draw(g, (B, H, Lq, Dqk), 0.5, bf), _draw(g, (B, H, Lk, Dqk), 0.5, bf), _draw(g, (B, H, Lk, Dv), 0.5, bf)
    x64 = [t.double() for t in (q, k, v, tq, tk, tv)]
    o, to, lse, mu = orc.jvp_closed_form(*x64, sm_scale=sm_scale)
    out = dict(q=q, k=k, v=v, tq=tq, tk=tk, tv=tv, sm_scale=torch.tensor(sm_scale),
               o=o.float(), to=to.float(), lse=lse.float(), mu=mu.float())
    if grads:
        do = _draw(g, (B, H, Lq, Dv), 1.0, bf)
        dq, dk, dv = orc.grads_dout_only(x64[0], x64[1], x64[2], do.double(), sm_scale=sm_scale)
        out.update(do=do, dq=dq.float(), dk=dk.float(), dv=dv.float())
    return out


def full_bwd():
    g = torch.Generator().manual_seed(7)
    bf = torch.bfloat16
    B, H, Lq, Lk, D = 1, 1, 300, 200, 64
    q, k, v = _draw(g, (B, H, Lq, D), 1.0, bf), _draw(g, (B, H, Lk, D), 1.0, bf), _draw(g, (B, H, Lk, D), 1.0, bf)
    tq, tk, tv = (_draw(g, (B, H, L, D), 0.1, bf) for L in (Lq, Lk, Lk))
    do, dto = _draw(g, (B, H, Lq, D), 1.0, bf), _draw(g, (B, H, Lq, D), 0.1, bf)
    gr = orc.grads_full(*(t.double() for t in (q, k, v, tq, tk, tv, do, dto)), sm_scale=D ** -0.5)
    names = ("dq", "dk", "dv", "dtq", "dtk", "dtv")
    out = dict(q=q, k=k, v=v, tq=tq, tk=tk, tv=tv, do=do, dto=dto, sm_scale=torch.tensor(D ** -0.5))
    out.update({n: x.float() for n, x in zip(names, gr)})
    return out


CASES = {
    "plumbing": plumbing,
    "ragged": lambda: _fwd_case(1, 1, 515, 515, 64, 64, 20, 0.5, grads=True),
    "cross": lambda: _fwd_case(1, 1, 700, 15, 128, 32, 20, 0.5, grads=False),
    "full_bwd": full_bwd,
}


def main():
    for name, fn in CASES.items():
        path = os.path.join(HERE, f"{name}.pt")
        torch.save(fn(), path)
        print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


if __name__ == "__main__":
    main()
