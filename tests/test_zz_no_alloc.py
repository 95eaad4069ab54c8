"""dmad_attn_jvp_bwd_noalloc: the backward with its workspace in the library's
static device scratch, called through the C ABI, against dmad_attn_jvp_bwd
with a caller workspace on the same inputs. Same kernels, same statistics:
the gradients must be bitwise equal. Two calls in a row, the second smaller
than the first (the scratch keeps the first call's contents), then the first
shape again, and fp32 calls (their statistics in the same scratch)."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, B, H, L, D, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    r = lambda sd: (torch.randn((B, L, H, D), generator=g) * sd).to(dtype).to(dev).transpose(1, 2)  # noqa: E731
    return {n: r(sd) for n, sd in (("q", 1.0), ("k", 1.0), ("v", 1.0), ("tq", 0.1), ("tk", 0.1), ("tv", 0.1),
                                   ("do", 1.0), ("dto", 0.1))}


def _backward(x, full, noalloc):
    from dmad_amd import _native as nat
    from dmad_amd.jvp_attention import jvp_attention_forward

    q, k, v, tq, tk, tv = (x[n] for n in ("q", "k", "v", "tq", "tk", "tv"))
    B, H, L, D = q.shape
    s = D ** -0.5
    o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
    dout, dto = x["do"], (x["dto"] if full else None)
    grads = [torch.empty_like(t) for t in (q, k, v)]
    tgrads = [torch.empty_like(t) for t in (q, k, v)] if full else [None, None, None]
    lib = nat.lib()
    args = [nat.dtype_code(q.dtype), B, H, L, L, D,
            nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(tq if full else None), nat.ptr(tk if full else None),
            nat.ptr(tv if full else None), nat.strides4(q), nat.strides4(k), nat.strides4(v),
            nat.ptr(o), nat.ptr(to if full else None), nat.strides4(o), nat.ptr(lse), nat.ptr(mu if full else None),
            nat.ptr(dout), nat.ptr(dto), nat.strides4(dout),
            *(nat.ptr(t) for t in grads), *(nat.ptr(t) for t in tgrads),
            nat.strides4(grads[0]), nat.strides4(grads[1]), nat.strides4(grads[2]), float(s)]
    if noalloc:
        nat.check(lib.dmad_attn_jvp_bwd_noalloc(*args, nat.stream_ptr(q.device)))
    else:
        n = ctypes.c_size_t(0)
        nat.check(lib.dmad_attn_bwd_workspace_bytes(2 if full else 0, B, H, L, L, D, ctypes.byref(n)))
        ws = torch.empty(max(n.value, 1), device=q.device, dtype=torch.uint8)
        nat.check(lib.dmad_attn_jvp_bwd(*args, nat.ptr(ws), ws.numel(), nat.stream_ptr(q.device)))
    torch.cuda.synchronize()
    return [t for t in grads + tgrads if t is not None]


CALLS = [
    # (B, H, L, D, full derivative with tangent gradients, dtype)
    (2, 3, 700, 128, True, torch.bfloat16),
    (1, 2, 300, 64, False, torch.bfloat16),
    (2, 3, 700, 128, True, torch.bfloat16),
    (1, 2, 257, 32, False, torch.float32),
    # fp32 with 256-wide heads needs only its statistics (512 KiB here), well inside the scratch
    (1, 32, 2048, 256, False, torch.float32),
]


def test_noalloc_backward_equals_workspace_backward(gpu):
    for i, (B, H, L, D, full, dtype) in enumerate(CALLS):
        print(f"case noalloc call {i}: B={B} H={H} L={L} D={D} full={full} {dtype}", flush=True)
        x = _inputs(gpu, B, H, L, D, seed=i, dtype=dtype)
        ref = _backward(x, full, noalloc=False)
        got = _backward(x, full, noalloc=True)
        assert len(got) == (6 if full else 3)
        for a, b in zip(got, ref):
            assert torch.isfinite(b).all()
            assert torch.equal(a, b)

