"""The op under HIP graph capture (torch.cuda.CUDAGraph).

Serving loops capture a whole denoising step and replay it; the library then
has to put nothing but kernel launches on the stream (no memsets, no host
synchronisation, no allocation outside torch's capture pool). One capture holds
the self-attention forward+JVP, the 512-key text cross-attention forward (two
workgroups per CU), the dO-only backward, the full-derivative backward with
tangent gradients and the allocation-free backward entry point. The graph is
replayed three times with eager work in between that rewrites other memory,
and every replay must equal the eager results bit for bit.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, B, H, L, Lx, D):
    g = torch.Generator().manual_seed(17)
    r = lambda L_, sd: (torch.randn((B, L_, H, D), generator=g) * sd).to(torch.bfloat16).to(dev).transpose(1, 2)  # noqa: E731
    return dict(q=r(L, 1.0), k=r(L, 1.0), v=r(L, 1.0), tq=r(L, 0.1), tk=r(L, 0.1), tv=r(L, 0.1), do=r(L, 1.0),
                dto=r(L, 0.1), kx=r(Lx, 1.0), vx=r(Lx, 1.0))


def _step(x):
    from dmad_amd import _native as nat
    from dmad_amd.jvp_attention import jvp_attention_backward, jvp_attention_forward

    q, k, v, tq, tk, tv, do, dto = (x[n] for n in ("q", "k", "v", "tq", "tk", "tv", "do", "dto"))
    B, H, L, D = q.shape
    s = D ** -0.5
    o, to, lse, mu = jvp_attention_forward(q, k, v, tq, tk, tv, s)
    ox, tox, _, _ = jvp_attention_forward(q, x["kx"], x["vx"], tq, None, None, s)
    g_a = jvp_attention_backward(q, k, v, None, None, None, o, None, lse, None, do, None, s, False)[:3]
    g_b = jvp_attention_backward(q, k, v, tq, tk, tv, o, to, lse, mu, do, dto, s, True)
    # the allocation-free entry point (dO-only gradients into preallocated outputs)
    g_n = [torch.empty_like(t) for t in (q, k, v)]
    nat.check(nat.lib().dmad_attn_jvp_bwd_noalloc(
        nat.DMAD_BF16, B, H, L, L, D, nat.ptr(q), nat.ptr(k), nat.ptr(v), None, None, None,
        nat.strides4(q), nat.strides4(k), nat.strides4(v), nat.ptr(o), None, nat.strides4(o), nat.ptr(lse), None,
        nat.ptr(do), None, nat.strides4(do), *(nat.ptr(t) for t in g_n), None, None, None,
        nat.strides4(g_n[0]), nat.strides4(g_n[1]), nat.strides4(g_n[2]), float(s), nat.stream_ptr(q.device)))
    return [o, to, lse, mu, ox, tox, *g_a, *g_b, *g_n]


def test_captured_step_replays_equal_eager(gpu):
    print("case graph capture B=1 H=4 L=1000 Lx=512 D=128", flush=True)
    x = _inputs(gpu, 1, 4, 1000, 512, 128)
    ref = [t.clone() for t in _step(x)]
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _step(x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _step(x)
    torch.cuda.synchronize()

    for i in range(3):
        junk = torch.randn(4096, 4096, device=gpu)  # eager work that rewrites other memory
        (junk @ junk).sum().item()
        del junk
        graph.replay()
        torch.cuda.synchronize()
        for j, (a, b) in enumerate(zip(out, ref)):
            assert torch.equal(a, b), (i, j)
