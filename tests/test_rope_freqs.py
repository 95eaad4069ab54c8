"""The 3D-RoPE angle table that shapes every Wan-size input (dmad_amd.workload.rope_freqs_3d),
against angles computed by hand from the reference formula, in float64 scalar code.

Reference (train/wan/rcm/networks/wan2pt1_jvp.py:71-74, 101-108, 151-168), head_dim 128:
  dim_h = dim_w = 128 // 6 * 2 = 42, dim_t = 128 - 84 = 44; theta = 10000 (NTK factor 1);
  angles of token (t, h, w) = [t * theta^(-2i/44) for i < 22] ++ [h * theta^(-2i/42) for i < 21]
                              ++ [w * theta^(-2i/42) for i < 21];
  tokens in (t, h, w) row-major order.
"""
import math

import pytest
import torch

from dmad_amd.workload import rope_freqs_3d


def _angles(t, h, w, head_dim=128, theta=10000.0):
    dim_h = head_dim // 6 * 2
    dim_t = head_dim - 2 * dim_h
    out = [t * theta ** (-(2 * i) / dim_t) for i in range(dim_t // 2)]
    out += [h * theta ** (-(2 * i) / dim_h) for i in range(dim_h // 2)]
    out += [w * theta ** (-(2 * i) / dim_h) for i in range(dim_h // 2)]
    return out


@pytest.mark.parametrize("grid", [(21, 30, 52), (21, 45, 80), (3, 4, 5)])
def test_angles_match_the_reference_formula(grid):
    T, Hh, W = grid
    f = rope_freqs_3d(T, Hh, W, 128)
    assert f.shape == (T * Hh * W, 64) and f.dtype == torch.float32
    picks = [(0, 0, 0), (0, 0, 1), (0, 1, 0), (1, 0, 0), (T - 1, Hh - 1, W - 1), (T // 2, Hh - 1, 0),
             (1, Hh // 3, W - 2), (T - 1, 0, W // 2)]
    for t, h, w in picks:
        token = (t * Hh + h) * W + w
        want = torch.tensor(_angles(t, h, w), dtype=torch.float64)
        got = f[token].double()
        assert torch.allclose(got, want, rtol=2e-6, atol=1e-6), (t, h, w, (got - want).abs().max())


def test_split_and_order_are_pinned():
    """A table with the h and w parts swapped, the t part the same width as the spatial ones,
    or tokens in (t, w, h) order fails the comparison above (Hh != W on these grids)."""
    T, Hh, W = 21, 30, 52
    f = rope_freqs_3d(T, Hh, W, 128)
    t, h, w = 5, 7, 40
    token = (t * Hh + h) * W + w
    want = torch.tensor(_angles(t, h, w), dtype=torch.float64)
    swapped = torch.tensor(_angles(t, w, h), dtype=torch.float64)
    assert torch.allclose(f[token].double(), want, rtol=2e-6, atol=1e-6)
    assert not torch.allclose(f[token].double(), swapped, rtol=1e-3, atol=1e-3)
    even = [t * 10000.0 ** (-(2 * i) / 42) for i in range(21)]
    assert not math.isclose(float(f[token, 1]), even[1], rel_tol=1e-3)
    wrong_order = (t * W + w) * Hh + h  # (t, w, h) row-major
    assert not torch.allclose(f[wrong_order].double(), want, rtol=1e-3, atol=1e-3)
