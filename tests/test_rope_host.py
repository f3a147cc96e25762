"""3-D RoPE tables (sr_dit/model.py) against the closed form, on the CPU.

rope_params (models.py:80-88): entry [p, j] = exp(i * p * theta^(-2j/dim)).
_rope_axis_dims (models.py:91-97): head_dim 128 -> 44/42/42 real dims, i.e.
22/21/21 complex pairs for the frame, row and column axes (the docstring's
own figures).  rope_apply (models.py:173-214) concatenates the three axes'
phasors in that order.  Every expected value here is computed from those
formulas with Python's cmath, independently of the product's tables, so a
wrong split, exponent, axis order or offset fails.
"""
import cmath
import math

import pytest
import torch

from sr_dit import model as mdl

THETA = 10000.0


def _phasor(pos, j, dim):
    return cmath.exp(1j * pos * THETA ** (-2.0 * j / dim))


def test_axis_split_for_head_dim_128():
    assert mdl.rope_axis_dims(128) == (44, 42, 42)
    assert sum(mdl.rope_axis_dims(128)) == 128


@pytest.mark.parametrize("dim", [44, 42])
def test_rope_params_closed_form(dim):
    tab = mdl.rope_params(1024, dim, THETA)
    assert tab.shape == (1024, dim // 2) and tab.dtype == torch.complex128
    for p in (0, 1, 7, 300, 1023):
        for j in (0, 1, dim // 4, dim // 2 - 1):
            want = _phasor(p, j, dim)
            got = complex(tab[p, j])
            assert abs(got - want) <= 1e-12, (p, j, got, want)


@pytest.mark.parametrize("t_offset,stride", [(0, (1, 1)), (5, (1, 1)), (1030, (1, 1)),
                                             (3, (2, 2))])
def test_rope_table_token_phasors(t_offset, stride):
    cfg = mdl.SRDiTConfig()
    f, h, w = 3, 9, 10
    tab = mdl.rope_table(cfg, f, h, w, t_offset, "cpu", hw_stride=stride)
    assert tab.shape == (f * h * w, 1, 64)
    s_h, s_w = stride
    for (t, y, x) in ((0, 0, 0), (2, 8, 9), (1, 4, 7)):
        row = tab[(t * h + y) * w + x, 0]
        for c in (0, 5, 21, 22, 30, 42, 43, 50, 63):
            if c < 22:
                want = _phasor(t_offset + t, c, 44)
            elif c < 43:
                want = _phasor(y * s_h, c - 22, 42)
            else:
                want = _phasor(x * s_w, c - 43, 42)
            got = complex(row[c])
            assert abs(got - want) <= 2e-6, (t, y, x, c, got, want)


def test_rope_apply_rotates_pairs():
    cfg = mdl.SRDiTConfig()
    tab = mdl.rope_table(cfg, 1, 2, 3, 7, "cpu")
    g = torch.Generator("cpu").manual_seed(0)
    x = torch.randn(6, 2, 128, generator=g)
    y = mdl.rope_apply(x, tab)
    for tok, head, c in ((0, 0, 0), (5, 1, 30), (3, 0, 63)):
        a, b = float(x[tok, head, 2 * c]), float(x[tok, head, 2 * c + 1])
        z = complex(a, b) * complex(tab[tok, 0, c])
        assert abs(float(y[tok, head, 2 * c]) - z.real) <= 1e-5
        assert abs(float(y[tok, head, 2 * c + 1]) - z.imag) <= 1e-5


@pytest.mark.parametrize("t_offset,stride", [(0, (1, 1)), (27, (1, 1)), (1100, (1, 1)), (9, (2, 3))])
def test_rope_table_from_longer_axis_tables(t_offset, stride):
    """The streaming loop gathers a new offset's table on the device from axis
    tables kept there, which may hold more positions than the grid needs: the
    gather equals rope_table bit for bit, and refuses tables that are too short."""
    cfg = mdl.SRDiTConfig()
    f, h, w = 3, 9, 16
    want = mdl.rope_table(cfg, f, h, w, t_offset, "cpu", hw_stride=stride)
    n_pos = mdl.rope_positions(cfg, f, h, w, t_offset, stride)
    for extra in (0, int(cfg.rope_max_seq_len)):
        axes = mdl.rope_axis_tables(cfg, n_pos + extra)
        got = mdl.rope_table_from_axes(axes, f, h, w, t_offset, stride)
        assert torch.equal(torch.view_as_real(got), torch.view_as_real(want))
    short = mdl.rope_axis_tables(cfg, t_offset + f - 1)
    with pytest.raises(ValueError):
        mdl.rope_table_from_axes(short, f, h, w, t_offset, stride)
