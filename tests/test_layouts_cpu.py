"""Row layouts the wrappers hand to the kernels: a size-1 dim's stride is arbitrary (torch's
views and reshapes set it freely), so it must neither set nor veto the token stride. The
DeltaNet output gate at one verify row per lane, `proj[..., a:b].reshape(B, 1, heads, dim)`,
is such a view: its size-1 dim carries the head block's extent, not the row pitch."""

from __future__ import annotations

import pytest
import torch

import _mtpk
import rownorm


def test_gate_slice_of_one_row_per_lane():
    b, vh, vd = 4, 64, 128
    proj = torch.zeros(b, 1, 3 * vh * vd)
    z = proj[..., vh * vd : 2 * vh * vd].reshape(b, 1, vh, vd)
    assert z.stride(1) != z.stride(0)  # the arbitrary stride the layout must ignore
    ts, hs, hpt, rows = rownorm._layout(z, heads=True)
    assert (ts, hs, hpt, rows) == (3 * vh * vd, vd, vh, b * vh)
    assert _mtpk.row_stride(proj) == 3 * vh * vd


@pytest.mark.parametrize("t", [1, 4])
def test_token_stride_matches_element_addresses(t):
    """Element (token i, head h, 0) sits at i * ts + h * hs for every layout accepted."""
    b, heads, dim = 3, 5, 16
    base = torch.arange(b * t * 7 * dim).reshape(b, t, 7 * dim)
    x = base[..., dim : dim + heads * dim].reshape(b, t, heads, dim)
    ts, hs, hpt, rows = rownorm._layout(x, heads=True)
    origin = int(x[0, 0, 0, 0])  # base holds each element's own storage offset
    for i in range(b):
        for s in range(t):
            for h in range(heads):
                assert int(x[i, s, h, 0]) - origin == (i * t + s) * ts + h * hs
    assert rows == b * t * heads and hpt == heads


def test_rows_that_do_not_collapse_are_refused():
    x = torch.zeros(4, 6, 32)[:, :3]  # [4, 3, 32]: stride(0) = 6 * 32 != 3 * stride(1)
    with pytest.raises(ValueError):
        rownorm._layout(x, heads=False)
    assert _mtpk.row_stride(x) is None
    assert _mtpk.row_stride(torch.zeros(1, 3, 32)[:, :, :8]) == 32
