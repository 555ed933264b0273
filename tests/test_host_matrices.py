"""The M2 / M3 host matrices (matrices.py; reference src/xpu/matrices.py):
the local-group matrix against the block-local stages applied pair by pair
and, composed with the global stages, against np.fft.fft; its unitarity
(M^H M = T I) and planar layout; the tail-group tables against their stages
and, with the local group, against np.fft.fft; and the tail partition.
Host-only: the module imports no torch."""
import os

import numpy as np
import pytest

from kunlunxin_fft_amd import matrices


def test_matrices_module_is_host_only():
    src = open(os.path.join(os.path.dirname(matrices.__file__), "matrices.py")).read()
    assert "import torch" not in src and "import triton" not in src


@pytest.mark.parametrize("tile", [2, 8, 16, 64, 128])
@pytest.mark.parametrize("direction", ["dit", "dif"])
def test_local_matrix_against_stage_loops(tile, direction):
    assert matrices.verify_local_matrix(tile, direction) < 1e-12


@pytest.mark.parametrize("n,tile", [(64, 64), (256, 64), (4096, 64), (4096, 8), (1024, 128), (32, 64)])
@pytest.mark.parametrize("direction", ["dit", "dif"])
def test_local_group_and_global_stages_give_the_dft(n, tile, direction):
    assert matrices.verify_decomposition(n, tile, direction) < 1e-12


@pytest.mark.parametrize("tile", [8, 64])
@pytest.mark.parametrize("direction", ["dit", "dif"])
def test_local_matrix_unitarity_and_layout(tile, direction):
    m = matrices.local_matrix(tile, direction)
    assert m.shape == (tile, tile) and m.dtype == np.complex128
    assert np.allclose(m.conj().T @ m, tile * np.eye(tile), atol=1e-10)
    mr, mi = matrices.local_matrix_planar(tile, direction)
    assert mr.shape == (tile, tile) and mr.dtype == np.float32 and mi.dtype == np.float32
    assert mr.flags["C_CONTIGUOUS"] and mi.flags["C_CONTIGUOUS"]
    np.testing.assert_allclose(mr + 1j * mi, m.T, atol=1e-6)


def test_local_matrix_closed_forms():
    """The whole block: DIT M @ bitrev(x) = fft(x), DIF bitrev(M @ x) = fft(x)."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(16) + 1j * rng.standard_normal(16)
    br = np.array([int(f"{i:04b}"[::-1], 2) for i in range(16)])
    np.testing.assert_allclose(matrices.local_matrix(16, "dit") @ x[br], np.fft.fft(x), atol=1e-12)
    np.testing.assert_allclose((matrices.local_matrix(16, "dif") @ x)[br], np.fft.fft(x), atol=1e-12)
    with pytest.raises(ValueError, match="direction"):
        matrices.local_matrix(16, "both")
    with pytest.raises(ValueError, match="power of two"):
        matrices.local_matrix(12)


@pytest.mark.parametrize("n0", [1, 2, 4, 8, 16, 64])
@pytest.mark.parametrize("glog", [1, 2, 3])
@pytest.mark.parametrize("direction", ["dit", "dif"])
def test_tail_group_table_against_stage_loops(n0, glog, direction):
    assert matrices.verify_tail_group(n0, glog, direction) < 1e-10
    cr, ci = matrices.tail_group_planar(n0, glog, direction)
    assert cr.shape == (1 << glog, n0 << glog) and cr.dtype == np.float32 and cr.flags["C_CONTIGUOUS"]


@pytest.mark.parametrize("tile,glog", [(8, 1), (8, 2), (8, 3), (16, 2), (64, 2), (64, 3)])
@pytest.mark.parametrize("direction", ["dit", "dif"])
def test_grouped_decomposition_gives_the_dft(tile, glog, direction):
    assert matrices.verify_grouped_decomposition(tile << glog, tile, glog, direction) < 1e-12
    with pytest.raises(ValueError, match="tile << glog"):
        matrices.verify_grouped_decomposition((tile << glog) * 2, tile, glog, direction)


@pytest.mark.parametrize("tile,logn,glog,maxp", [
    (8, 16, 2, 4096), (8, 16, 1, 4096), (64, 16, 3, 8192), (64, 16, 3, 128),
    (16, 20, 2, 1024), (64, 16, 2, 8192), (8, 4, 2, 4096), (64, 16, 4, 4096)])
def test_tail_groups_partition(tile, logn, glog, maxp):
    groups, singles = matrices.tail_groups(tile, logn, glog, maxp)
    covered = sorted([n0 << s for n0, g in groups for s in range(g)] + list(singles))
    assert covered == [1 << s for s in range(tile.bit_length() - 1, logn)]
    assert all(2 <= g <= max(glog, 2) and (n0 << g) <= maxp for n0, g in groups)
    periods = [n0 << g for n0, g in groups]
    assert periods == sorted(periods)
    if glog == 1:
        assert groups == []  # a group has at least two stages
    if singles and groups:
        last = groups[-1][0] << (groups[-1][1] - 1)
        assert all(s > last for s in singles)


def test_tail_groups_greedy_choice():
    """From the smallest stage up, each group takes the most stages that fit."""
    assert matrices.tail_groups(8, 8, 3, 4096) == ([(8, 3), (64, 2)], [])
    assert matrices.tail_groups(64, 16, 3, 128) == ([], [1 << s for s in range(6, 16)])
    assert matrices.tail_groups(8, 6, 2, 32) == ([(8, 2)], [32])
