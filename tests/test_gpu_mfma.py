"""The dense-dot matrix-core flow (DENSE_MFMA, the reference's M2
``fft_{dit,dif}_matrix[_batch]``: every Stockham butterfly a DFT-8 matrix
product on the fp32 MFMA units, the first two passes the 8 x 8 factored
DFT-64) against the CPU oracle: every core length 2..16384, forward and
inverse with every norm, ragged batches (blocks hold several transforms),
R2C / C2R around the MFMA core, and the config-5 cells N = 64..2^14 x
B in {1, 16, 64, 256}.  Gate: rel-L2 and peak-normalised max error <= 1e-5.
"""
import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import ExecutionPlan, execute_fft_plan, native

pytestmark = pytest.mark.gpu

TOL = 1e-5


def seeded(n, b, seed=0):
    rng = np.random.default_rng(102026 + 100000 * seed + 10 * n + b)
    x = (rng.standard_normal((b, n)) + 1j * rng.standard_normal((b, n))).astype(np.complex64)
    return x[0] if b == 1 else x


def check(got, ref, label):
    l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
    assert l2 <= TOL and mx <= TOL, f"{label}: rel_l2={l2:.3e} max_rel={mx:.3e}"


def mkplan(n, b, tt="c2c", td="forward", norm="backward", direction="dit"):
    name = ("fft_dit_matrix" if direction == "dit" else "fft_dif_matrix") + ("_batch" if b > 1 else "")
    return ExecutionPlan(n=n, batch=b, direction=direction, precision="fp32", selection_source="table",
                         reason="test", fallback=False, executed=name, block=256, flow_id="test",
                         flow_realization="matrix-resident", processing_unit="dense-dot-fft64", params={},
                         transform_type=tt, transform_direction=td, norm=norm)


def test_matrix_names_resolve_to_the_mfma_flow(gpu):
    from kunlunxin_fft_amd.entry import _resolve

    for n, b in ((64, 1), (4096, 3), (1 << 14, 2)):
        nplan, _ = _resolve(mkplan(n, b), 0)
        assert nplan.flow_name == "dense-mfma" and nplan.info.launches == 1
    nplan, _ = _resolve(mkplan(1 << 15, 1), 0)  # beyond the core range: the library's choice
    assert nplan.flow_name != "dense-mfma"


@pytest.mark.parametrize("n", [1 << k for k in range(1, 15)])
@pytest.mark.parametrize("b", [1, 3, 37])
def test_mfma_forward_matches_oracle(gpu, n, b):
    x = seeded(n, b)
    y = execute_fft_plan(mkplan(n, b), torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, oracle.fft_dit(x), f"dense-mfma N={n} B={b}")


@pytest.mark.parametrize("n", [2, 16, 64, 512, 4096, 1 << 14])
@pytest.mark.parametrize("norm", ["none", "forward", "backward", "ortho"])
@pytest.mark.parametrize("td", ["forward", "inverse"])
def test_mfma_all_norms(gpu, n, norm, td):
    b = 5
    x = seeded(n, b, seed=1)
    y = execute_fft_plan(mkplan(n, b, td=td, norm=norm), torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, oracle.c2c(x, td, norm), f"dense-mfma N={n} {td} {norm}")


@pytest.mark.parametrize("n", [4, 64, 1024, 1 << 15])
@pytest.mark.parametrize("b", [1, 6])
def test_mfma_core_real_flows(gpu, n, b):
    """R2C / C2R with the MFMA flow run the half-length complex core on the
    matrix cores, with the stitch / pre-twiddle kernels around it."""
    rng = np.random.default_rng(7 + n + b)
    xr = rng.standard_normal((b, n)).astype(np.float32)
    xr = xr[0] if b == 1 else xr
    X = execute_fft_plan(mkplan(n, b, tt="r2c"), torch.from_numpy(xr).to(gpu))
    check(X.cpu().numpy(), oracle.r2c_dedicated(xr), f"dense-mfma r2c N={n} B={b}")
    y = execute_fft_plan(mkplan(n, b, tt="c2r", td="inverse"), X).cpu().numpy()
    check(y, xr.astype(np.float64), f"dense-mfma r2c->c2r N={n} B={b}")


@pytest.mark.parametrize("n", [1 << k for k in range(6, 15)])
@pytest.mark.parametrize("b", [1, 16, 64, 256])
@pytest.mark.parametrize("direction", ["dit", "dif"])
def test_config5_cells_mfma_candidate(gpu, n, b, direction):
    """The FFT64 MFMA candidate on the config-5 sweep cells (N >= 64)."""
    x = seeded(n, b)
    y = execute_fft_plan(mkplan(n, b, direction=direction), torch.from_numpy(x).to(gpu)).cpu().numpy()
    ref = oracle.fft_dit(x) if n * b <= (1 << 20) else np.fft.fft(x.astype(np.complex128))
    check(y, ref, f"C5 dense-mfma N={n} B={b} {direction}")


def test_mfma_reexecution_bitwise_stable(gpu):
    x = torch.from_numpy(seeded(4096, 64, seed=2)).to(gpu)
    p = mkplan(4096, 64)
    y0 = execute_fft_plan(p, x)
    for _ in range(3):
        assert torch.equal(execute_fft_plan(p, x), y0)


def test_mfma_plan_limits(gpu):
    with pytest.raises(ValueError, match="DENSE_MFMA"):
        native.NativePlan(1 << 15, 1, "c2c", "forward", "backward", native.FLOW_DENSE_MFMA)
    with pytest.raises(ValueError, match="DENSE_MFMA"):
        native.NativePlan(1, 1, "c2c", "forward", "backward", native.FLOW_DENSE_MFMA)
    p = native.NativePlan(1 << 14, 2, "c2c", "forward", "backward", native.FLOW_DENSE_MFMA)
    assert p.info.threads_per_block == 1024 and p.workspace_size() == 0
