"""Four-step compositions around an external sub-FFT core (reference
src/xpu/adapter_hybrid.py run_hybrid, composition.py): the vendor core
(rocFFT through torch.fft) and the local core (this library's four-step)
against the CPU oracle, through run_hybrid and through execute_fft_plan on a
composition plan; and the twiddle-transpose boundary kernel
(mfft_twiddle_transpose) against numpy."""
import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import execute_fft_plan, native
from kunlunxin_fft_amd.entry import _composition_plan
from kunlunxin_fft_amd.hybrid import plan_hybrid, run_hybrid

pytestmark = pytest.mark.gpu

TOL = 1e-5


def seeded(n, b, seed):
    rng = np.random.default_rng(seed + 10 * n + b)
    x = (rng.standard_normal((b, n)) + 1j * rng.standard_normal((b, n))).astype(np.complex64)
    return x[0] if b == 1 else x


def check(got, ref, label):
    l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
    assert l2 <= TOL and mx <= TOL, f"{label}: rel_l2={l2:.3e} max_rel={mx:.3e}"


@pytest.mark.parametrize("rows,cols,b", [(32, 32, 1), (16, 128, 3), (64, 32, 2), (1024, 1024, 1), (2, 16, 5),
                                         (64, 1, 2)])
@pytest.mark.parametrize("td", ["forward", "inverse"])
def test_twiddle_transpose(gpu, rows, cols, b, td):
    rng = np.random.default_rng(rows * 7 + cols)
    s = (rng.standard_normal((b, rows, cols)) + 1j * rng.standard_normal((b, rows, cols))).astype(np.complex64)
    out = torch.empty((b, cols, rows), dtype=torch.complex64, device=gpu)
    native.twiddle_transpose(torch.from_numpy(s).to(gpu).data_ptr(), out.data_ptr(), rows, cols, b, td,
                             torch.cuda.current_stream(gpu).cuda_stream)
    n = rows * cols
    sign = -1.0 if td == "forward" else 1.0
    w = np.exp(sign * 2j * np.pi * np.outer(np.arange(rows), np.arange(cols)) / n)
    ref = np.transpose(s.astype(np.complex128) * w, (0, 2, 1))
    got = out.cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-6 * np.abs(ref).max()


def test_twiddle_transpose_rejects_bad_shapes(gpu):
    x = torch.zeros(64, dtype=torch.complex64, device=gpu)
    y = torch.zeros(64, dtype=torch.complex64, device=gpu)
    st = torch.cuda.current_stream(gpu).cuda_stream
    with pytest.raises(ValueError, match="powers of two"):
        native.twiddle_transpose(x.data_ptr(), y.data_ptr(), 6, 8, 1, "forward", st)
    with pytest.raises(ValueError, match="overlap"):
        native.twiddle_transpose(x.data_ptr(), x.data_ptr(), 8, 8, 1, "forward", st)


HYBRID_SHAPES = [(1024, 1, 32), (2048, 16, 64), (4096, 64, 16), (2048, 1, 128), (1 << 16, 4, 256), (1 << 12, 3, 2)]


# the local core needs tile and N/tile in [16, 1024] (plan_hybrid rejects
# other splits for it: tests/test_host_entry.py::test_hybrid_plan_contract)
@pytest.mark.parametrize("n,b,tile,core", [(n, b, t, core) for core in ("vendor", "local") for n, b, t in HYBRID_SHAPES
                                           if core == "vendor" or (16 <= t <= 1024 and 16 <= n // t <= 1024)])
def test_run_hybrid_matches_oracle(gpu, n, b, tile, core):
    x = seeded(n, b, 61)
    y = run_hybrid(torch.from_numpy(x).to(gpu), plan_hybrid(n, b, tile=tile, core=core)).cpu().numpy()
    check(y, oracle.fft_dit(x), f"run_hybrid {core} N={n} B={b} tile={tile}")


@pytest.mark.parametrize("td,norm", [("inverse", "backward"), ("forward", "ortho"), ("inverse", "none")])
def test_run_hybrid_vendor_inverse_and_norms(gpu, td, norm):
    n, b, tile = 2048, 8, 64
    x = seeded(n, b, 62)
    y = run_hybrid(torch.from_numpy(x).to(gpu), plan_hybrid(n, b, tile=tile, transform_direction=td,
                                                            norm=norm)).cpu().numpy()
    check(y, oracle.c2c(x, td, norm), f"run_hybrid vendor {td} {norm}")


@pytest.mark.parametrize("core", ["vendor", "local"])
def test_composition_plan_executes_its_core(gpu, core):
    """execute_fft_plan on a composition plan runs the entry's core: the
    vendor core through run_hybrid (rocFFT sub-FFTs + the boundary kernel),
    the local core as one native four-step plan."""
    n, b, tile = 2048, 16, 64
    comp = {"flow_id": f"composition-{core}", "flow_realization": "four-step-composition",
            "processing_unit": core, "guard_pct": 5.0, "reason": "test", "tile": tile, "core": core}
    plan = _composition_plan(comp, n, b, "dit", "fp32", "forward", "backward")
    x = seeded(n, b, 63)
    y = execute_fft_plan(plan, torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, oracle.fft_dit(x), f"composition plan {core}")


@pytest.mark.parametrize("core,n,b,tile", [("vendor", 1024, 16, 64), ("vendor", 1 << 16, 2, 256),
                                           ("local", 1024, 16, 64), ("local", 1 << 16, 2, 256)])
def test_profile_hybrid_matches_run_hybrid(gpu, core, n, b, tile):
    """profile_hybrid gives run_hybrid's bits and times every phase
    (reference tests/test_adapter_hybrid.py:141-164)."""
    from kunlunxin_fft_amd.hybrid import profile_hybrid

    x = torch.from_numpy(seeded(n, b, 7)).to(gpu)
    plan = plan_hybrid(n, b, tile, core)
    y1 = run_hybrid(x, plan)
    y2, phases = profile_hybrid(x, plan)
    assert torch.equal(y1, y2)
    check(y2.cpu().numpy(), oracle.fft_dit(x.cpu().numpy()) if n <= 4096 else
          np.fft.fft(x.cpu().numpy().astype(np.complex128)), f"profile_hybrid {core} N={n}")
    assert phases["core"] == core and phases["hidden_copies"] == []
    if core == "vendor":
        for key in ("gather_ms", "stage1_core_ms", "twiddle_transpose_ms", "stage2_core_ms", "scatter_ms"):
            assert phases[key] >= 0.0, key
        assert phases["stage2_in_contiguous"] is True and phases["stage1_out_contiguous"] is True
    else:
        assert phases["fused_four_step_ms"] > 0.0


def test_time_cell_summarises_every_trial(gpu):
    from kunlunxin_fft_amd.hybrid import time_cell

    x = torch.from_numpy(seeded(4096, 8, 3)).to(gpu)
    plan = plan_hybrid(4096, 8, 64, "local")
    first_ms, stats = time_cell(lambda t: run_hybrid(t, plan), x, warmup=3, trials=11)
    assert first_ms > 0 and stats["n"] == 11 and 0 < stats["p50"] <= stats["max"]
