"""The reference's runner names on the GPU, through ``execute_fft_plan`` and
through the tensor-level runner functions: the M1 (``fft_dit_fused``), M2
(``fft_{dit,dif}_matrix[_batch]``), M3 (``fft_{dit,dif}_grouped``) and
hybrid (``run_hybrid``, a composition plan) names run this build's LDS /
four-step kernels and must give the oracle's transform; and the
``twiddle=`` contract of the stage runners (validated, used when it holds
the forward roots, ValueError otherwise).
"""
import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import ExecutionPlan, execute_fft_plan, runner
from kunlunxin_fft_amd.entry import _composition_plan

pytestmark = pytest.mark.gpu

TOL = 1e-5


def seeded(n, b, seed):
    rng = np.random.default_rng(seed + 10 * n + b)
    x = (rng.standard_normal((b, n)) + 1j * rng.standard_normal((b, n))).astype(np.complex64)
    return x[0] if b == 1 else x


def check(got, ref, label):
    l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
    assert l2 <= TOL and mx <= TOL, f"{label}: rel_l2={l2:.3e} max_rel={mx:.3e}"


def ref_fft(x):
    return oracle.fft_dit(x) if x.size <= (1 << 16) else np.fft.fft(x.astype(np.complex128))


def mkplan(executed, n, b, params=None, td="forward", norm="backward"):
    return ExecutionPlan(n=n, batch=b, direction="dit", precision="fp32", selection_source="table",
                         reason="test", fallback=False, executed=executed, block=256, flow_id="test",
                         flow_realization="test", processing_unit="test", params=params or {},
                         transform_direction=td, norm=norm)


SINGLE = ["fft_dit_fused", "fft_dit_matrix", "fft_dif_matrix", "fft_dit_grouped", "fft_dif_grouped"]
BATCH = ["fft_dit_matrix_batch", "fft_dif_matrix_batch"]


@pytest.mark.parametrize("name", SINGLE)
@pytest.mark.parametrize("n", [16, 64, 1024, 1 << 15, 1 << 16, 1 << 20])
def test_alias_names_single(gpu, name, n):
    x = seeded(n, 1, 31)
    y = execute_fft_plan(mkplan(name, n, 1), torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, ref_fft(x), f"{name} N={n}")


@pytest.mark.parametrize("name", BATCH)
@pytest.mark.parametrize("n,b", [(64, 3), (2048, 16), (1 << 14, 5), (1 << 17, 2)])
def test_alias_names_batch(gpu, name, n, b):
    x = seeded(n, b, 32)
    y = execute_fft_plan(mkplan(name, n, b), torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, ref_fft(x), f"{name} N={n} B={b}")


@pytest.mark.parametrize("n,b,tile", [(2048, 16, 64), (1 << 12, 1, 32), (1 << 16, 3, 256)])
def test_run_hybrid_composition_plan(gpu, n, b, tile):
    """A composition plan (selection_source "composition", runner
    run_hybrid with the entry's tile) runs the four-step with n1 = N/tile."""
    comp = {"flow_id": "hybrid-test", "flow_realization": "four-step", "processing_unit": "stockham-radix16",
            "guard_pct": 5.0, "reason": "test", "tile": tile}
    plan = _composition_plan(comp, n, b, "dit", "fp32", "forward", "backward")
    assert plan.executed == "run_hybrid" and plan.selection_source == "composition"
    x = seeded(n, b, 33)
    y = execute_fft_plan(plan, torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, ref_fft(x), f"run_hybrid N={n} B={b} tile={tile}")


@pytest.mark.parametrize("fn,n", [("fft_dit_fused", 4096), ("fft_dit_matrix", 256), ("fft_dif_matrix", 1 << 16),
                                  ("fft_dit_grouped", 512), ("fft_dif_grouped", 1 << 18)])
def test_alias_runner_functions(gpu, fn, n):
    x = seeded(n, 1, 34)
    y = getattr(runner, fn)(torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, ref_fft(x), f"runner.{fn} N={n}")


@pytest.mark.parametrize("fn", ["fft_dit_matrix_batch", "fft_dif_matrix_batch"])
def test_alias_runner_batch_functions(gpu, fn):
    x = seeded(1024, 4, 35)
    y = getattr(runner, fn)(torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, ref_fft(x), f"runner.{fn}")


@pytest.mark.parametrize("fn", ["fft_dit", "fft_dif", "fft_dit_radix4", "fft_dif_radix4"])
@pytest.mark.parametrize("n", [8, 1024, 1 << 16])
def test_twiddle_contract(gpu, fn, n):
    """A table of the forward roots (the reference's own float32-angle
    tables, or this build's) gives the same result as no table; a table
    of other values, the wrong length, dtype or device raises."""
    x = torch.from_numpy(seeded(n, 1, 36)).to(gpu)
    f = getattr(runner, fn)
    y0 = f(x).cpu().numpy()
    check(y0, ref_fft(x.cpu().numpy()), f"{fn} N={n}")
    idx = torch.arange(n >> 1, device=gpu, dtype=torch.float32)
    ang = (-2.0 * np.pi * idx / n).to(torch.float32)  # reference runner.py:93-97
    ref_tables = (torch.cos(ang), torch.sin(ang))
    for tw in (ref_tables, runner.twiddle_tables(n, gpu)):
        np.testing.assert_array_equal(f(x, twiddle=tw).cpu().numpy(), y0)
    bad = (ref_tables[0].clone(), ref_tables[1].clone())
    bad[1][-1] += 1e-3
    with pytest.raises(ValueError, match="differs"):
        f(x, twiddle=bad)
    with pytest.raises(ValueError, match="length"):
        f(x, twiddle=(ref_tables[0][:-1], ref_tables[1][:-1]))
    with pytest.raises(TypeError, match="float32"):
        f(x, twiddle=(ref_tables[0].double(), ref_tables[1]))
    with pytest.raises(ValueError, match="device"):
        f(x, twiddle=(ref_tables[0].cpu(), ref_tables[1].cpu()))
    with pytest.raises(TypeError, match="tuple"):
        f(x, twiddle=[ref_tables[0], ref_tables[1]])


# ---- the reference's full keyword sets (src/xpu/runner.py:118-1472) on the GPU

BATCH_STAGE = ["fft_dit_batch", "fft_dif_batch", "fft_dit_radix4_batch", "fft_dif_radix4_batch"]


@pytest.mark.parametrize("fn", BATCH_STAGE)
@pytest.mark.parametrize("variant", ["spread", "folded"])
@pytest.mark.parametrize("block", [64, 1024, 2048])
def test_batch_stage_runners_reference_keywords(gpu, fn, variant, block):
    """Both variants, the reference's default block (1024), a block above
    a workgroup's 1024 threads (clamped) and a forward-roots twiddle table
    give the oracle's transform; the twiddle table changes nothing."""
    n, b = 1024, 4
    x = torch.from_numpy(seeded(n, b, 37)).to(gpu)
    f = getattr(runner, fn)
    if "radix4" in fn and variant == "folded":  # the reference lowers 'spread' only for radix-4 batches
        with pytest.raises(ValueError, match="spread"):
            f(x, block=block, variant=variant)
        return
    y = f(x, block=block, variant=variant).cpu().numpy()
    check(y, ref_fft(x.cpu().numpy()), f"{fn} block={block} variant={variant}")
    np.testing.assert_array_equal(f(x, block, variant, runner.twiddle_tables(n, gpu)).cpu().numpy(), y)


@pytest.mark.parametrize("fn", ["fft_dit", "fft_dif", "fft_dit_radix4", "fft_dif_radix4"])
@pytest.mark.parametrize("n", [4, 8, 2048])
def test_stage_runners_default_block(gpu, fn, n):
    """block=1024 (the reference's default) over fewer butterflies than
    threads: the stage kernels' bounds checks hold."""
    x = torch.from_numpy(seeded(n, 1, 38)).to(gpu)
    check(getattr(runner, fn)(x).cpu().numpy(), ref_fft(x.cpu().numpy()), f"{fn} N={n}")


@pytest.mark.parametrize("fn,args", [
    ("fft_dit_fused", dict(block=256, tile=32)),
    ("fft_dit_matrix", dict(block=512, tile=64, rows=16)),
    ("fft_dif_matrix", dict(block=512, tile=128, rows=4)),
    ("fft_dit_grouped", dict(block=1024, tile=64, rows=8, glog=3, maxp=2048, cells=2)),
    ("fft_dif_grouped", dict(block=1024, tile=64, rows=8, glog=2, maxp=4096, cells=1)),
])
def test_alias_runners_reference_keywords(gpu, fn, args):
    n = 4096
    x = torch.from_numpy(seeded(n, 1, 39)).to(gpu)
    y = getattr(runner, fn)(x, twiddle=runner.twiddle_tables(n, gpu), **args).cpu().numpy()
    check(y, ref_fft(x.cpu().numpy()), f"runner.{fn} {args}")


@pytest.mark.parametrize("fn", ["fft_dit_matrix_batch", "fft_dif_matrix_batch", "fft_dit_matrix_packet_batch"])
def test_matrix_batch_runners_reference_keywords(gpu, fn):
    n, b = 512, 4
    x = torch.from_numpy(seeded(n, b, 40)).to(gpu)
    kw = dict(block=1024, tile=64, rows=8, twiddle=runner.twiddle_tables(n, gpu))
    kw.update({"packets": 2} if "packet" in fn else {"variant": "spread"})
    y = getattr(runner, fn)(x, **kw).cpu().numpy()
    check(y, ref_fft(x.cpu().numpy()), f"runner.{fn}")


def test_batch_runner_contract_errors(gpu):
    """The reference's batch-runner errors (test_fft.py:405-419, 456-465,
    483-497) on the GPU, before any launch: 'folded' for the matrix and
    radix-4 batches, a rank-1 input, a block that is not a power of two,
    a batch that is not a power of two, and the packet runner's limits."""
    good = torch.complex(torch.ones(4, 64, device=gpu), torch.zeros(4, 64, device=gpu))
    for fn in ("fft_dit_matrix_batch", "fft_dif_matrix_batch", "fft_dit_radix4_batch", "fft_dif_radix4_batch"):
        with pytest.raises(ValueError, match="spread"):
            getattr(runner, fn)(good, variant="folded")
    with pytest.raises(ValueError):
        runner.fft_dit_matrix_batch(good.view(-1))
    with pytest.raises(ValueError):
        runner.fft_dit_matrix_batch(good, block=1000)
    with pytest.raises(ValueError, match="power of two"):
        runner.fft_dit_batch(torch.ones((3, 64), dtype=torch.complex64, device=gpu))
    x16 = torch.ones((16, 1024), dtype=torch.complex64, device=gpu)
    with pytest.raises(ValueError, match="ceiling"):
        runner.fft_dit_matrix_packet_batch(x16, packets=4)
    with pytest.raises(ValueError, match="power of two"):
        runner.fft_dit_matrix_packet_batch(x16, packets=3)
    with pytest.raises(ValueError, match="divide"):
        runner.fft_dit_matrix_packet_batch(x16[:1], packets=2)
    for packets in (1, 2):
        y = runner.fft_dit_matrix_packet_batch(x16, packets=packets).cpu().numpy()
        check(y, np.fft.fft(x16.cpu().numpy().astype(np.complex128), axis=-1), f"packet batch packets={packets}")


def test_bit_reverse_permute_block_keyword(gpu):
    n = 256
    x = torch.arange(n, dtype=torch.float32).to(torch.complex64).to(gpu)
    y = runner.bit_reverse_permute(x, block=1024).cpu().real.to(torch.int64).numpy()
    assert [int(y[oracle.bit_reverse(i, 8)]) for i in range(n)] == list(range(n))
    with pytest.raises(ValueError, match="power of two"):
        runner.bit_reverse_permute(x, block=1000)


def test_time_call_detailed_on_a_plan(gpu):
    """The reference's trial protocol on an execute: shuffled trials, api
    wall time and device (event) time, both positive, device time the
    smaller."""
    from kunlunxin_fft_amd import plan_fft

    plan = plan_fft("dit", 2048, batch=16)
    x = torch.from_numpy(seeded(2048, 16, 41)).to(gpu)
    d = runner.time_call_detailed(lambda: execute_fft_plan(plan, x), warmup=3, trials=20, seed=0)
    assert d["api_ms"]["trials"] == 20 and d["kernel_ms"] is not None
    assert 0 < d["kernel_ms"]["median"] <= d["api_ms"]["median"]
    assert "api_ms" in d["metric_note"] and "kernel_ms" in d["metric_note"]
    ms = runner.time_call(lambda: execute_fft_plan(plan, x), warmup=2, iters=10)
    assert 0 < ms < 1000


def test_xpu_context_guard(gpu):
    prev = torch.cuda.current_device()
    with runner.xpu_context(0) as idx:
        assert idx == 0 and torch.cuda.current_device() == 0
    assert torch.cuda.current_device() == prev


def test_device_name_and_index(gpu):
    name = runner.device_name()
    assert "gfx950" in name and "CUs" in name, name
    assert runner.current_device_index() == torch.cuda.current_device()
