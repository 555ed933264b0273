"""The phase / launch ledger on the GPU (reference tests/test_ledger_hw.py
covers the same contract): the ledger observes and changes nothing (the
same bits with it on or off, no ledger left active after a headline call),
``measure_phases`` aggregates every trial, and ``launch_ledger``'s
analytic launch count and four-step geometry equal what the native plan
reports for itself (mfft_plan_query) over every flow."""
import json

import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import ExecutionPlan, entry, execute_fft_plan, ledger, plan_fft, runner

pytestmark = pytest.mark.gpu


def x_c2c(n, b, seed=7):
    g = torch.Generator().manual_seed(seed)
    return torch.complex(torch.randn(b, n, generator=g), torch.randn(b, n, generator=g)).cuda()


def with_ledger(plan, x, sync):
    led = ledger.PhaseLedger(sync=sync)
    tok = ledger.ACTIVE.set(led)
    try:
        y = execute_fft_plan(plan, x)
        torch.cuda.synchronize()
    finally:
        ledger.ACTIVE.reset(tok)
    return y, led


@pytest.mark.parametrize("tt,n", [("c2c", 512), ("r2c", 512), ("c2r", 512), ("c2c", 1 << 17)])
def test_values_identical_with_and_without_ledger(gpu, tt, n):
    td = "inverse" if tt == "c2r" else "forward"
    plan = plan_fft("dit", n, batch=4, transform_type=tt, transform_direction=td)
    if tt == "r2c":
        x = torch.randn(4, n, generator=torch.Generator().manual_seed(3)).cuda()
    elif tt == "c2r":
        x = x_c2c(n // 2 + 1, 4)
    else:
        x = x_c2c(n, 4)
    y0 = execute_fft_plan(plan, x)
    y1, led = with_ledger(plan, x, sync=False)
    assert torch.equal(y0, y1), "the ledger changed the result"
    assert [p["name"] for p in led.phases] == ["plan-validate", "core-invoke"]
    y2 = execute_fft_plan(plan, x)  # the fast path again once the ledger is gone
    assert torch.equal(y0, y2) and ledger.ACTIVE.get() is None


def test_synchronized_ledger_keeps_results(gpu):
    x = x_c2c(2048, 8)
    plan = plan_fft("dit", 2048, batch=8)
    y, led = with_ledger(plan, x, sync=True)
    ref = oracle.fft_dit(x.cpu().numpy())
    assert oracle.rel_l2(y.cpu().numpy(), ref) <= 1e-5
    s = led.summary()
    assert s["sync_added"] is True and s["kind"].startswith("fresh measured") and s["errors"] == []


def test_failing_phase_is_recorded(gpu):
    plan = plan_fft("dit", 256, batch=4)
    led = ledger.PhaseLedger(sync=True)
    tok = ledger.ACTIVE.set(led)
    try:
        with pytest.raises(ValueError, match="shape"):
            execute_fft_plan(plan, x_c2c(256, 3))
    finally:
        ledger.ACTIVE.reset(tok)
    (p,) = led.phases
    assert p["name"] == "plan-validate" and p["error"].startswith("ValueError")


def test_measure_phases_aggregates(gpu):
    plan = plan_fft("dit", 512, batch=4)
    out = ledger.measure_phases(plan, x_c2c(512, 4), trials=7, warmup=3)
    assert out["kind"].startswith("fresh measured") and out["sync_added"] is True and out["trials"] == 7
    assert out["trial_wall_p50_ms"] > 0 and out["phase_sum_mean_ms"] > 0
    for name in ("plan-validate", "core-invoke"):
        assert out["phases"][name]["calls"] == 7, name
    assert ledger.ACTIVE.get() is None
    json.dumps(out)


def mkplan(executed, n, b, params=None, tt="c2c"):
    td = "inverse" if tt == "c2r" else "forward"
    return ExecutionPlan(n=n, batch=b, direction="dit", precision="fp32", selection_source="table",
                         reason="test", fallback=False, executed=executed, block=256, params=params or {},
                         transform_type=tt, transform_direction=td)


NATIVE_CASES = [
    ("fft_lds_fused_batch", 1024, 64, {"elems": 16}, "c2c"),
    ("fft_lds_fused_batch", 4096, 8, {}, "r2c"),
    ("fft_lds_fused_batch", 4096, 8, {}, "c2r"),
    ("fft_lds_fused_batch", 1 << 16, 8, {}, "c2c"),
    ("fft_four_step_batch", 1 << 20, 4, {}, "c2c"),
    ("fft_four_step_batch", 1 << 16, 60, {"n1": 128, "chunk_rows": 16}, "c2c"),
    ("fft_four_step_batch", 1 << 18, 4, {"schedule": 2}, "c2c"),
    ("fft_four_step_batch", 1 << 18, 8, {}, "r2c"),
    ("fft_four_step_batch", 1 << 18, 8, {}, "c2r"),
    ("fft_four_step_batch", 1 << 18, 8, {"schedule": 1, "chunk_rows": 3}, "r2c"),
    ("fft_four_step_batch", 1 << 18, 8, {"schedule": 1, "chunk_rows": 3}, "c2r"),
    ("fft_four_step_batch", 1 << 18, 8, {"schedule": 1}, "c2r"),
    ("fft_four_step_batch", 1 << 20, 1, {"schedule": 3}, "c2c"),
    ("fft_four_step_batch", 1 << 18, 8, {"schedule": 3, "chunk_rows": 3}, "r2c"),
    ("fft_dit_batch", 1024, 16, {}, "c2c"),
    ("fft_dif_batch", 4096, 4, {}, "r2c"),
    ("fft_dit_radix4_batch", 2048, 4, {}, "c2c"),
    ("fft_dif_radix4_batch", 4096, 4, {}, "c2r"),
    ("fft_dit_matrix_batch", 2048, 4, {}, "c2c"),
    ("fft_dif_matrix_batch", 1024, 4, {}, "r2c"),
    ("fft_dit", 1, 1, {}, "c2c"),
    ("fft_dit_fused", 1 << 16, 2, {}, "c2c"),
    ("run_hybrid", 4096, 4, {"flow_kind": "composition", "tile": 64, "core": "local"}, "c2c"),
]


@pytest.mark.parametrize("case", NATIVE_CASES, ids=[f"{c[0]}-{c[1]}-{c[2]}-{c[4]}" for c in NATIVE_CASES])
def test_launch_ledger_matches_the_native_plan(gpu, case):
    executed, n, b, params, tt = case
    plan = mkplan(executed, n, b, params, tt)
    lg = ledger.launch_ledger(plan)
    nat = runner.get_native_plan(executed, n, b, tt, plan.transform_direction, plan.norm, plan.block, params,
                                 torch.cuda.current_device())
    info = nat.info
    assert lg["available"] and lg["launches"] == info.launches, (lg["launches"], info.launches)
    assert lg["flow"] == nat.flow_name
    if lg["flow"] == "four-step":
        assert (lg["n1"], lg["n2"]) == (info.n1, info.n2)
        assert lg["chunk_rows"] == (info.chunk_rows if 0 < info.chunk_rows < b else b)


def test_headline_path_has_no_active_ledger(gpu):
    assert ledger.ACTIVE.get() is None
    plan = plan_fft("dit", 256, batch=4)
    x = x_c2c(256, 4)
    execute_fft_plan(plan, x)
    execute_fft_plan(plan, x)
    assert ledger.ACTIVE.get() is None and id(plan) in entry._FAST
    np.testing.assert_array_equal(execute_fft_plan(plan, x).cpu().numpy(), execute_fft_plan(plan, x).cpu().numpy())
