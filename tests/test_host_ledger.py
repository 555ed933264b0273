"""The phase / launch ledger on the host (reference tests/test_ledger_host.py
covers the same contract): the phase hook is a shared no-op without an
active ledger, records and re-raises with one; ``launch_ledger`` gives this
library's launches and HBM bytes for every flow, with the closed forms
below (the same ones the GPU test checks against the native plan's own
launch count); ``batch_fill_analysis`` keeps the reference's 1.5x rule.
No GPU needed."""
import json

import pytest

from kunlunxin_fft_amd import ExecutionPlan, ledger


def plan(executed, n=1024, batch=16, params=None, transform_type="c2c", transform_direction="forward",
         norm="backward", block=256):
    return ExecutionPlan(n=n, batch=batch, direction="dit", precision="fp32", selection_source="table",
                         reason="t", fallback=False, executed=executed, block=block, params=params or {},
                         transform_type=transform_type, transform_direction=transform_direction, norm=norm)


def test_phase_noop_when_inactive():
    assert ledger.current_ledger() is None
    ctx = ledger.phase("core-invoke")
    for _ in range(3):
        with ledger.phase("core-invoke") as v:
            assert v is None
        assert ledger.phase("plan-validate") is ctx  # one shared object: nothing allocated per call


def test_phase_records_on_active_ledger():
    led = ledger.PhaseLedger(sync=False)
    tok = ledger.ACTIVE.set(led)
    try:
        with ledger.phase("plan-validate"):
            pass
        with ledger.phase("core-invoke"):
            pass
        with ledger.phase("core-invoke"):
            pass
    finally:
        ledger.ACTIVE.reset(tok)
    assert ledger.current_ledger() is None
    assert [p["name"] for p in led.phases] == ["plan-validate", "core-invoke", "core-invoke"]
    s = led.summary()
    assert s["kind"].startswith("fresh measured") and s["sync_added"] is False
    assert s["phase_order"] == ["plan-validate", "core-invoke"]
    assert s["phases"]["core-invoke"]["calls"] == 2 and s["phases"]["plan-validate"]["calls"] == 1
    assert s["phases"]["core-invoke"]["max_ms"] >= s["phases"]["core-invoke"]["p50_ms"] >= 0.0
    assert s["errors"] == []
    json.dumps(s)


def test_phase_records_error_and_reraises():
    led = ledger.PhaseLedger(sync=False)
    with pytest.raises(ValueError, match="boom"):
        with led.phase("core-invoke"):
            raise ValueError("boom")
    assert led.phases[0]["error"] == "ValueError: boom"
    assert led.summary()["errors"] == [{"name": "core-invoke", "error": "ValueError: boom"}]


# (executed, n, batch, params, transform_type) -> (family, launches, HBM bytes over algorithmic bytes)
CASES = [
    (("fft_lds_fused_batch", 1024, 64, {"elems": 16}, "c2c"), ("lds-single-pass", 1, 1.0)),
    (("fft_lds_fused", 32768, 1, {}, "c2c"), ("lds-single-pass", 1, 1.0)),
    (("fft_four_step_batch", 1 << 20, 64, {}, "c2c"), ("four-step-two-pass", 2, 2.0)),
    (("fft_four_step_batch", 1 << 16, 64, {"n1": 128, "chunk_rows": 16}, "c2c"), ("four-step-two-pass", 8, 2.0)),
    (("fft_four_step_batch", 1 << 16, 60, {"chunk_rows": 16}, "c2c"), ("four-step-two-pass", 8, 2.0)),
    (("fft_four_step_batch", 1 << 18, 4, {"schedule": 2}, "c2c"), ("four-step-fused-l2", 2, 1.0)),
    (("fft_dit_batch", 1024, 64, {}, "c2c"), ("stage-radix2", 10, 10.0)),
    (("fft_dif", 2048, 1, {}, "c2c"), ("stage-radix2", 11, 11.0)),
    (("fft_dit_radix4_batch", 1024, 64, {}, "c2c"), ("stage-radix4", 5, 5.0)),
    (("fft_dif_radix4_batch", 2048, 8, {}, "c2c"), ("stage-radix4", 6, 6.0)),
    (("fft_dit_matrix_batch", 2048, 16, {}, "c2c"), ("dense-mfma", 1, 1.0)),
    (("fft_dit", 1, 1, {}, "c2c"), ("lds-single-pass", 1, 1.0)),        # no stage: the library picks
    (("fft_dit_fused", 1 << 16, 4, {}, "c2c"), ("four-step-two-pass", 2, 2.0)),
    (("fft_dif_grouped", 4096, 4, {}, "c2c"), ("lds-single-pass", 1, 1.0)),
    (("fft_lds_fused_batch", 1 << 16, 8, {}, "c2c"), ("four-step-two-pass", 2, 2.0)),  # past the LDS core
]


@pytest.mark.parametrize("args,want", CASES, ids=[f"{a[0]}-{a[1]}-{a[2]}" for a, _ in CASES])
def test_launch_ledger_c2c_closed_forms(args, want):
    executed, n, b, params, tt = args
    lg = ledger.launch_ledger(plan(executed, n, b, params, tt))
    family, launches, ratio = want
    assert lg["available"] is True and lg["estimate"] is True and lg["kind"].startswith("analytic estimate")
    assert (lg["family"], lg["launches"]) == (family, launches)
    assert lg["algorithmic_bytes"] == 16 * n * b
    assert lg["gm_bytes"] == round(ratio * 16 * n * b)
    logn = n.bit_length() - 1
    assert lg["flops"] == 5.0 * n * logn * b
    json.dumps(lg)


def test_four_step_geometry():
    lg = ledger.launch_ledger(plan("fft_four_step_batch", 1 << 20, 64))
    assert (lg["n1"], lg["n2"], lg["chunk_rows"], lg["schedule"]) == (1024, 1024, 64, 0)
    lg = ledger.launch_ledger(plan("fft_four_step_batch", 1 << 17, 64, {"n1": 256, "chunk_rows": 32}))
    assert (lg["n1"], lg["n2"], lg["chunk_rows"]) == (256, 512, 32)
    # an n1 the library cannot split with falls back to the default split
    lg = ledger.launch_ledger(plan("fft_four_step_batch", 1 << 17, 64, {"n1": 8}))
    assert (lg["n1"], lg["n2"]) == (256, 512)


def test_reference_family_is_reported_beside_this_library_flow():
    assert ledger.launch_ledger(plan("fft_dit", 1024, 1))["reference_family"] == "baseline_m0_rank1_loop"
    assert ledger.launch_ledger(plan("fft_dit_batch"))["reference_family"] == "incumbent_m4_folded"
    assert ledger.launch_ledger(plan("fft_dit_radix4_batch"))["reference_family"] == "m5_batch"
    assert ledger.launch_ledger(plan("fft_dit_matrix_batch"))["reference_family"] == "m2_batch"
    assert ledger.launch_ledger(plan("fft_lds_fused_batch"))["reference_family"] is None
    # the reference's folded radix-2 count is this library's too: log2(n) launches of 2*8*n*b bytes
    lg = ledger.launch_ledger(plan("fft_dit_batch", 1024, 64))
    assert lg["launches"] == 10 and lg["gm_bytes"] == 10 * 2 * 1024 * 64 * 8


def test_real_flows_fused_and_not():
    n, b = 4096, 8
    half, zrow = 8 * (n // 2 + 1) * b, 8 * (n // 2) * b
    alg_r2c = 4 * n * b + half
    # LDS: stitch in the core's store, one launch, algorithmic bytes only
    lg = ledger.launch_ledger(plan("fft_lds_fused_batch", n, b, transform_type="r2c"))
    assert lg["launches"] == 1 and lg["epilogue_launches"] == 0 and lg["gm_bytes"] == alg_r2c
    assert all(o["fused"] and o["in_bytes"] == 0 for o in lg["real_compat_ops"])
    assert any("stitch" in o["op"] for o in lg["real_compat_ops"])
    assert lg["flops"] == 5.0 * (n // 2) * 11 * b + 10.0 * (n // 4 + 1) * b
    # a stage flow: log2(n/2) launches plus the stitch kernel over the half spectrum
    lg = ledger.launch_ledger(plan("fft_dit_batch", n, b, transform_type="r2c"))
    assert (lg["core_launches"], lg["epilogue_launches"], lg["launches"]) == (11, 1, 12)
    assert lg["gm_bytes"] == 11 * 2 * zrow + zrow + half
    (stitch,) = [o for o in lg["real_compat_ops"] if "stitch" in o["op"]]
    assert stitch["fused"] is False and (stitch["in_bytes"], stitch["out_bytes"]) == (zrow, half)
    # c2r on the stage flow: the pre-twiddle kernel first
    lg = ledger.launch_ledger(plan("fft_dit_radix4_batch", n, b, transform_type="c2r",
                                   transform_direction="inverse"))
    assert (lg["core_launches"], lg["epilogue_launches"]) == (6, 1)
    assert lg["gm_bytes"] == 6 * 2 * zrow + half + zrow
    ops = [o["op"] for o in lg["real_compat_ops"]]
    assert any("pre-twiddle" in o for o in ops) and any("normalization" in o for o in ops)


def test_real_four_step_schedules():
    n, b = 1 << 18, 64
    zrow = 8 * (n // 2) * b
    alg = 4 * n * b + 8 * (n // 2 + 1) * b
    # schedule 0: stitch fused into the passes, Z round trip only
    lg = ledger.launch_ledger(plan("fft_four_step_batch", n, b, transform_type="r2c"))
    assert lg["launches"] == 2 and lg["gm_bytes"] == alg + 2 * zrow
    # schedule 1 chunked: the stitch runs once per chunk
    lg = ledger.launch_ledger(plan("fft_four_step_batch", n, b, {"schedule": 1, "chunk_rows": 16},
                                   transform_type="c2r", transform_direction="inverse"))
    assert (lg["core_launches"], lg["epilogue_launches"]) == (8, 4)
    # schedule 3 (narrow groups): the stitch as its own launch too
    lg = ledger.launch_ledger(plan("fft_four_step_batch", n, b, {"schedule": 3}, transform_type="r2c"))
    assert (lg["core_launches"], lg["epilogue_launches"]) == (2, 1) and lg["schedule"] == 3
    # schedule 1 unchunked: one epilogue launch
    lg = ledger.launch_ledger(plan("fft_four_step_batch", n, b, {"schedule": 1}, transform_type="r2c"))
    assert (lg["core_launches"], lg["epilogue_launches"]) == (2, 1)


def test_inverse_and_scale_ops_are_fused():
    lg = ledger.launch_ledger(plan("fft_lds_fused_batch", transform_direction="inverse"))
    ops = {o["op"]: o for o in lg["real_compat_ops"]}
    assert any("inverse" in k for k in ops) and any("normalization" in k for k in ops)
    assert all(o["fused"] and o["in_bytes"] == o["out_bytes"] == 0 for o in ops.values())
    assert lg["gm_bytes"] == lg["algorithmic_bytes"]
    # forward under "backward" applies no scale; "ortho" scales both ways; "none" never
    names = lambda **k: [o["op"] for o in ledger.launch_ledger(plan("fft_lds_fused", **k))["real_compat_ops"]]  # noqa: E731
    assert names() == []
    assert any("normalization" in o for o in names(norm="ortho"))
    assert names(norm="none", transform_direction="inverse") == [
        "inverse direction (twiddle sign; no conjugate pass)"]


def test_composition_plans():
    lg = ledger.launch_ledger(plan("run_hybrid", 4096, 4, {"flow_kind": "composition", "tile": 64,
                                                            "core": "vendor"}))
    assert lg["available"] is False and "opaque" in lg["why"] and "plan_ledger" in lg["why"]
    assert lg["real_compat_ops"] == [] and "launches" not in lg
    # this library's own core: a four-step with n1 = n / tile
    lg = ledger.launch_ledger(plan("run_hybrid", 4096, 4, {"flow_kind": "composition", "tile": 64,
                                                            "core": "local"}))
    assert lg["available"] and lg["family"] == "four-step-two-pass" and (lg["n1"], lg["n2"]) == (64, 64)


def test_unknown_runner_is_an_honest_absence():
    lg = ledger.launch_ledger(plan("fft_unknown_fn"))
    assert lg["available"] is False and "no registered" in lg["why"] and "launches" not in lg


def _case(n, b, sem, sel, ven):
    return {"N": n, "batch": b, "semantic": sem, "selector_ms": sel, "vendor_ms": ven}


def test_batch_fill_analysis_growth():
    cases = [_case(1024, 1, "c2c-forward", 1.0, 0.1), _case(1024, 16, "c2c-forward", 40.0, 0.1),
             _case(1024, 64, "c2c-forward", 320.0, 0.1), _case(1024, 256, "c2c-forward", 2000.0, 0.1),
             _case(512, 64, "c2c-forward", 1.0, 0.1)]
    (row,) = ledger.batch_fill_analysis(cases, n_values=[1024])
    assert row["kind"].startswith("summary-derived") and [p["B"] for p in row["points"]] == [1, 16, 64, 256]
    # per point: 2000 ms over 1024*256 points against 1 ms over 1024 points
    assert row["selector_per_point_growth_smallest_to_largest_B"] == pytest.approx(2000.0 / 256)
    assert row["vendor_per_point_growth_smallest_to_largest_B"] == pytest.approx(1.0 / 256)
    assert row["poor_batch_fill"] is True
    assert "no worker/wave hardware counters" in row["conclusion_scope"]
    # a flat per-point cost is not poor fill
    flat = [_case(64, b, "r2c-forward", 0.01 * b, 0.01) for b in (1, 4, 16)]
    (row,) = ledger.batch_fill_analysis(flat)
    assert row["selector_per_point_growth_smallest_to_largest_B"] == pytest.approx(1.0)
    assert row["poor_batch_fill"] is False


def test_batch_fill_analysis_needs_three_points():
    assert ledger.batch_fill_analysis([_case(1024, 1, "c2c-forward", 1.0, 0.1),
                                       _case(1024, 16, "c2c-forward", 2.0, 0.1)]) == []
    assert ledger.batch_fill_analysis([{"N": 1, "batch": 1, "semantic": "c2c-forward", "selector_ms": None,
                                        "vendor_ms": 1.0}]) == []
