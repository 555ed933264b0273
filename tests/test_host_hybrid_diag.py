"""The composition diagnostics on the host: summarize_samples with the
reference's rules (tests/test_adapter_hybrid.py:115-138 checks the same
values), and plan_ledger's accounting for both cores.  No GPU needed."""
import json

import pytest

from kunlunxin_fft_amd.hybrid import plan_hybrid, plan_ledger, summarize_samples


def test_summarize_samples_even_count():
    s = summarize_samples([4.0, 1.0, 3.0, 2.0])
    assert s["n"] == 4 and s["p50"] == pytest.approx(2.5) and s["max"] == 4.0
    assert s["mad"] == pytest.approx(1.0)  # |dev| 1.5, 0.5, 0.5, 1.5 -> median 1.0
    assert s["outlier_threshold"] == pytest.approx(5.5) and s["outlier_count"] == 0
    assert s["p95"] == 4.0  # sorted[round(0.95 * 3)]


def test_summarize_samples_outliers():
    s = summarize_samples([1.0] * 9 + [100.0])
    assert s["outlier_count"] == 1 and s["outlier_values"] == [100.0] and s["max"] == 100.0
    s = summarize_samples([1.0, 2.0, 3.0, 4.0, 100.0])
    assert (s["p50"], s["mad"], s["outlier_values"], s["p95"]) == (3.0, 1.0, [100.0], 100.0)
    # MAD 0: the threshold falls back to 1.5 * p50
    s = summarize_samples([2.0] * 8 + [4.0])
    assert s["mad"] == 0.0 and s["outlier_threshold"] == 3.0 and s["outlier_values"] == [4.0]
    assert summarize_samples([]) == {"n": 0}


def test_plan_ledger_vendor_core():
    n, b, tile = 4096, 4, 64
    led = plan_ledger(plan_hybrid(n, b, tile))
    assert led["core"] == "vendor" and led["core_launches_est"] is None and led["core_api_calls"] == 2
    assert led["core_calls"] == {"stage1": b * tile, "stage1_len": n // tile, "stage2": b * (n // tile),
                                 "stage2_len": tile}
    # gather, twiddle-transpose and scatter, each reading and writing the batch once
    assert len(led["materialized_boundaries"]) == 3
    assert led["gm_bytes_framework_est"] == 3 * 2 * 8 * n * b
    # an inverse under "backward" adds the scale pass
    inv = plan_ledger(plan_hybrid(n, b, tile, transform_direction="inverse"))
    assert inv["gm_bytes_framework_est"] == 4 * 2 * 8 * n * b
    json.dumps(led)


def test_plan_ledger_local_core():
    led = plan_ledger(plan_hybrid(1 << 16, 2, 256, core="triton"))  # the reference's name for its own core
    assert led["core"] == "local" and led["core_launches_est"] == 2 and led["gm_bytes_framework_est"] == 0
    assert led["gm_bytes_core_est"] == 4 * 8 * (1 << 16) * 2
