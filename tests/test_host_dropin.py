"""The reference's public surface, name by name: every name its package
exports that this build keeps (src/xpu/__init__.py:12-163), the runner
signatures (src/xpu/runner.py:118-1635), the timing helpers' return
schema, the contract error metric, the size matrix and run manifest
(src/xpu/config.py:98-352) and the environment freshness gate
(src/xpu/selector.py:482-510).  No GPU needed: calls that would launch stop
at the GPU check with RuntimeError, after the keywords were accepted."""
import inspect
import math

import numpy as np
import pytest
import torch

import kunlunxin_fft_amd as pkg
from kunlunxin_fft_amd import runner
from kunlunxin_fft_amd.config import ConfigError, DeviceProfile

# (runner name, parameter names in the reference's order, their defaults)
REFERENCE_RUNNERS = [
    ("fft_dit", ["x", "block", "twiddle"], {"block": 1024, "twiddle": None}),
    ("fft_dif", ["x", "block", "twiddle"], {"block": 1024, "twiddle": None}),
    ("fft_dit_fused", ["x", "block", "tile", "twiddle"], {"block": 1024, "tile": 64, "twiddle": None}),
    ("fft_dit_matrix", ["x", "block", "tile", "rows", "twiddle"],
     {"block": 1024, "tile": 64, "rows": 8, "twiddle": None}),
    ("fft_dif_matrix", ["x", "block", "tile", "rows", "twiddle"],
     {"block": 1024, "tile": 64, "rows": 8, "twiddle": None}),
    ("fft_dit_grouped", ["x", "block", "tile", "rows", "glog", "maxp", "cells", "twiddle"],
     {"block": 1024, "tile": 64, "rows": 8, "glog": 2, "maxp": 4096, "cells": 1, "twiddle": None}),
    ("fft_dif_grouped", ["x", "block", "tile", "rows", "glog", "maxp", "cells", "twiddle"],
     {"block": 1024, "tile": 64, "rows": 8, "glog": 2, "maxp": 4096, "cells": 1, "twiddle": None}),
    ("fft_dit_batch", ["x", "block", "variant", "twiddle"], {"block": 1024, "variant": "spread", "twiddle": None}),
    ("fft_dif_batch", ["x", "block", "variant", "twiddle"], {"block": 1024, "variant": "spread", "twiddle": None}),
    ("fft_dit_matrix_batch", ["x", "block", "tile", "rows", "variant", "twiddle"],
     {"block": 1024, "tile": 64, "rows": 8, "variant": "spread", "twiddle": None}),
    ("fft_dif_matrix_batch", ["x", "block", "tile", "rows", "variant", "twiddle"],
     {"block": 1024, "tile": 64, "rows": 8, "variant": "spread", "twiddle": None}),
    ("fft_dit_matrix_packet_batch", ["x", "block", "tile", "rows", "packets", "twiddle"],
     {"block": 1024, "tile": 64, "rows": 8, "packets": 2, "twiddle": None}),
    ("fft_dit_radix4_batch", ["x", "block", "variant", "twiddle"],
     {"block": 1024, "variant": "spread", "twiddle": None}),
    ("fft_dif_radix4_batch", ["x", "block", "variant", "twiddle"],
     {"block": 1024, "variant": "spread", "twiddle": None}),
    ("fft_dit_radix4", ["x", "block", "twiddle"], {"block": 1024, "twiddle": None}),
    ("fft_dif_radix4", ["x", "block", "twiddle"], {"block": 1024, "twiddle": None}),
    ("bit_reverse_permute", ["x", "block"], {"block": 1024}),
    ("time_call", ["fn", "warmup", "iters"], {"warmup": 5, "iters": 20}),
    ("time_call_detailed", ["fn", "warmup", "trials", "seed"], {"warmup": 10, "trials": 50, "seed": 0}),
]

# every name the reference package exports that is not a Triton kernel object
REFERENCE_EXPORTS = [
    "ConfigError", "DesignSpace", "DeviceProfile", "ExecutionPlan", "ExecutionReport", "Manifest",
    "SizeMatrix", "Selection", "SUPPORTED_NORMS", "SUPPORTED_TRANSFORMS", "SUPPORTED_TRANSFORM_DIRECTIONS",
    "build_manifest", "composition_select", "execute_fft_plan", "git_commit", "git_dirty",
    "load_composition_table", "load_table", "norm_scale", "plan_fft", "select",
    "bit_reverse_permute", "device_name", "device_ready", "fft_dif", "fft_dit", "fft_dit_fused",
    "fft_dit_matrix", "fft_dif_matrix", "fft_dit_grouped", "fft_dif_grouped", "fft_dit_batch",
    "fft_dif_batch", "fft_dit_matrix_batch", "fft_dif_matrix_batch", "fft_dit_matrix_packet_batch",
    "fft_dit_radix4", "fft_dif_radix4", "fft_dit_radix4_batch", "fft_dif_radix4_batch", "log2_exact",
    "run_fft", "time_call", "time_call_detailed", "twiddle_tables", "xpu_context", "validate_input",
]


@pytest.mark.parametrize("name", REFERENCE_EXPORTS)
def test_reference_export_resolves(name):
    assert name in dir(pkg), name
    assert getattr(pkg, name) is not None


@pytest.mark.parametrize("name,params,defaults", REFERENCE_RUNNERS, ids=[r[0] for r in REFERENCE_RUNNERS])
def test_runner_signature_matches_the_reference(name, params, defaults):
    sig = inspect.signature(getattr(runner, name))
    got = [p for p in sig.parameters.values() if p.kind in (p.POSITIONAL_OR_KEYWORD, p.POSITIONAL_ONLY)]
    assert [p.name for p in got] == params
    for k, v in defaults.items():
        assert sig.parameters[k].default == v, (k, sig.parameters[k].default)


@pytest.mark.parametrize("name,params,defaults", [r for r in REFERENCE_RUNNERS if r[1][0] == "x"],
                         ids=[r[0] for r in REFERENCE_RUNNERS if r[1][0] == "x"])
def test_runner_accepts_the_reference_keywords(name, params, defaults):
    """A reference call with every keyword spelled out gets past argument
    binding and stops at the GPU check (this container has no GPU)."""
    batched = "batch" in name
    x = torch.zeros((2, 64) if batched else (64,), dtype=torch.complex64)
    kw = {k: v for k, v in defaults.items()}
    with pytest.raises(RuntimeError, match="GPU"):
        getattr(runner, name)(x, **kw)


def test_batch_runners_reject_an_unknown_variant():
    x = torch.zeros((2, 64), dtype=torch.complex64)
    for name in ("fft_dit_batch", "fft_dif_radix4_batch", "fft_dit_matrix_batch"):
        with pytest.raises(ValueError, match="variant"):
            getattr(runner, name)(x, variant="tiled")


def test_radix4_and_matrix_batches_take_spread_only():
    """reference test_fft.py:405-419, 456-465: 'folded' is refused, naming 'spread'."""
    x = torch.zeros((4, 64), dtype=torch.complex64)
    for name in ("fft_dit_radix4_batch", "fft_dif_radix4_batch", "fft_dit_matrix_batch", "fft_dif_matrix_batch"):
        with pytest.raises(ValueError, match="spread"):
            getattr(runner, name)(x, variant="folded")
    # the M4 batch runners lower both variants
    for name in ("fft_dit_batch", "fft_dif_batch"):
        with pytest.raises(RuntimeError, match="GPU"):
            getattr(runner, name)(x, variant="folded")


def test_packet_batch_checks_packets():
    """reference test_fft.py:483-497: packets a power of two, at most 2, dividing B."""
    x = torch.zeros((16, 1024), dtype=torch.complex64)
    with pytest.raises(ValueError, match="ceiling"):
        runner.fft_dit_matrix_packet_batch(x, packets=4)
    with pytest.raises(ValueError, match="power of two"):
        runner.fft_dit_matrix_packet_batch(x, packets=3)
    with pytest.raises(ValueError, match="divide"):
        runner.fft_dit_matrix_packet_batch(torch.zeros((1, 1024), dtype=torch.complex64), packets=2)


def test_fused_schedule_needs_the_opt_in():
    x = torch.zeros((2, 1 << 16), dtype=torch.complex64)
    with pytest.raises(ValueError, match="allow_fused_schedule"):
        runner.fft_four_step_batch(x, n1=256, schedule=2)
    with pytest.raises(RuntimeError, match="GPU"):  # accepted, then the GPU check
        runner.fft_four_step_batch(x, n1=256, schedule=2, allow_fused_schedule=True)


def test_fused_schedule_is_not_a_table_candidate():
    from kunlunxin_fft_amd.config import DesignSpace
    from kunlunxin_fft_amd.selector import entry_contract_violations

    assert 2 not in DesignSpace.load().fourstep_schedule
    entry = {"N": 1 << 16, "batch": 512, "direction": "dit", "block": 256, "flow_id": "four-step-two-pass",
             "flow_realization": "four-step", "processing_unit": "stockham-radix16",
             "executed": "fft_four_step_batch", "params": {"n1": 256, "chunk_rows": 0, "schedule": 2}}
    assert any("schedule" in v for v in entry_contract_violations(entry))


def test_validate_input_require_complex():
    x = torch.zeros(64, dtype=torch.float32)
    with pytest.raises(TypeError, match="complex64"):
        pkg.validate_input(x)
    # without the dtype requirement the next check is the GPU
    with pytest.raises(RuntimeError, match="GPU"):
        pkg.validate_input(x, require_complex=False)


def test_time_call_protocol_without_gpu():
    calls = []
    ms = runner.time_call(lambda: calls.append(1), warmup=2, iters=5)
    assert isinstance(ms, float) and ms >= 0 and len(calls) == 7
    calls.clear()
    d = runner.time_call_detailed(lambda: calls.append(1), warmup=3, trials=11, seed=7)
    assert len(calls) == 14
    assert set(d) == {"api_ms", "kernel_ms", "metric_note"}
    assert set(d["api_ms"]) == {"median", "min", "p10", "p90", "trials"} and d["api_ms"]["trials"] == 11
    assert d["api_ms"]["min"] <= d["api_ms"]["p10"] <= d["api_ms"]["median"] <= d["api_ms"]["p90"]
    assert d["kernel_ms"] is None  # no device events without a GPU


def test_time_call_detailed_shuffles_trials_by_seed():
    import random

    order = list(range(50))
    random.Random(0).shuffle(order)
    assert order != list(range(50))  # the reference's seed-0 order is a real permutation


def test_max_rel_error_contract():
    from kunlunxin_fft_amd.error_metric import max_rel_error, rel_l2

    ref = np.array([3 + 4j, 0 + 0j, -1 + 0j])
    got = ref + np.array([0.001 - 0.002j, 0, 0])
    # max(|dRe|, |dIm|) = 0.002 over max|ref| = 5
    assert math.isclose(max_rel_error(got, ref), 0.002 / 5)
    assert max_rel_error(ref, ref) == 0.0
    # a NaN in the imaginary part only (builtin max would keep the finite real part)
    bad = ref.copy()
    bad[1] = complex(0.0, float("nan"))
    assert max_rel_error(bad, ref) == float("inf")
    assert max_rel_error(ref, np.array([np.inf, 1, 1])) == float("inf")
    # all-zero reference: the scale floors at 1e-12
    assert math.isclose(max_rel_error(np.array([1e-13]), np.array([0.0])), 0.1)
    assert math.isclose(rel_l2(got, ref), math.sqrt(0.001 ** 2 + 0.002 ** 2) / math.sqrt(26))
    assert rel_l2(bad, ref) == float("inf") and rel_l2(ref, ref) == 0.0


def test_size_matrix_loads_powers_of_two():
    sm = pkg.SizeMatrix.load()
    for seq in (sm.correctness_sizes, sm.bench_sizes, sm.blocksizes):
        assert seq and all(v > 0 and v & (v - 1) == 0 for v in seq)
    assert max(sm.bench_sizes) == DeviceProfile.load().max_n
    assert isinstance(sm.vendor_baseline_max_n, int)


def test_manifest_is_pinned_to_the_profile():
    prof = DeviceProfile.load()
    m = pkg.build_manifest(prof, block=512, command="pytest")
    d = m.to_dict()
    assert d["profile_hash"] == prof.hash() and d["gfx_arch"] == "gfx950" and d["block"] == 512
    assert isinstance(d["commit"], str) and d["commit"] and isinstance(d["dirty"], bool)
    with pytest.raises(ConfigError, match="unknown manifest field"):
        pkg.build_manifest(prof, no_such_field=1)
    assert isinstance(pkg.git_commit(), str) and isinstance(pkg.git_dirty(), bool)


def test_assert_current_environment_fails_closed():
    with pytest.raises(RuntimeError, match="env_hash"):
        pkg.assert_current_environment({"entries": []})
    # no GPU here: the live fingerprint is unknown, so any bound table fails
    with pytest.raises(RuntimeError, match="unknown"):
        pkg.assert_current_environment({"env_hash": "0123456789abcdef"})


def test_device_guards_need_a_gpu():
    with pytest.raises(RuntimeError, match="GPU"):
        with pkg.xpu_context(0):
            pass
    from kunlunxin_fft_amd.context import device_context

    with pytest.raises(RuntimeError, match="GPU"):
        with device_context(torch.device("cuda:0")):
            pass


# ---- the real-flow epilogues' host references (runner.py:1776-1834)

@pytest.mark.parametrize("n", [4, 8, 64, 1024])
@pytest.mark.parametrize("b", [1, 3])
def test_real_epilogue_refs_against_numpy(n, b):
    """r2c_stitch_ref of the packed pairs' FFT is numpy's rfft; c2r_pre_ref,
    a forward FFT and c2r_unpack_ref with scale 2/N are numpy's irfft, the
    DC and Nyquist imaginary parts ignored."""
    rng = np.random.default_rng(3 * n + b)
    x = rng.standard_normal((b, n))
    z = np.fft.fft(x[:, 0::2] + 1j * x[:, 1::2], axis=-1).astype(np.complex64)
    X = runner.r2c_stitch_ref(torch.from_numpy(z), n).numpy()
    ref = np.fft.rfft(x, axis=-1)
    assert np.abs(X - ref).max() <= 1e-6 * np.abs(ref).max()
    assert np.all(X[:, 0].imag == 0) and np.all(X[:, n // 2].imag == 0)
    h = (rng.standard_normal((b, n // 2 + 1)) + 1j * rng.standard_normal((b, n // 2 + 1))).astype(np.complex64)
    Z = runner.c2r_pre_ref(torch.from_numpy(h), n).numpy()
    u = np.fft.fft(Z.astype(np.complex128), axis=-1).astype(np.complex64)
    y = runner.c2r_unpack_ref(torch.from_numpy(u), n, 2.0 / n).numpy()
    h64 = h.astype(np.complex128)
    h64[:, 0] = h64[:, 0].real
    h64[:, n // 2] = h64[:, n // 2].real
    want = np.fft.irfft(h64, n=n, axis=-1)
    assert y.shape == (b, n) and y.dtype == np.float32
    assert np.abs(y - want).max() <= 1e-6 * np.abs(want).max()


def test_real_epilogue_ref_contracts():
    """reference test_semantic_real_flow_host.py:321-330."""
    with pytest.raises(ValueError, match="N/2"):
        runner.r2c_stitch_ref(torch.zeros(32, dtype=torch.complex64), 128)
    with pytest.raises(ValueError, match="N/2\\+1"):
        runner.c2r_pre_ref(torch.zeros(64, dtype=torch.complex64), 128)
    with pytest.raises(ValueError, match="N/2"):
        runner.c2r_unpack_ref(torch.zeros(63, dtype=torch.complex64), 128)


def test_real_epilogues_check_before_the_gpu():
    """The runners' contract (reference runner.py:1661-1684) raises before
    anything needs a GPU: a CPU tensor is a ValueError, a wrong dtype a
    TypeError."""
    z = torch.zeros(32, dtype=torch.complex64)
    with pytest.raises(ValueError, match="GPU"):
        runner.r2c_stitch(z, 64)
    with pytest.raises(TypeError, match="complex64"):
        runner.c2r_pre(torch.zeros(33), 64)
    with pytest.raises(TypeError, match="torch.Tensor"):
        runner.c2r_unpack([0j] * 32, 64)


# (module, name, leading parameters in the reference's order, their defaults):
# the module-level helpers beside the runners (ledger.py, adapter_hybrid.py,
# semantic.py, composition.py, context.py); trailing parameters this build
# adds after them are allowed
REFERENCE_HELPERS = [
    ("ledger", "phase", ["name"], {}),
    ("ledger", "current_ledger", [], {}),
    ("ledger", "launch_ledger", ["plan"], {}),
    ("ledger", "measure_phases", ["plan", "x", "trials", "warmup"], {"trials": 30, "warmup": 5}),
    ("ledger", "batch_fill_analysis", ["cases", "n_values"], {"n_values": None}),
    ("ledger", "PhaseLedger", ["sync"], {"sync": True}),
    ("hybrid", "plan_hybrid", ["n", "batch", "tile", "core"], {"tile": 64, "core": "vendor"}),
    ("hybrid", "run_hybrid", ["x", "plan"], {}),
    ("hybrid", "plan_ledger", ["plan"], {}),
    ("hybrid", "summarize_samples", ["samples"], {}),
    ("hybrid", "time_cell", ["fn", "x", "warmup", "trials"], {}),
    ("hybrid", "profile_hybrid", ["x", "plan"], {}),
    ("semantic", "spec", ["label"], {}),
    ("semantic", "family", ["transform_type"], {}),
    ("semantic", "family_allows", ["transform_type", "flow_id"], {}),
    ("semantic", "family_size", ["transform_type"], {}),
    ("semantic", "validate_taxonomy", [], {}),
    ("composition", "composition_entry_violations", ["entry", "table"], {}),
    ("composition", "table_violations", ["table"], {}),
    ("context", "current_device_index", [], {}),
    ("context", "xpu_context", ["device"], {"device": 0}),
]


@pytest.mark.parametrize("mod,name,params,defaults", REFERENCE_HELPERS,
                         ids=[f"{m}.{n}" for m, n, _, _ in REFERENCE_HELPERS])
def test_helper_signature_matches_the_reference(mod, name, params, defaults):
    import importlib

    obj = getattr(importlib.import_module(f"kunlunxin_fft_amd.{mod}"), name)
    sig = inspect.signature(obj)
    got = [p.name for p in sig.parameters.values() if p.kind in (p.POSITIONAL_OR_KEYWORD, p.POSITIONAL_ONLY)]
    assert got[:len(params)] == params, got
    for k, v in defaults.items():
        assert sig.parameters[k].default == v, (k, sig.parameters[k].default)
