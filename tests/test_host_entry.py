"""Host-only plan API contract (no GPU): restates the reference's
tests/test_entry.py, test_selector.py and test_semantic_key.py contracts
against this package's plan_fft / select / load_table."""
import json

import pytest

from kunlunxin_fft_amd import DeviceProfile, ExecutionPlan, load_table, norm_scale, plan_fft
from kunlunxin_fft_amd.config import ConfigError
from kunlunxin_fft_amd.entry import (
    REAL_FLOW_MARK, _check_plan_input, _dispatch, _m0_plan,
)
from kunlunxin_fft_amd.selector import GUARD_PCT, Selection, find_entry, select

PROF = DeviceProfile.load().hash()
ENV = "e" * 16


def _entry(n=2048, batch=1, direction="dit", real="lds-resident", unit="stockham-radix16",
           executed=None, params=None, block=256, **extra):
    e = {"N": n, "batch": batch, "direction": direction, "block": block,
         "flow_id": "lds-stockham-single-pass", "flow_realization": real,
         "processing_unit": unit, "params": params or {}, "incumbent_ms": 1.0,
         "challenger_ms": 0.5, "reason": "measured"}
    if executed:
        e["executed"] = executed
    e.update(extra)
    return e


def _table(entries=(), fallbacks=()):
    return {"profile_hash": PROF, "env_hash": ENV, "precision": "fp32", "guard_pct": GUARD_PCT,
            "env": {"device_model": "gfx950", "multiprocessor_count": 256, "max_shared_mem": 163840},
            "entries": list(entries), "previous_fallbacks": list(fallbacks)}


def _write(tmp_path, table):
    p = tmp_path / "t.json"
    p.write_text(json.dumps(table))
    return str(p)


@pytest.mark.parametrize("real,unit,direction,batch,expect", [
    ("global-stage", "radix2-scalar", "dit", 1, "fft_dit"),
    ("global-stage", "radix2-scalar", "dif", 1, "fft_dif"),
    ("global-stage", "radix2-scalar", "dit", 4, "fft_dit_batch"),
    ("global-stage", "radix4-scalar", "dit", 1, "fft_dit_radix4"),
    ("global-stage", "radix4-scalar", "dif", 16, "fft_dif_radix4_batch"),
    ("lds-resident", "stockham-radix16", "dit", 1, "fft_lds_fused"),
    ("lds-resident", "stockham-radix16", "dif", 64, "fft_lds_fused_batch"),
    ("four-step", "stockham-radix16", "dit", 1, "fft_four_step"),
    ("four-step", "stockham-radix16", "dit", 256, "fft_four_step_batch"),
    ("fused-inplace", "radix2-scalar", "dit", 1, "fft_dit_fused"),
    ("matrix-resident", "dense-dot-fft64", "dif", 1, "fft_dif_matrix"),
    ("matrix-resident", "dense-dot-fft64", "dit", 4, "fft_dit_matrix_batch"),
    ("grouped-boundary", "composite-linear-map", "dit", 1, "fft_dit_grouped"),
])
def test_dispatch_covers_known_lowerings(real, unit, direction, batch, expect):
    sel = Selection(n=2048, direction=direction, batch=batch, precision="fp32", source="table",
                    reason="t", block=256, flow_id="x", flow_realization=real, processing_unit=unit)
    assert _dispatch(sel) == expect


@pytest.mark.parametrize("real,unit,direction,batch", [
    ("fused-inplace", "radix2-scalar", "dif", 1),
    ("fused-inplace", "radix2-scalar", "dit", 4),
    ("grouped-boundary", "composite-linear-map", "dit", 16),
])
def test_dispatch_returns_none_for_unlowered(real, unit, direction, batch):
    sel = Selection(n=16, direction=direction, batch=batch, precision="fp32", source="table",
                    reason="t", block=256, flow_id="x", flow_realization=real, processing_unit=unit)
    assert _dispatch(sel) is None


def test_plan_rejects_invalid_direction():
    for bad in ("inverse", "r2c"):
        with pytest.raises(ValueError, match="unsupported direction"):
            plan_fft(bad, 16, profile_hash=PROF, table=_table())


def test_plan_rejects_invalid_precision():
    with pytest.raises(ValueError, match="unsupported precision"):
        plan_fft("dit", 16, precision="fp64", profile_hash=PROF, table=_table())


@pytest.mark.parametrize("kwargs", [dict(transform_type="stft"), dict(transform_type="dct"),
                                    dict(transform_direction="sideways"), dict(norm="l2")])
def test_plan_rejects_unsupported_semantics(kwargs):
    with pytest.raises(ValueError):
        plan_fft("dit", 16, profile_hash=PROF, table=_table(), **kwargs)


@pytest.mark.parametrize("kwargs", [dict(transform_type="r2c", transform_direction="inverse"),
                                    dict(transform_type="c2r", transform_direction="forward")])
def test_real_transforms_are_direction_locked(kwargs):
    with pytest.raises(ValueError, match="forward transform|inverse transform"):
        plan_fft("dit", 16, profile_hash=PROF, table=_table(), **kwargs)


def test_plan_rejects_before_table_query():
    class Boom:
        def __getitem__(self, key):
            raise AssertionError("table queried before validation")

        def get(self, *a):
            raise AssertionError("table queried before validation")

    for bad in (dict(transform_type="stft"), dict(norm="madeup"), dict(transform_direction="x")):
        with pytest.raises(ValueError):
            plan_fft("dit", 16, table=Boom(), **bad)


@pytest.mark.parametrize("n", [0, 3, 12, 1 << 21])
def test_plan_rejects_bad_lengths(n):
    with pytest.raises(ValueError):
        plan_fft("dit", n, profile_hash=PROF, table=_table())


def test_plan_executes_table_winner():
    t = _table([_entry(2048, 1, "dit", executed="fft_lds_fused", params={"elems": 16})])
    plan = plan_fft("dit", 2048, profile_hash=PROF, table=t, env_hash=ENV)
    assert not plan.fallback and plan.selection_source == "table"
    assert plan.executed == "fft_lds_fused" and plan.params["elems"] == 16


def test_plan_falls_back_on_unknown_n():
    plan = plan_fft("dit", 4096, profile_hash=PROF, table=_table([_entry(2048)]), env_hash=ENV)
    assert plan.fallback and plan.executed == "fft_dit" and plan.selection_source == "abstain"
    assert "no measured entry" in plan.reason


def test_plan_rounds_a_batch_without_exact_key():
    """A batch with no exact key (not a power of two, or past the table's
    grid) takes the measured decision of the smallest table batch at or
    above it, or past the largest batch of this N, the largest: entry tier
    batch-rounded, source table, the rounding in the reason.  Batch 1
    entries never answer a batch above 1; unknown N, a profile or
    environment mismatch still abstain."""
    t = _table([_entry(2048, 1, "dit", executed="fft_lds_fused", params={"elems": 8}),
                _entry(2048, 64, "dit", executed="fft_lds_fused_batch", params={"elems": 16}),
                _entry(2048, 128, "dit", executed="fft_four_step_batch", real="four-step",
                       params={"n1": 64})])
    for batch, want, rounded in ((100, "fft_four_step_batch", 128), (65, "fft_four_step_batch", 128),
                                 (3, "fft_lds_fused_batch", 64), (63, "fft_lds_fused_batch", 64),
                                 (1000, "fft_four_step_batch", 128), (256, "fft_four_step_batch", 128)):
        sel = select("dit", 2048, batch=batch, profile_hash=PROF, table=t, env_hash=ENV)
        assert sel.source == "table" and sel.entry_tier == "batch-rounded", (batch, sel.reason)
        assert sel.executed == want and f"batch={rounded}" in sel.reason, (batch, sel.reason)
        plan = plan_fft("dit", 2048, batch=batch, profile_hash=PROF, table=t, env_hash=ENV)
        assert not plan.fallback and plan.executed == want and plan.batch == batch
        assert plan.params["table_batch"] == rounded == sel.table_batch
    # exact keys answer as before, with no rounding marker
    assert select("dit", 2048, batch=64, profile_hash=PROF, table=t, env_hash=ENV).entry_tier == "legacy"
    assert "table_batch" not in plan_fft("dit", 2048, batch=64, profile_hash=PROF, table=t, env_hash=ENV).params
    # no entry of this N, or a binding mismatch: abstain
    assert plan_fft("dit", 4096, batch=100, profile_hash=PROF, table=t, env_hash=ENV).fallback
    assert plan_fft("dit", 2048, batch=100, profile_hash="f" * 16, table=t, env_hash=ENV).fallback
    assert plan_fft("dit", 2048, batch=100, profile_hash=PROF, table=t, env_hash="0" * 16).fallback
    # the other decomposition has no entries here
    assert plan_fft("dif", 2048, batch=100, profile_hash=PROF, table=t, env_hash=ENV).fallback
    # only a batch-1 entry: a batch above 1 abstains
    only1 = _table([_entry(2048, 1, "dit", executed="fft_lds_fused")])
    assert plan_fft("dit", 2048, batch=5, profile_hash=PROF, table=only1, env_hash=ENV).fallback


def test_rounding_on_the_shipped_table_matches_the_next_power_of_two():
    """On the shipped table (indexed), an odd batch takes the next power of
    two's entry for every semantic, and a batch past 2^32 elements the
    largest batch's."""
    from kunlunxin_fft_amd.selector import default_table, find_entry, rounded_batch

    t = default_table()
    for n in (16, 1024, 1 << 15, 1 << 20):
        for batch in (3, 100, 1000):
            for sem in (("c2c", "forward", "backward"), ("r2c", "forward", "backward"),
                        ("c2r", "inverse", "backward")):
                up = 1 << (batch - 1).bit_length()
                if n * up > (1 << 32):
                    continue
                assert rounded_batch(t, n, batch, "dit", *sem) == up
                sel = select("dit", n, batch=batch, profile_hash=t["profile_hash"], table=t,
                             env_hash=t["env_hash"], transform_type=sem[0], transform_direction=sem[1])
                e = find_entry(t, n, up, "dit", *sem)
                assert sel.entry_tier == "batch-rounded" and sel.executed == e["executed"]
                assert {k: v for k, v in sel.params.items()} == (e.get("params") or {})
    biggest = (1 << 32) // (1 << 20)
    assert rounded_batch(t, 1 << 20, 3 * biggest, "dit") == biggest


def test_plan_falls_back_on_missing_profile():
    plan = plan_fft("dit", 2048, profile_hash=None, table=_table([_entry()]), env_hash=ENV)
    assert plan.fallback and plan.executed == "fft_dit"
    assert "profile_hash is required" in plan.reason


def test_plan_falls_back_on_profile_mismatch():
    plan = plan_fft("dit", 2048, profile_hash="f" * 16, table=_table([_entry()]), env_hash=ENV)
    assert plan.fallback and "profile hash" in plan.reason


def test_plan_falls_back_on_env_mismatch_or_unknown():
    t = _table([_entry()])
    assert "environment hash" in plan_fft("dit", 2048, profile_hash=PROF, table=t, env_hash="0" * 16).reason
    assert "unknown" in plan_fft("dit", 2048, profile_hash=PROF, table=t, env_hash=None).reason
    unbound = dict(t, env_hash="")
    assert "env_hash" in plan_fft("dit", 2048, profile_hash=PROF, table=unbound, env_hash=ENV).reason


def test_plan_falls_back_for_dif_fused_entry():
    t = _table([_entry(16, 1, "dif", real="fused-inplace", unit="radix2-scalar", params={})])
    plan = plan_fft("dif", 16, profile_hash=PROF, table=t, env_hash=ENV)
    assert plan.fallback and plan.executed == "fft_dif" and "no lowering" in plan.reason


def test_plan_falls_back_for_batched_m1_entry():
    t = _table([_entry(16, 4, "dit", real="fused-inplace", unit="radix2-scalar")])
    plan = plan_fft("dit", 16, batch=4, profile_hash=PROF, table=t, env_hash=ENV)
    assert plan.fallback and plan.executed == "fft_dit_batch" and "no lowering" in plan.reason
    assert plan.params["variant"] == "folded"


def test_semantic_tier_outranks_legacy_and_fallback_outranks_both():
    legacy = _entry(1024, 1, "dit", executed="fft_lds_fused")
    sem = _entry(1024, 1, "dit", executed="fft_four_step", real="four-step",
                 transform_type="c2c", transform_direction="inverse", normalization="backward")
    t = _table([legacy, sem])
    inv = plan_fft("dit", 1024, profile_hash=PROF, table=t, env_hash=ENV, transform_direction="inverse")
    fwd = plan_fft("dit", 1024, profile_hash=PROF, table=t, env_hash=ENV)
    assert inv.executed == "fft_four_step" and fwd.executed == "fft_lds_fused"
    fb = _entry(1024, 1, "dit", real="global-stage", unit="radix2-scalar", executed="fft_dit",
                transform_type="c2c", transform_direction="inverse", normalization="backward",
                previous_fallback_provenance={})
    t2 = _table([legacy, sem], [fb])
    e = find_entry(t2, 1024, 1, "dit", "c2c", "inverse", "backward")
    assert e is fb
    plan = plan_fft("dit", 1024, profile_hash=PROF, table=t2, env_hash=ENV, transform_direction="inverse")
    assert plan.executed == "fft_dit" and plan.params.get("previous_fallback") is True


def test_real_plans_are_dedicated_and_marked():
    t = _table([_entry(1024, 1, "dit", executed="fft_lds_fused")])
    r2c = plan_fft("dit", 1024, profile_hash=PROF, table=t, env_hash=ENV, transform_type="r2c")
    c2r = plan_fft("dif", 1024, profile_hash=None, table=t, transform_type="c2r", norm="ortho")
    assert r2c.transform_direction == "forward" and c2r.transform_direction == "inverse"
    assert r2c.params["real_compat"] == REAL_FLOW_MARK == c2r.params["real_compat"]
    assert r2c.executed == "fft_lds_fused" and c2r.fallback


def test_inverse_reuses_forward_lowering_on_legacy_entry():
    t = _table([_entry(1024, 16, "dif", executed="fft_lds_fused_batch")])
    inv = plan_fft("dif", 1024, batch=16, profile_hash=PROF, table=t, env_hash=ENV,
                   transform_direction="inverse", norm="ortho")
    fwd = plan_fft("dif", 1024, batch=16, profile_hash=PROF, table=t, env_hash=ENV)
    assert inv.executed == fwd.executed and inv.params == fwd.params and inv.norm == "ortho"


def test_norm_scale_matches_torch_fft_semantics():
    n = 16
    assert norm_scale(n, "forward", "none") == 1.0
    assert norm_scale(n, "forward", "forward") == 1.0 / n
    assert norm_scale(n, "forward", "backward") == 1.0
    assert norm_scale(n, "inverse", "none") == 1.0
    assert norm_scale(n, "inverse", "forward") == 1.0
    assert norm_scale(n, "inverse", "backward") == 1.0 / n
    for d in ("forward", "inverse"):
        assert norm_scale(n, d, "ortho") == 1.0 / n ** 0.5
    with pytest.raises(ValueError):
        norm_scale(n, "sideways", "none")


def _plan(n=16, batch=1, tt="c2c"):
    return ExecutionPlan(n=n, batch=batch, direction="dit", precision="fp32",
                         selection_source="table", reason="t", fallback=False, executed="fft_dit",
                         block=256, transform_type=tt)


def test_plan_input_contracts():
    _check_plan_input(_plan(16, 1), (16,), "complex64")
    _check_plan_input(_plan(4096, 16), (16, 4096), "complex64")
    with pytest.raises(ValueError, match="N=16"):
        _check_plan_input(_plan(16, 1), (32,), "complex64")
    with pytest.raises(ValueError, match="rank-1"):
        _check_plan_input(_plan(16, 1), (1, 16), "complex64")
    with pytest.raises(ValueError, match=r"\(4, 4096\)"):
        _check_plan_input(_plan(4096, 4), (16, 4096), "complex64")
    with pytest.raises(TypeError, match="complex64"):
        _check_plan_input(_plan(16, 1), (16,), "float32")
    _check_plan_input(_plan(64, 1, "r2c"), (64,), "float32")
    with pytest.raises(TypeError):
        _check_plan_input(_plan(64, 1, "r2c"), (64,), "complex64")
    _check_plan_input(_plan(64, 1, "c2r"), (33,), "complex64")
    with pytest.raises(ValueError):
        _check_plan_input(_plan(64, 1, "c2r"), (64,), "complex64")


def test_m0_plan_is_reference_shaped():
    p = _m0_plan(64, 4, "dif", "fp32", "why", True)
    assert p.executed == "fft_dif_batch" and p.fallback and p.selection_source == "abstain"
    assert p.flow_realization == "global-stage" and p.processing_unit == "radix2-scalar"


def test_load_table_refuses_contract_violations(tmp_path):
    bad = [
        _entry(2048, 1, "dit", real="lds-resident", params={"elems": 64}),
        _entry(2048, 1, "dit", real="nope", unit="nope"),
        _entry(2048, 1, "dit", executed="fft_dit"),          # runner outside its family
        _entry(2048, 4, "dit", executed="fft_lds_fused"),    # single runner at batch 4
        _entry(2048, 1, "dit", real="four-step", params={"n1": 3}),
        _entry(2048, 1, "dit", real="global-stage", unit="radix2-scalar", block=32),
        _entry(3000, 1, "dit"),
    ]
    for e in bad:
        with pytest.raises(ConfigError):
            load_table(_write(tmp_path, _table([e])))
    ok = load_table(_write(tmp_path, _table([_entry(executed="fft_lds_fused", params={"elems": 8})])))
    assert len(ok["entries"]) == 1


def test_load_table_refuses_unbound_fallbacks(tmp_path):
    fb = _entry(1024, 1, "dit", executed="fft_lds_fused", transform_type="c2c",
                transform_direction="forward", normalization="backward")
    with pytest.raises(ConfigError, match="provenance"):
        load_table(_write(tmp_path, _table([], [fb])))


def test_shipped_table_loads_and_binds_this_profile():
    t = load_table()
    assert t["profile_hash"] == PROF
    assert t["precision"] == "fp32"


def test_indexed_lookup_equals_the_scan():
    """find_entry on the package's shared table (indexed once per file
    version) answers exactly as the scan over an unindexed copy, for every
    cell and semantic, previous-fallback cells included."""
    import copy

    from kunlunxin_fft_amd.selector import default_table, find_entry

    shared = default_table()
    plain = copy.deepcopy(shared)
    sems = [("c2c", "forward", "backward"), ("c2c", "inverse", "ortho"), ("r2c", "forward", "backward"),
            ("c2r", "inverse", "backward"), ("r2c", "forward", "ortho")]
    cells = {(e["N"], e["batch"], e["direction"]) for e in shared["entries"] + shared.get("previous_fallbacks", [])}
    cells |= {(3000, 1, "dit"), (1024, 3, "dit")}
    for n, b, d in sorted(cells):
        for sem in sems:
            got, want = find_entry(shared, n, b, d, *sem), find_entry(plain, n, b, d, *sem)
            assert (got is None) == (want is None) and (got is None or got == want), (n, b, d, sem)


M0_NAMES = {"fft_dit", "fft_dit_batch", "fft_dif", "fft_dif_batch"}


def test_shipped_table_covers_the_grid():
    """Every power-of-two batch of every power-of-two N = 16 .. 2^20 up to
    2^32 elements has a C2C entry for both decompositions and an exact R2C
    and C2R entry, each a promoted challenger (no cell of the grid keeps M0,
    so no power-of-two batch of these N runs the radix-2 baseline)."""
    t = load_table()
    have = {}
    for e in t["entries"]:
        key = (e["N"], e["batch"], e["direction"], e.get("transform_type", "c2c"))
        assert key not in have, key
        have[key] = e["executed"]
    for k in range(4, 21):
        for j in range(0, 33 - k):
            n, b = 1 << k, 1 << j
            for key in ((n, b, "dit", "c2c"), (n, b, "dif", "c2c"), (n, b, "dit", "r2c"), (n, b, "dit", "c2r")):
                assert key in have, key
                assert have[key] not in M0_NAMES, (key, have[key])


def test_select_abstains_without_profile():
    s = select("dit", 2048, table=_table([_entry()]), env_hash=ENV)
    assert not s.selected and "profile_hash is required" in s.reason


def test_composition_fails_closed():
    from kunlunxin_fft_amd.composition import composition_select, load_composition_table

    from kunlunxin_fft_amd.selector import GUARD_PCT

    # the shipped table was measured on MI355X: no composition beat its
    # incumbent by the guard, so it holds no entry, only the measurements
    t = load_composition_table()
    assert t is not None and t["profile_hash"] == PROF and t["entries"] == []
    assert len(t["measurements"]) == 10
    for row in t["measurements"]:
        best = min(row["candidates"].values())
        assert (row["incumbent_ms"] - best) / row["incumbent_ms"] * 100.0 < GUARD_PCT, row
        assert composition_select("dit", row["N"], batch=row["batch"], profile_hash=PROF,
                                  env_hash=t["env_hash"]) is None
    assert composition_select("dit", 2048, batch=16, profile_hash=PROF, env_hash=ENV) is None


def test_entry_module_does_not_import_torch():
    import kunlunxin_fft_amd.entry as entry_mod

    src = open(entry_mod.__file__).read()
    lines = [ln for ln in src.splitlines() if "import torch" in ln and not ln.strip().startswith("#")]
    assert all(ln.startswith("    ") for ln in lines), lines


def test_device_profile_hash_is_stable():
    p = DeviceProfile.load()
    assert p.hash() == DeviceProfile.load().hash() and len(p.hash()) == 16
    assert p.gfx_arch == "gfx950" and p.compute_units == 256


def test_env_fingerprint_unknown_without_gpu():
    import torch

    from kunlunxin_fft_amd import envcheck

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert envcheck.current_env_hash() is None


def test_external_core_registry_and_composition_contract():
    """The external-core registry loads and validates; a composition entry
    must name its tile and core; composition_select honours the exact shape,
    semantics, profile and environment binding; the plan it yields routes to
    run_hybrid with the entry's tile and core."""
    import copy

    from kunlunxin_fft_amd import composition
    from kunlunxin_fft_amd.config import ConfigError
    from kunlunxin_fft_amd.entry import _composition_plan

    reg = composition.load_external_cores()
    cores = composition.composition_cores(reg)
    assert set(cores) == {"vendor", "local"}
    assert cores["vendor"]["classification"] == "materialized-external-subtransform"
    bad = copy.deepcopy(reg)
    bad["cores"][0]["classification"] = "magic"
    import json
    import tempfile
    with tempfile.NamedTemporaryFile("w", suffix=".json", delete=False) as f:
        json.dump(bad, f)
    with pytest.raises(ConfigError, match="classification"):
        composition.load_external_cores(f.name)
    entry = {"N": 2048, "batch": 16, "direction": "dit", "tile": 64, "core": "vendor", "flow_id": "c",
             "flow_realization": "four-step-composition", "processing_unit": "rocfft_torch_fft",
             "candidate_ms": 0.01, "incumbent_ms": 0.02, "guard_pct": 50.0, "reason": "test",
             "evidence": {"incumbent": "fft_lds_fused_batch", "candidates": {"vendor@64": 0.01},
                          "err_rel_l2": 3e-7}}
    table = {"kind": composition.KIND, "profile_hash": PROF, "env_hash": ENV, "precision": "fp32",
             "guard_pct": 2.0, "entries": [entry]}
    assert composition.table_violations(table) == []
    # one entry's contract, rule by rule (the reference's composition_entry_violations)
    viol = lambda **kw: composition.composition_entry_violations(dict(entry, **kw), table)  # noqa: E731
    assert viol() == []
    assert any("DIT only" in v for v in viol(direction="dif"))
    assert any("positive int" in v for v in viol(N=2048.0)) and any("positive int" in v for v in viol(batch=0))
    assert any("unknown core" in v for v in viol(core="cufft"))
    assert any("tile" in v for v in viol(tile=48)) and any("tile" in v for v in viol(tile=8))
    assert any("recomputed" in v for v in viol(guard_pct=49.0))
    assert any("err_rel_l2" in v for v in viol(evidence=dict(entry["evidence"], err_rel_l2=2e-5)))
    assert any("evidence missing" in v for v in viol(evidence={"incumbent": "x"}))
    assert viol(core="triton") == []  # the reference's name for the library's own core
    assert any("missing" in v for v in composition.table_violations(
        dict(table, entries=[{k: v for k, v in entry.items() if k != "core"}])))
    assert any("guard" in v for v in composition.table_violations(
        dict(table, entries=[dict(entry, candidate_ms=0.0199, guard_pct=0.5)])))
    sel = lambda **kw: composition.composition_select(  # noqa: E731
        "dit", kw.pop("n", 2048), batch=kw.pop("batch", 16), profile_hash=kw.pop("prof", PROF),
        env_hash=kw.pop("env", ENV), table=table, **kw)
    assert sel() == entry
    assert sel(batch=64) is None and sel(prof="0" * 16) is None and sel(env="1" * 16) is None
    assert sel(transform_direction="inverse") is None and sel(normalization="ortho") is None
    plan = _composition_plan(entry, 2048, 16, "dit", "fp32", "forward", "backward")
    assert plan.executed == "run_hybrid" and plan.params["core"] == "vendor" and plan.params["tile"] == 64


def test_hybrid_plan_contract():
    from kunlunxin_fft_amd.hybrid import HybridPlan, plan_hybrid

    p = plan_hybrid(2048, 16, tile=64)
    assert p.stage2_len == 32 and p.core == "vendor"
    # the reference's checks and key phrases (test_adapter_hybrid.py:19-30)
    with pytest.raises(ValueError, match="must divide"):
        plan_hybrid(2048, 1, tile=48)
    with pytest.raises(ValueError, match="powers of two"):
        plan_hybrid(960, 16, tile=64)  # divides, but N is not a power of two
    with pytest.raises(ValueError, match="must divide"):
        plan_hybrid(2048, 1, tile=4096)
    with pytest.raises(ValueError, match="DIT only"):
        HybridPlan(n=1024, batch=16, tile=64, direction="dif")
    with pytest.raises(ValueError, match="unknown core"):
        plan_hybrid(1024, 16, tile=64, core="external")
    # the reference's in-library core name selects this library's own core
    assert plan_hybrid(2048, 1, tile=64, core="triton").core == "local"
    with pytest.raises(ValueError):
        plan_hybrid(1 << 12, 1, tile=8, core="local")  # the local core needs tile >= 16


def test_semantic_specs_and_families():
    """The reference's semantic helpers (semantic.py:36-125): labels map to
    the selector's exact keys, families are the shared cores plus a real
    type's own flow, and the taxonomy self-check is clean."""
    from kunlunxin_fft_amd import semantic

    assert semantic.spec("c2r").key == ("c2r", "inverse", "backward")
    assert semantic.spec("c2c-inverse").transform_direction == "inverse"
    with pytest.raises(KeyError, match="unknown semantic label"):
        semantic.spec("c2c-sideways")
    assert semantic.family("c2c") == semantic.CORE_FLOWS
    assert semantic.family("r2c") - semantic.CORE_FLOWS == {"dedicated-r2c-pack-v1"}
    assert semantic.family_allows("c2r", "dedicated-c2r-hermitian-v1")
    assert not semantic.family_allows("r2c", "dedicated-c2r-hermitian-v1")
    assert semantic.family_size("r2c") == len(semantic.CORE_FLOWS) + 1
    with pytest.raises(KeyError):
        semantic.family("dct")
    assert semantic.validate_taxonomy() == []


def test_device_helpers_without_a_gpu():
    from kunlunxin_fft_amd import runner

    if not runner.device_ready():
        assert runner.device_name() == "cpu"


def test_default_table_is_read_once_per_file_version(tmp_path):
    """plan_fft's table lookups reuse the validated table until the file
    changes; load_table still returns a private copy each call."""
    import json
    import os

    from kunlunxin_fft_amd import selector

    src = selector.TABLE_PATH
    path = tmp_path / "t.json"
    path.write_text(open(src).read())
    a = selector.default_table(str(path))
    assert selector.default_table(str(path)) is a
    assert selector.load_table(str(path)) is not a and selector.load_table(str(path)) == a
    t = json.loads(path.read_text())
    t["entries"] = t["entries"][:3]
    path.write_text(json.dumps(t))
    os.utime(path, ns=(1, 1))  # a new version even within one mtime tick
    b = selector.default_table(str(path))
    assert b is not a and len(b["entries"]) == 3
    # an invalid new version raises, as load_table does
    path.write_text("{}")
    with pytest.raises(ConfigError):
        selector.default_table(str(path))


def test_composition_table_is_read_once_per_file_version(tmp_path):
    """composition_select reuses the validated composition table until the
    file changes, and the new version's entries then answer (an index of the
    shared selector table follows its file version too)."""
    import json
    import os

    from kunlunxin_fft_amd import composition, selector

    path = tmp_path / "c.json"
    path.write_text(open(composition.TABLE_PATH).read())
    a = composition._default_composition_table(str(path))
    assert composition._default_composition_table(str(path)) is a
    assert composition.load_composition_table(str(path)) is not a
    t = json.loads(path.read_text())
    t["measurements"] = t["measurements"][:2]
    path.write_text(json.dumps(t))
    os.utime(path, ns=(1, 1))
    b = composition._default_composition_table(str(path))
    assert b is not a and len(b["measurements"]) == 2
    assert composition._default_composition_table(str(tmp_path / "missing.json")) is None
    # the selector's index is dropped with the table version it belonged to
    sp = tmp_path / "t.json"
    sp.write_text(open(selector.TABLE_PATH).read())
    old = selector.default_table(str(sp))
    assert id(old) in selector._INDEX
    t = json.loads(sp.read_text())
    t["entries"] = t["entries"][:3]
    sp.write_text(json.dumps(t))
    os.utime(sp, ns=(2, 2))
    new = selector.default_table(str(sp))
    assert selector._INDEX.get(id(old), (None,))[0] is not old and selector._INDEX[id(new)][0] is new
