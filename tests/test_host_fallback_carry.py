"""The table builder's per-cell regression guard (carry_previous_fallbacks),
against a synthetic previously deployed table and a scripted paired timer:
a cell the rebuild would regress becomes a previous_fallbacks cell that the
loader accepts and that plan_fft runs with entry tier "previous-fallback";
nothing crosses environments; a previous fallback that no longer clears the
guard, or left the design space, is dropped with a reason.  No GPU needed."""
import copy
import json

import pytest

import kunlunxin_fft_amd as pkg
from kunlunxin_fft_amd.config import DeviceProfile
from kunlunxin_fft_amd.selector import FALLBACK_CARRY_CONTRACT, fallback_binding_violations, select
from kunlunxin_fft_amd.table_builder import carry_previous_fallbacks, cell_key

ENV = "65329e88886145f1"
PROFILE = DeviceProfile.load().hash()
DEVICE = {"device_model": "gfx950", "multiprocessor_count": 256, "max_shared_mem": 163840}


def lds_entry(n, b, elems, **extra):
    e = {"N": n, "batch": b, "direction": "dit", "incumbent_ms": 0.2, "incumbent_block": 256,
         "challenger_ms": 0.1, "evidence": {}, "reason": f"lds elems {elems}", "block": 256,
         "flow_id": "lds-stockham-single-pass", "flow_realization": "lds-resident",
         "processing_unit": "stockham-radix16", "params": {"elems": elems, "variant": "folded"},
         "executed": "fft_lds_fused_batch"}
    e.update(extra)
    return e


def table(entries, fallbacks=(), env=ENV):
    return {"schema_version": 1, "device": "amd-instinct-mi355x", "profile_hash": PROFILE, "env_hash": env,
            "env": dict(DEVICE), "precision": "fp32", "guard_pct": 2.0, "entries": list(entries),
            "previous_fallbacks": list(fallbacks)}


class Timer:
    """Paired timer with scripted medians per runner geometry; records calls."""

    def __init__(self, ms_by_elems):
        self.ms = ms_by_elems
        self.calls = []

    def __call__(self, new, old):
        self.calls.append((cell_key(new), new["params"].get("elems"), old["params"].get("elems")))
        f = lambda e: [self.ms[e["params"].get("elems")] * (1 + 0.001 * k) for k in (-1, 0, 1)]  # noqa: E731
        return f(new), f(old)


def test_regressed_cell_becomes_a_bound_fallback(tmp_path):
    prev = table([lds_entry(1024, 64, 16), lds_entry(2048, 64, 16)])
    new = table([lds_entry(1024, 64, 32), lds_entry(2048, 64, 16)])
    timer = Timer({16: 0.100, 32: 0.110})  # the rebuilt elems-32 choice is 10% slower
    fbs, drops, recs = carry_previous_fallbacks(prev, "ab" * 32, new, timer, guard=2.0)
    assert drops == [] and len(recs) == 1 and len(timer.calls) == 1  # the unchanged cell is not timed
    (fb,) = fbs
    assert fb["params"]["elems"] == 16 and fb["executed"] == "fft_lds_fused_batch"
    assert (fb["transform_type"], fb["transform_direction"], fb["normalization"]) == ("c2c", "forward", "backward")
    prov = fb["previous_fallback_provenance"]
    assert prov["carry_contract"] == FALLBACK_CARRY_CONTRACT and prov["source_env_hash"] == ENV
    assert prov["source_table_sha256"] == "ab" * 32 and len(prov["source_result_sha256"]) == 64
    assert prov["source_device"] == DEVICE and abs(prov["selector_vs_previous"] - 0.1) < 1e-6
    new["previous_fallbacks"] = fbs
    assert fallback_binding_violations(new) == []
    # the loader accepts the table; the planner runs the fallback cell
    path = tmp_path / "table.json"
    path.write_text(json.dumps(new))
    tab = pkg.load_table(str(path))
    sel = select("dit", 1024, 64, profile_hash=PROFILE, table=tab, env_hash=ENV)
    assert sel.entry_tier == "previous-fallback" and sel.params["elems"] == 16
    plan = pkg.plan_fft("dit", 1024, batch=64, profile_hash=PROFILE, table=tab, env_hash=ENV)
    assert plan.params.get("previous_fallback") is True and plan.params["elems"] == 16
    assert plan.reason.startswith("previous-deployed per-cell fallback")
    # other semantics and other cells still take the rebuilt entries
    plan2 = pkg.plan_fft("dit", 2048, batch=64, profile_hash=PROFILE, table=tab, env_hash=ENV)
    assert "previous_fallback" not in plan2.params
    plan3 = pkg.plan_fft("dit", 1024, batch=64, profile_hash=PROFILE, table=tab, env_hash=ENV,
                         transform_direction="inverse")
    assert plan3.params["elems"] == 32 and "previous_fallback" not in plan3.params


def test_a_change_within_the_guard_carries_nothing():
    prev = table([lds_entry(1024, 64, 16)])
    new = table([lds_entry(1024, 64, 32)])
    fbs, drops, recs = carry_previous_fallbacks(prev, "00" * 32, new, Timer({16: 0.100, 32: 0.1015}), guard=2.0)
    assert fbs == [] and drops == [] and len(recs) == 1


def test_nothing_crosses_environments():
    prev = table([lds_entry(1024, 64, 16)], env="ffffffffffffffff")
    new = table([lds_entry(1024, 64, 32)])
    timer = Timer({16: 0.05, 32: 0.2})
    fbs, drops, recs = carry_previous_fallbacks(prev, "00" * 32, new, timer, guard=2.0)
    assert fbs == [] and recs == [] and timer.calls == []
    assert len(drops) == 1 and "env_hash" in drops[0]


def test_previous_fallbacks_are_reconfirmed_or_dropped():
    old_fb = lds_entry(1024, 64, 8, transform_type="c2c", transform_direction="forward", normalization="backward",
                       previous_fallback_provenance={
                           "carry_contract": FALLBACK_CARRY_CONTRACT, "source_env_hash": ENV,
                           "source_profile_hash": PROFILE, "source_precision": "fp32", "source_device": DEVICE,
                           "source_table_sha256": "11" * 32, "source_result_sha256": "22" * 32,
                           "paired_confirm": "earlier rebuild"})
    prev = table([lds_entry(1024, 64, 16), lds_entry(4096, 64, 16)], fallbacks=[old_fb])
    # the previous decision for the cell is its fallback (elems 8), not its entry
    new = table([lds_entry(1024, 64, 32), lds_entry(4096, 64, 16)])
    fbs, drops, _ = carry_previous_fallbacks(prev, "33" * 32, new, Timer({8: 0.090, 32: 0.100}), guard=2.0)
    (fb,) = fbs
    assert fb["params"]["elems"] == 8
    assert fb["previous_fallback_provenance"]["source_table_sha256"] == "33" * 32  # rebound to the new source
    # still faster, but no longer by the guard: dropped with a reason
    fbs, drops, _ = carry_previous_fallbacks(prev, "33" * 32, new, Timer({8: 0.099, 32: 0.100}), guard=2.0)
    assert fbs == [] and len(drops) == 1 and "dropped" in drops[0]


def test_previous_fallbacks_failing_their_binding_are_dropped():
    bad = lds_entry(1024, 64, 8, transform_type="c2c", transform_direction="forward", normalization="backward",
                    previous_fallback_provenance={"carry_contract": FALLBACK_CARRY_CONTRACT})
    prev = table([lds_entry(1024, 64, 16)], fallbacks=[bad])
    new = table([lds_entry(1024, 64, 16)])
    timer = Timer({8: 0.01, 16: 0.1})
    fbs, drops, _ = carry_previous_fallbacks(prev, "00" * 32, new, timer, guard=2.0)
    # the unbound cell is not a previous decision; the previous entry equals the rebuilt one
    assert fbs == [] and timer.calls == [] and any("binding contract" in d for d in drops)


def test_previous_decisions_outside_the_design_space_are_not_carried():
    fb = lds_entry(1024, 64, 16, transform_type="c2c", transform_direction="forward", normalization="backward")
    fb.update(flow_id="four-step-two-pass", flow_realization="four-step", executed="fft_four_step_batch",
              params={"n1": 32, "chunk_rows": 0, "schedule": 2, "variant": "folded"})
    fb["previous_fallback_provenance"] = {
        "carry_contract": FALLBACK_CARRY_CONTRACT, "source_env_hash": ENV, "source_profile_hash": PROFILE,
        "source_precision": "fp32", "source_device": DEVICE, "source_table_sha256": "11" * 32,
        "source_result_sha256": "22" * 32, "paired_confirm": "earlier rebuild"}
    prev = table([lds_entry(1024, 64, 16)], fallbacks=[fb])
    new = table([lds_entry(1024, 64, 32)])
    timer = Timer({16: 0.01, 32: 0.1})
    fbs, drops, _ = carry_previous_fallbacks(prev, "00" * 32, new, timer, guard=2.0)
    assert fbs == [] and timer.calls == [] and any("design space" in d for d in drops)


def test_fallback_cells_missing_from_the_rebuild_are_dropped():
    fb = copy.deepcopy(lds_entry(8192, 64, 16, transform_type="c2c", transform_direction="forward",
                                 normalization="backward"))
    fb["previous_fallback_provenance"] = {
        "carry_contract": FALLBACK_CARRY_CONTRACT, "source_env_hash": ENV, "source_profile_hash": PROFILE,
        "source_precision": "fp32", "source_device": DEVICE, "source_table_sha256": "11" * 32,
        "source_result_sha256": "22" * 32, "paired_confirm": "earlier rebuild"}
    prev = table([lds_entry(1024, 64, 16)], fallbacks=[fb])
    new = table([lds_entry(1024, 64, 16)])
    fbs, drops, _ = carry_previous_fallbacks(prev, "00" * 32, new, Timer({16: 0.1}), guard=2.0)
    assert fbs == [] and any("not in the rebuilt sweep" in d for d in drops)


@pytest.mark.parametrize("prev", [None, {}])
def test_no_previous_table(prev):
    assert carry_previous_fallbacks(prev, None, table([]), Timer({}), guard=2.0) == ([], [], [])


@pytest.mark.parametrize("mutate,phrase", [
    (lambda p: p.update(source_env_hash="f" * 16), "source env"),
    (lambda p: p.update(source_profile_hash="f" * 16), "source profile"),
    (lambda p: p.update(source_precision="bf16"), "source precision"),
    (lambda p: p.update(source_device={"device_model": "gfx942", "multiprocessor_count": 304,
                                       "max_shared_mem": 65536}), "source device"),
    (lambda p: p.pop("source_result_sha256"), "missing binding key"),
    (lambda p: p.update(carry_contract="fallback-env-binding-v0"), "carry_contract"),
    (None, "provenance"),
])
def test_load_table_refuses_unbound_fallback_cells(tmp_path, mutate, phrase):
    """The loader's binding contract, with the reference's key phrases
    (test_selector.py:645-701)."""
    prev = table([lds_entry(1024, 64, 16)])
    new = table([lds_entry(1024, 64, 32)])
    fbs, _, _ = carry_previous_fallbacks(prev, "ab" * 32, new, Timer({16: 0.1, 32: 0.2}), guard=2.0)
    if mutate is None:
        fbs[0].pop("previous_fallback_provenance")
    else:
        mutate(fbs[0]["previous_fallback_provenance"])
    new["previous_fallbacks"] = fbs
    path = tmp_path / "t.json"
    path.write_text(json.dumps(new))
    with pytest.raises(pkg.ConfigError, match=phrase):
        pkg.load_table(str(path))
