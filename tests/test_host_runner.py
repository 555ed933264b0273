"""Host logic between the plan and the C ABI: runner parameters -> native
flow parameters, the selector's design-space contract for them, and the
table builder's candidate set.  No GPU needed."""
import json
import os

import pytest

from kunlunxin_fft_amd import native
from kunlunxin_fft_amd.config import DesignSpace
from kunlunxin_fft_amd.runner import flow_params
from kunlunxin_fft_amd.selector import entry_contract_violations
from kunlunxin_fft_amd.table_builder import candidates, real_candidates


def test_lds_params_map_to_elems_and_stagger():
    assert flow_params("fft_lds_fused_batch", 4096, "c2c", 256, {"elems": 16, "stagger": 2}) == \
        (native.FLOW_LDS_FUSED, (16, 2))
    # 32 elements need >= 1024 points; 2^13..2^14 take 16 or 32; 2^15 only 32
    assert flow_params("fft_lds_fused", 512, "c2c", 256, {"elems": 32})[1] == (0, 0)
    assert flow_params("fft_lds_fused", 8192, "c2c", 256, {"elems": 8})[1] == (0, 0)
    assert flow_params("fft_lds_fused", 32768, "c2c", 256, {"elems": 16, "stagger": 3})[1] == (0, 3)
    # a real transform's core is n/2: up to 32768 in the LDS kernel; r2c and
    # c2r cores below 32768 take 16 where a c2c entry says 32
    assert flow_params("fft_lds_fused", 2048, "r2c", 256, {"elems": 32})[1] == (16, 0)
    assert flow_params("fft_lds_fused", 1 << 16, "r2c", 256, {})[0] == native.FLOW_LDS_FUSED
    assert flow_params("fft_lds_fused", 1 << 16, "r2c", 256, {"elems": 32, "stagger": 1})[1] == (0, 1)
    assert flow_params("fft_lds_fused", 1 << 17, "r2c", 256, {})[0] == native.FLOW_AUTO
    assert flow_params("fft_lds_fused", 1 << 16, "c2r", 256, {})[0] == native.FLOW_LDS_FUSED
    # c2r takes 16 elements per thread where a c2c entry says 32 (core < 32768)
    assert flow_params("fft_lds_fused_batch", 1 << 14, "c2r", 256, {"elems": 32, "stagger": 1})[1] == (16, 1)
    assert flow_params("fft_lds_fused_batch", 1 << 11, "c2r", 256, {"elems": 32})[1] == (16, 0)
    assert flow_params("fft_lds_fused_batch", 1 << 14, "c2c", 256, {"elems": 32})[1] == (32, 0)


def test_four_step_params_map_to_split_chunk_schedule_order():
    p = {"n1": 512, "chunk_rows": 32, "schedule": 1, "pass2_order": 1}
    assert flow_params("fft_four_step_batch", 1 << 18, "c2c", 256, p) == (native.FLOW_FOUR_STEP, (512, 32, 1, 1))
    # an n1 that leaves n2 outside [16, 1024] falls back to the library's split
    assert flow_params("fft_four_step", 1 << 20, "c2c", 256, {"n1": 256})[1][0] == 0
    # the fused schedule only where both factors are 2^7..2^9 within 2x
    assert flow_params("fft_four_step", 1 << 20, "c2c", 256, {"n1": 1024, "schedule": 2})[1][2] == 0
    assert flow_params("fft_four_step", 1 << 16, "c2c", 256, {"n1": 256, "schedule": 2})[1][2] == 2
    # cores below 256 points leave the flow to the library
    assert flow_params("fft_four_step", 256, "r2c", 256, {})[0] == native.FLOW_AUTO


def test_stage_flows_validate_the_block():
    assert flow_params("fft_dit_batch", 1024, "c2c", 512, {}) == (native.FLOW_RADIX2_DIT, (512,))
    # any power of two, as in the reference; the workgroup clamps to 64..1024 threads
    assert flow_params("fft_dit", 1024, "c2c", 32, {}) == (native.FLOW_RADIX2_DIT, (64,))
    assert flow_params("fft_dit", 1024, "c2c", 2048, {}) == (native.FLOW_RADIX2_DIT, (1024,))
    with pytest.raises(ValueError):
        flow_params("fft_dit", 1024, "c2c", 96, {})
    with pytest.raises(ValueError):
        flow_params("no_such_runner", 1024, "c2c", 256, {})


def _entry(params, real="lds-resident", unit="stockham-radix16", n=1 << 14, b=2048, executed="fft_lds_fused_batch"):
    return {"N": n, "batch": b, "direction": "dit", "block": 256, "flow_id": "x", "flow_realization": real,
            "processing_unit": unit, "params": dict(params, variant="folded"), "executed": executed,
            "incumbent_ms": 1.0, "challenger_ms": 0.5, "reason": "test"}


def test_contract_accepts_published_params_and_refuses_others():
    sp = DesignSpace.load()
    ok = _entry({"elems": 32, "stagger": max(sp.lds_stagger)})
    assert not [v for v in entry_contract_violations(ok) if "stagger" in v]
    bad = _entry({"elems": 32, "stagger": 7})
    assert any("stagger" in v for v in entry_contract_violations(bad))
    fs = _entry({"n1": 512, "chunk_rows": 0, "pass2_order": 1}, real="four-step", n=1 << 18, b=128,
                executed="fft_four_step_batch")
    assert not [v for v in entry_contract_violations(fs) if "pass2_order" in v]
    fs_bad = _entry({"n1": 512, "chunk_rows": 0, "pass2_order": 2}, real="four-step", n=1 << 18, b=128,
                    executed="fft_four_step_batch")
    assert any("pass2_order" in v for v in entry_contract_violations(fs_bad))


def test_builder_offers_stagger_and_row_order_only_where_they_act():
    sp = DesignSpace.load()
    big = [c for c in candidates(1 << 15, 1024, "dit", sp) if c[1].startswith("fft_lds")]
    assert {c[3].get("stagger", 0) for c in big} == set(sp.lds_stagger)
    small = [c for c in candidates(1 << 15, 16, "dit", sp) if c[1].startswith("fft_lds")]
    assert {c[3].get("stagger", 0) for c in small} == {0}
    fs_batch = [c for c in candidates(1 << 18, 128, "dit", sp) if c[1].startswith("fft_four_step")]
    assert {c[3].get("pass2_order", 0) for c in fs_batch} == set(sp.fourstep_pass2_order)
    assert all(c[3].get("schedule", 0) in sp.fourstep_schedule for c in fs_batch)
    fs_one = [c for c in candidates(1 << 18, 1, "dit", sp) if c[1].startswith("fft_four_step")]
    assert {c[3].get("pass2_order", 0) for c in fs_one} == {0}
    # every candidate's parameters pass the loader's own contract
    for c in big + fs_batch:
        label, name, block, params, (real, unit, flow_id) = c
        e = _entry(params, real=real, unit=unit, n=1 << (15 if name.startswith("fft_lds") else 18),
                   b=1024 if name.startswith("fft_lds") else 128, executed=name)
        assert not entry_contract_violations(e), (label, entry_contract_violations(e))


def test_shipped_table_uses_only_published_params():
    sp = DesignSpace.load()
    path = os.path.join(os.path.dirname(__file__), "..", "kunlunxin-fft_amd", "config", "selector_table.json")
    t = json.load(open(path))
    for e in t["entries"]:
        p = e["params"]
        assert p.get("stagger", 0) in (0,) + sp.lds_stagger
        assert p.get("pass2_order", 0) in sp.fourstep_pass2_order
        assert p.get("schedule", 0) in sp.fourstep_schedule


def test_real_candidates_respect_the_real_modes():
    """Both real modes run the LDS kernel up to a 32768-point core, with 32
    elements per thread only there; every candidate passes the loader's
    contract as an exact-semantic entry."""
    sp = DesignSpace.load()
    for n in (1 << 10, 1 << 14, 1 << 15, 1 << 16, 1 << 20):
        b = max(64, (1 << 25) // n)
        for tt, td in (("r2c", "forward"), ("c2r", "inverse")):
            cands = real_candidates(n, b, tt, sp)
            assert cands
            lds = [c for c in cands if c[1].startswith("fft_lds")]
            assert all(c[3].get("elems") != 32 for c in lds if n // 2 < 32768)
            assert bool(lds) == (n // 2 <= 32768)
            for label, name, block, params, (real, unit, flow_id) in cands:
                e = _entry(params, real=real, unit=unit, n=n, b=b, executed=name)
                e.update(transform_type=tt, transform_direction=td, normalization="backward")
                assert not entry_contract_violations(e), (tt, n, label, entry_contract_violations(e))


def test_twiddle_contract_on_host_tensors():
    """runner.check_twiddle (reference validate.py:71-84 plus a value check),
    run on CPU tensors: forward-root tables pass, others raise."""
    import math

    import torch

    from kunlunxin_fft_amd.runner import TWIDDLE_TOL, check_twiddle, twiddle_tables

    for n in (2, 8, 1 << 12):
        x = torch.zeros(n, dtype=torch.complex64)
        check_twiddle(None, x)
        check_twiddle(twiddle_tables(n, "cpu"), x)
        # the reference's own tables: float32 angle, then cos/sin (runner.py:93-97)
        ang = (-2.0 * math.pi * torch.arange(n >> 1, dtype=torch.float32) / n).to(torch.float32)
        check_twiddle((torch.cos(ang), torch.sin(ang)), x)
        wr, wi = twiddle_tables(n, "cpu")
        wi = wi.clone()
        wi[0] += 10 * TWIDDLE_TOL
        with pytest.raises(ValueError, match="differs"):
            check_twiddle((wr, wi), x)
        # the inverse roots are a different table
        if n > 2:
            with pytest.raises(ValueError, match="differs"):
                check_twiddle((wr, -twiddle_tables(n, "cpu")[1]), x)
    # a checked table is remembered for its own tensor objects only: another
    # tensor at the same address and version (here a detached alias, written
    # through .data, which leaves the version alone) is checked again
    x = torch.zeros(16, dtype=torch.complex64)
    wr, wi = twiddle_tables(16, "cpu")
    check_twiddle((wr, wi), x)
    alias = wi.detach()
    assert alias.data_ptr() == wi.data_ptr() and alias._version == wi._version
    alias.data[1] += 10 * TWIDDLE_TOL
    with pytest.raises(ValueError, match="differs"):
        check_twiddle((wr, alias), x)
    wr, wi = twiddle_tables(16, "cpu")
    with pytest.raises(ValueError, match="length"):
        check_twiddle((wr[:4], wi[:4]), x)
    with pytest.raises(TypeError, match="float32"):
        check_twiddle((wr.double(), wi), x)
    with pytest.raises(TypeError, match="tuple"):
        check_twiddle([wr, wi], x)
    with pytest.raises(TypeError, match="torch.Tensor"):
        check_twiddle((wr, wi.numpy()), x)


def test_semantic_families():
    from kunlunxin_fft_amd.semantic import family_allows

    assert family_allows("r2c", "dedicated-r2c-pack-v1")
    assert not family_allows("c2r", "dedicated-r2c-pack-v1")
    assert not family_allows("c2c", "dedicated-c2r-hermitian-v1")
    assert all(family_allows(t, "four-step-two-pass") for t in ("c2c", "r2c", "c2r"))
    with pytest.raises(KeyError):
        family_allows("dct", "four-step-two-pass")


def test_release_retired_destroys_each_handle_once(monkeypatch):
    """Plans dropped by their owners wait in a list until release_retired
    destroys them; two threads releasing at once must not both take (and
    destroy) the same handles.  The list's copy is slowed down here so that,
    without the lock, both threads would copy it before either removed it."""
    import threading
    import time

    destroyed = []

    class FakeLib:
        def mfft_plan_destroy(self, h):
            destroyed.append(h)

    class SlowList(list):
        def __getitem__(self, i):
            got = list.__getitem__(self, i)
            if isinstance(i, slice):
                time.sleep(0.05)  # after the copy: others may copy the same items now
            return got

    retired = SlowList((("h%d" % i), 0) for i in range(100))
    monkeypatch.setattr(native, "_lib", FakeLib())
    monkeypatch.setattr(native, "_RETIRED", retired)
    start = threading.Barrier(4)
    counts = []

    def release():
        start.wait()
        counts.append(native.release_retired())

    threads = [threading.Thread(target=release) for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert sorted(destroyed) == sorted("h%d" % i for i in range(100))
    assert sum(counts) == 100 and len(retired) == 0


def test_staged_form_maps_only_where_it_exists():
    """The staged LDS form (params[2] = 1) reaches the C ABI for fewer than
    16 threads per transform of the core; elsewhere the mapping drops it, as
    the library would refuse it.  The builder offers it exactly there."""
    lds = native.FLOW_LDS_FUSED
    assert flow_params("fft_lds_fused_batch", 16, "c2c", 256, {"elems": 4, "stage": 1}) == (lds, (4, 0, 1))
    assert flow_params("fft_lds_fused_batch", 16, "c2c", 256, {"stage": 1}) == (lds, (0, 0, 1))  # default 16: T = 1
    assert flow_params("fft_lds_fused_batch", 128, "c2c", 256, {"elems": 16, "stage": 1}) == (lds, (16, 0, 1))
    assert flow_params("fft_lds_fused_batch", 64, "c2c", 256, {"elems": 4, "stage": 1}) == (lds, (4, 0))  # T = 16
    assert flow_params("fft_lds_fused_batch", 256, "c2c", 256, {"stage": 1}) == (lds, (0, 0))  # default 16: T = 16
    # real transforms: the core of length n/2 decides
    assert flow_params("fft_lds_fused_batch", 32, "r2c", 256, {"elems": 4, "stage": 1}) == (lds, (4, 0, 1))
    assert flow_params("fft_lds_fused_batch", 32, "c2r", 256, {"elems": 4, "stage": 1}) == (lds, (4, 0, 1))
    assert flow_params("fft_lds_fused_batch", 128, "r2c", 256, {"elems": 4, "stage": 1}) == (lds, (4, 0))  # T = 16
    sp = DesignSpace.load()
    for n in (16, 32, 64, 128, 256):
        staged = [c for c in candidates(n, 4096, "dit", sp) if c[3].get("stage")]
        want = {e for e in sp.lds_elems if e != 32 and n // min(e, n) < 16}
        assert {c[3]["elems"] for c in staged} == want, n
        for label, name, block, params, (real, unit, flow_id) in staged:
            e = _entry(params, real=real, unit=unit, n=n, b=4096, executed=name)
            assert not entry_contract_violations(e), (label, entry_contract_violations(e))
    bad = _entry({"elems": 4, "stage": 2}, n=16, b=4096)
    assert any("stage" in v for v in entry_contract_violations(bad))
