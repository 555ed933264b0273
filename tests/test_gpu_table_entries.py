"""Every C2C cell of the shipped selector table, through plan_fft and
execute_fft_plan: the plan resolves to the table's decision for the cell
(its previous-fallback cell where it has one, else its entry), and the
result matches numpy's float64 FFT on the first, a middle and the last row.
(The exact-semantic R2C / C2R entries run in test_gpu_parity.py.)"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import DeviceProfile, execute_fft_plan, plan_fft

pytestmark = pytest.mark.gpu

TOL = 1e-5
TABLE = os.path.join(os.path.dirname(__file__), "..", "kunlunxin-fft_amd", "config", "selector_table.json")


def _cells():
    t = json.load(open(TABLE))
    fallbacks = {(e["N"], e["batch"], e["direction"]): e for e in t.get("previous_fallbacks", [])
                 if e.get("transform_type", "c2c") == "c2c" and e.get("transform_direction", "forward") == "forward"
                 and e.get("normalization", "backward") == "backward"}
    out = []
    for e in t["entries"]:
        if "transform_type" in e:
            continue
        key = (e["N"], e["batch"], e["direction"])
        want = fallbacks.get(key, e)
        out.append(pytest.param(e["N"], e["batch"], e["direction"], want["executed"], want.get("params") or {},
                                id=f"N{e['N']}-B{e['batch']}-{e['direction']}"))
    return out


PROF = DeviceProfile.load().hash()


@pytest.mark.parametrize("n,b,direction,executed,params", _cells())
def test_table_cell_runs_its_decision_correctly(gpu, n, b, direction, executed, params):
    plan = plan_fft(direction, n, batch=b, profile_hash=PROF)
    assert plan.selection_source == "table" and not plan.fallback, plan.reason
    assert plan.executed == executed
    assert {k: v for k, v in plan.params.items() if k != "previous_fallback"} == params
    g = torch.Generator(gpu).manual_seed(n + 7 * b)
    x = torch.randn((b, n), dtype=torch.complex64, device=gpu, generator=g)
    y = execute_fft_plan(plan, x if b > 1 else x[0]).reshape(b, n)
    rows = sorted({0, b // 2, b - 1})
    ref = np.fft.fft(x[rows].cpu().numpy().astype(np.complex128))
    got = y[rows].cpu().numpy()
    l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
    assert l2 <= TOL and mx <= TOL, f"N={n} B={b} {direction} ({executed} {params}): rel_l2={l2:.3e} max={mx:.3e}"
    del x, y
