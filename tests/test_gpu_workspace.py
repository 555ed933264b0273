"""Caller-owned workspace through the C ABI: mfft_plan_create_ex with
MFFT_PLAN_CALLER_WORKSPACE, mfft_plan_workspace_size and mfft_execute_ws.

The same kernels run with the plan's own scratch or with the caller's, so the
results must be bit-identical, whatever the workspace held before; both are
also checked against numpy float64 to the north-star gate.
"""
import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import native

pytestmark = pytest.mark.gpu

TOL = 1e-5
ALIGN = 256

# n, batch, transform, direction, flow, params, (needs the real-flow buffer, needs the stage ping-pong)
CASES = [
    (4096, 3, "c2c", "forward", native.FLOW_RADIX2_DIT, (256,), (False, True)),
    (2048, 5, "c2c", "inverse", native.FLOW_RADIX4_DIF, (), (False, True)),
    (1 << 16, 3, "r2c", "forward", native.FLOW_FOUR_STEP, (256,), (True, False)),
    (1024, 4, "c2r", "inverse", native.FLOW_RADIX2_DIT, (), (True, True)),
    (4096, 2, "r2c", "forward", native.FLOW_LDS_FUSED, (), (False, False)),
    (1 << 18, 2, "c2c", "forward", native.FLOW_FOUR_STEP, (512,), (False, False)),
]


def _ids(c):
    return f"{c[2]}-{c[3]}-N{c[0]}-B{c[1]}-flow{c[4]}"


def _inputs(n, b, tt, gpu, seed):
    rng = np.random.default_rng(seed)
    if tt == "r2c":
        h = rng.standard_normal((b, n)).astype(np.float32)
    else:
        m = n // 2 + 1 if tt == "c2r" else n
        h = (rng.standard_normal((b, m)) + 1j * rng.standard_normal((b, m))).astype(np.complex64)
    return h, torch.from_numpy(h).to(gpu)


def _out(n, b, tt, gpu):
    if tt == "r2c":
        return torch.empty((b, n // 2 + 1), dtype=torch.complex64, device=gpu)
    if tt == "c2r":
        return torch.empty((b, n), dtype=torch.float32, device=gpu)
    return torch.empty((b, n), dtype=torch.complex64, device=gpu)


def _reference(h, n, tt, td):
    if tt == "r2c":
        return np.fft.rfft(h.astype(np.float64))
    if tt == "c2r":
        return np.fft.irfft(h.astype(np.complex128), n=n)
    x = h.astype(np.complex128)
    return np.fft.fft(x) if td == "forward" else np.fft.ifft(x)


def _workspace(nbytes, gpu, fill=float("nan")):
    # float32 storage rounded up; torch's caching allocator hands out
    # 512-byte aligned blocks
    w = torch.full(((max(nbytes, 4) + 3) // 4,), fill, dtype=torch.float32, device=gpu)
    assert w.data_ptr() % ALIGN == 0
    return w


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_caller_workspace_matches_plan_workspace(gpu, case):
    n, b, tt, td, flow, params, (need_a, need_b) = case
    st = torch.cuda.current_stream(gpu).cuda_stream
    own = native.NativePlan(n, b, tt, td, "backward", flow, params)
    cw = native.NativePlan(n, b, tt, td, "backward", flow, params, caller_workspace=True)
    core = b * (n // 2 if tt != "c2c" else n) * 8
    a_end = -(-core // ALIGN) * ALIGN if need_a else 0
    expect = (a_end + core) if need_b else (core if need_a else 0)
    assert own.workspace_size() == expect and cw.workspace_size() == expect
    assert own.info.workspace_bytes == expect  # held by the plan
    assert cw.info.workspace_bytes == 0         # held by nobody but the caller

    h, x = _inputs(n, b, tt, gpu, seed=1000 + n + b)
    y0 = _out(n, b, tt, gpu)
    own.execute(x.data_ptr(), y0.data_ptr(), st)
    ws = _workspace(expect, gpu)
    y1 = _out(n, b, tt, gpu)
    cw.execute_ws(x.data_ptr(), y1.data_ptr(), ws.data_ptr() if expect else 0, ws.numel() * 4, st)
    y2 = _out(n, b, tt, gpu)
    own.execute_ws(x.data_ptr(), y2.data_ptr(), ws.data_ptr() if expect else 0, ws.numel() * 4, st)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1) and torch.equal(y0, y2)
    ref = _reference(h, n, tt, td)
    got = y1.cpu().numpy()
    assert oracle.rel_l2(got, ref) <= TOL and oracle.max_rel_error(got, ref) <= TOL

    if expect:
        with pytest.raises(ValueError, match="mfft_execute_ws"):
            cw.execute(x.data_ptr(), y1.data_ptr(), st)
        with pytest.raises(ValueError, match="smaller"):
            cw.execute_ws(x.data_ptr(), y1.data_ptr(), ws.data_ptr(), expect - 8, st)
        roomy = _workspace(expect + ALIGN, gpu)
        with pytest.raises(ValueError, match="aligned"):
            cw.execute_ws(x.data_ptr(), y1.data_ptr(), roomy.data_ptr() + 8, roomy.numel() * 4 - 8, st)
        with pytest.raises(ValueError, match="needs"):
            cw.execute_ws(x.data_ptr(), y1.data_ptr(), 0, 0, st)
        big = _workspace(expect + y1.numel() * y1.element_size() + ALIGN, gpu)
        with pytest.raises(ValueError, match="overlap"):
            # output placed inside the workspace
            cw.execute_ws(x.data_ptr(), big.data_ptr() + ALIGN, big.data_ptr(), big.numel() * 4, st)
    else:
        cw.execute(x.data_ptr(), y1.data_ptr(), st)  # nothing to bring: the plain execute works


def test_caller_workspace_two_streams(gpu):
    """One plan, two streams, a workspace each: the executes may overlap in
    time and must not disturb each other."""
    n, b = 4096, 64
    p = native.NativePlan(n, b, "c2c", "forward", "backward", native.FLOW_RADIX2_DIT, (256,),
                          caller_workspace=True)
    nb = p.workspace_size()
    s1, s2 = torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)
    h1, x1 = _inputs(n, b, "c2c", gpu, seed=11)
    h2, x2 = _inputs(n, b, "c2c", gpu, seed=12)
    w1, w2 = _workspace(nb, gpu), _workspace(nb, gpu)
    y1, y2 = _out(n, b, "c2c", gpu), _out(n, b, "c2c", gpu)
    torch.cuda.synchronize()
    for _ in range(3):
        p.execute_ws(x1.data_ptr(), y1.data_ptr(), w1.data_ptr(), nb, s1.cuda_stream)
        p.execute_ws(x2.data_ptr(), y2.data_ptr(), w2.data_ptr(), nb, s2.cuda_stream)
    torch.cuda.synchronize()
    for h, y in ((h1, y1), (h2, y2)):
        ref = np.fft.fft(h.astype(np.complex128))
        assert oracle.rel_l2(y.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("flow,params,n", [(native.FLOW_LDS_FUSED, (), 4096), (native.FLOW_FOUR_STEP, (256,), 1 << 16),
                                           (native.FLOW_FOUR_STEP, (0, 0, 1), 1 << 17),
                                           (native.FLOW_FOUR_STEP, (0, 0, 3), 1 << 18)])
def test_no_workspace_plan_two_streams(gpu, flow, params, n):
    """A plan that needs no workspace holds nothing an execute writes, so two
    streams may run it at once."""
    b = 32
    p = native.NativePlan(n, b, "c2c", "forward", "backward", flow, params)
    assert p.workspace_size() == 0 and p.info.workspace_bytes == 0
    s1, s2 = torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)
    h1, x1 = _inputs(n, b, "c2c", gpu, seed=21)
    h2, x2 = _inputs(n, b, "c2c", gpu, seed=22)
    y1, y2 = _out(n, b, "c2c", gpu), _out(n, b, "c2c", gpu)
    torch.cuda.synchronize()
    for _ in range(3):
        p.execute(x1.data_ptr(), y1.data_ptr(), s1.cuda_stream)
        p.execute(x2.data_ptr(), y2.data_ptr(), s2.cuda_stream)
    torch.cuda.synchronize()
    for h, y in ((h1, y1), (h2, y2)):
        rows = [0, b - 1]
        ref = np.fft.fft(h[rows].astype(np.complex128))
        assert oracle.rel_l2(y[rows].cpu().numpy(), ref) <= TOL


def test_plan_api_two_streams_share_cached_plans(gpu):
    """execute_fft_plan on two streams at once, for plans that need scratch
    (an M0 stage flow and a 2^18-point R2C over the four-step core): the
    cached native plans take their scratch per call from torch's allocator
    on the calling stream, so overlapping executes do not share it.  Every
    result equals the same plan's eager result on the default stream."""
    from kunlunxin_fft_amd import ExecutionPlan, execute_fft_plan

    def mk(executed, n, b, tt="c2c", params=None):
        return ExecutionPlan(n=n, batch=b, direction="dit", precision="fp32", selection_source="table",
                             reason="test", fallback=False, executed=executed, block=256, flow_id="test",
                             flow_realization="test", processing_unit="test", params=params or {},
                             transform_type=tt)

    m0 = mk("fft_dit_batch", 4096, 64)
    r2c = mk("fft_four_step_batch", 1 << 18, 4, tt="r2c", params={"n1": 256})
    xs = {}
    for plan, seed in ((m0, 41), (r2c, 42)):
        rng = np.random.default_rng(seed)
        for k in range(2):
            if plan.transform_type == "r2c":
                h = rng.standard_normal((plan.batch, plan.n)).astype(np.float32)
            else:
                h = (rng.standard_normal((plan.batch, plan.n))
                     + 1j * rng.standard_normal((plan.batch, plan.n))).astype(np.complex64)
            xs[(id(plan), k)] = torch.from_numpy(h).to(gpu)
    eager = {key: execute_fft_plan(m0 if key[0] == id(m0) else r2c, x).cpu() for key, x in xs.items()}
    s1, s2 = torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)
    torch.cuda.synchronize()
    outs = {}
    for _ in range(3):
        for k, st in ((0, s1), (1, s2)):
            with torch.cuda.stream(st):
                for plan in (m0, r2c):
                    x = xs[(id(plan), k)]
                    x.record_stream(st)
                    outs[(id(plan), k)] = execute_fft_plan(plan, x)
    torch.cuda.synchronize()
    for key, y in outs.items():
        assert torch.equal(y.cpu(), eager[key]), key


def test_clear_native_cache_keeps_plans_working(gpu):
    """runner.clear_native_cache drops every cached native plan and destroys
    those nothing holds (after a device sync); a plan executed before keeps
    its own native plan, a new one of the same shape gets a fresh one, and
    both give the same result as before."""
    from kunlunxin_fft_amd import ExecutionPlan, execute_fft_plan, runner

    def mk(n, b):
        return ExecutionPlan(n=n, batch=b, direction="dit", precision="fp32", selection_source="table",
                             reason="test", fallback=False, executed="fft_lds_fused_batch", block=256,
                             flow_id="test", flow_realization="test", processing_unit="test", params={})

    rng = np.random.default_rng(77)
    h = (rng.standard_normal((8, 1024)) + 1j * rng.standard_normal((8, 1024))).astype(np.complex64)
    x = torch.from_numpy(h).to(gpu)
    plan = mk(1024, 8)
    before = execute_fft_plan(plan, x).cpu()
    # a second shape, so that the cache holds a plan no ExecutionPlan refers to
    execute_fft_plan(mk(2048, 4), torch.zeros((4, 2048), dtype=torch.complex64, device=gpu))
    runner.clear_native_cache()
    assert native.retired_count() == 0
    assert torch.equal(execute_fft_plan(plan, x).cpu(), before)
    assert torch.equal(execute_fft_plan(mk(1024, 8), x).cpu(), before)
    ref = np.fft.fft(h.astype(np.complex128))
    assert oracle.rel_l2(before.numpy(), ref) <= TOL


@pytest.mark.parametrize("n,batch,flow,params", [
    (1024, 1 << 25, native.FLOW_LDS_FUSED, ()),          # 2^31 work-items per launch
    (1 << 20, 1 << 16, native.FLOW_FOUR_STEP, (1024,)),  # 2^31 per pass
])
def test_plans_below_the_dispatch_limit_are_created(gpu, n, batch, flow, params):
    """A dispatch holds fewer than 2^32 work-items, so plan creation refuses
    shapes whose largest launch would reach that (CPU tests); shapes below it
    are accepted.  These plans take no workspace and are only created:
    executing them would need 256 GiB of buffers."""
    p = native.NativePlan(n, batch, "c2c", "forward", "backward", flow, params)
    assert p.info.batch == batch and p.ws_bytes == 0
