"""Seeded random configurations through the plan API, against numpy float64.

Each case draws a runner (M0, M5, LDS, four-step), a transform type and
direction, a norm, N, a ragged batch, and the runner's parameters (threads
per block, elements per thread, start stagger, staged form, n1, chunk rows, schedule 0, 1 or 3,
pass-2 row order) from their published ranges (N <= 2^20), then checks the GPU result
to the north-star gate (rel-L2 and peak-normalised worst element <= 1e-5).
Sizes stay small enough (N * B <= 2^21) that the whole set runs in seconds.
A second set drives the real LDS modes through the C ABI with an explicit
16 or 32 elements per thread, and a third the fused four-step schedule with
random queue and ring settings.
"""
import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import ExecutionPlan, execute_fft_plan, native

pytestmark = pytest.mark.gpu

TOL = 1e-5
NORMS = ("none", "forward", "backward", "ortho")
# runner, smallest and largest log2 of the complex core
FLOWS = (("fft_dit", 1, 16), ("fft_dif", 1, 16), ("fft_dit_radix4", 2, 16), ("fft_dif_radix4", 2, 16),
         ("fft_lds_fused", 0, 15), ("fft_four_step", 8, 20))


def _cases(count=400, seed=20261202):
    rng = np.random.default_rng(seed)
    stage_rng = np.random.default_rng(seed + 1)  # the LDS staged form, drawn apart from the rest
    narrow_rng = np.random.default_rng(seed + 2)  # the narrow four-step schedule, likewise
    out = []
    for i in range(count):
        stage = int(stage_rng.integers(2))
        narrow = int(narrow_rng.integers(3)) == 0
        name, lo, hi = FLOWS[int(rng.integers(len(FLOWS)))]
        tt = ("c2c", "c2c", "r2c", "c2r")[int(rng.integers(4))]
        real = tt != "c2c"
        logc = int(rng.integers(lo, min(hi, 19 if real else 20) + 1))  # N <= 2^20
        logn = logc + (1 if real else 0)
        b = int(rng.integers(1, min(40, max(1, (1 << 21) >> logn)) + 1))
        td = "forward" if tt == "r2c" else ("inverse" if tt == "c2r" else ("forward", "inverse")[int(rng.integers(2))])
        norm = NORMS[int(rng.integers(4))]
        block, params = 256, {}
        if name in ("fft_dit", "fft_dif", "fft_dit_radix4", "fft_dif_radix4"):
            block = (64, 128, 256, 512, 1024)[int(rng.integers(5))]
        elif name == "fft_lds_fused":
            params = {"elems": (0, 4, 8, 16, 32)[int(rng.integers(5))], "stagger": (0, 0, 1, 3)[int(rng.integers(4))]}
            if stage:  # taken where fewer than 16 threads hold a transform, dropped elsewhere
                params["stage"] = 1
        else:
            params = {"n1": (0, 16, 32, 64, 128, 256, 512, 1024)[int(rng.integers(8))],
                      "chunk_rows": (0, 0, 1, 2, 3, 5)[int(rng.integers(6))], "schedule": int(rng.integers(2)),
                      "pass2_order": int(rng.integers(2))}
            if narrow:
                params["schedule"] = 3
        out.append(pytest.param(i, name, tt, td, norm, 1 << logn, b, block, params,
                                id=f"{i}-{name}-{tt}-{td}-{norm}-N{1 << logn}-B{b}"))
    return out


def _reference(x, tt, td, norm, n):
    if tt == "c2c":
        return oracle.c2c(x, td, norm) if n <= 4096 else _np_c2c(x, td, norm)
    np_norm = {"none": "backward" if tt == "r2c" else "forward", "forward": "forward", "backward": "backward",
               "ortho": "ortho"}[norm]
    if tt == "r2c":
        return np.fft.rfft(x.astype(np.float64), norm=np_norm)
    return np.fft.irfft(x.astype(np.complex128), n=n, norm=np_norm)


def _np_c2c(x, td, norm):
    x = x.astype(np.complex128)
    n = x.shape[-1]
    if td == "forward":
        return np.fft.fft(x, norm="backward" if norm == "none" else norm)
    if norm in ("none", "forward"):
        return np.fft.ifft(x, norm="backward") * n
    return np.fft.ifft(x, norm=norm)


@pytest.mark.parametrize("case,name,tt,td,norm,n,b,block,params", _cases())
def test_random_configuration(gpu, case, name, tt, td, norm, n, b, block, params):
    rng = np.random.default_rng(7000 + case)
    m = n // 2 + 1 if tt == "c2r" else n
    if tt == "r2c":
        h = rng.standard_normal((b, n)).astype(np.float32)
    else:
        h = (rng.standard_normal((b, m)) + 1j * rng.standard_normal((b, m))).astype(np.complex64)
    if b == 1:
        h = h[0]
    plan = ExecutionPlan(n=n, batch=b, direction="dit", precision="fp32", selection_source="table",
                         reason="random configuration", fallback=False,
                         executed=name + ("_batch" if b > 1 else ""), block=block, flow_id="test",
                         flow_realization="test", processing_unit="test", params=params, transform_type=tt,
                         transform_direction=td, norm=norm)
    y = execute_fft_plan(plan, torch.from_numpy(h).to(gpu)).cpu().numpy()
    ref = _reference(h, tt, td, norm, n)
    l2 = oracle.rel_l2(y, ref)
    mx = oracle.max_rel_error(y, ref)
    assert l2 <= TOL and mx <= TOL, f"rel_l2={l2:.3e} max_rel={mx:.3e}"


def _real_lds_cases(count=200, seed=4242):
    """Real LDS modes through the C ABI with an explicit 16 or 32 elements per
    thread (the plan API maps 32 to 16 below a 32768-point core), a start
    stagger, a norm and a ragged batch."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        tt = ("r2c", "c2r")[int(rng.integers(2))]
        e = (16, 32)[int(rng.integers(2))]
        logc = int(rng.integers(10, 16)) if e == 32 else int(rng.integers(6, 15))
        n = 1 << (logc + 1)
        b = int(rng.integers(1, min(40, max(1, (1 << 21) >> (logc + 1))) + 1))
        norm = NORMS[int(rng.integers(4))]
        stg = (0, 0, 1, 3)[int(rng.integers(4))]
        out.append(pytest.param(i, tt, e, n, b, norm, stg, id=f"{i}-{tt}-e{e}-N{n}-B{b}-{norm}-s{stg}"))
    return out


@pytest.mark.parametrize("case,tt,elems,n,b,norm,stagger", _real_lds_cases())
def test_random_real_lds_through_abi(gpu, case, tt, elems, n, b, norm, stagger):
    rng = np.random.default_rng(9000 + case)
    td = "forward" if tt == "r2c" else "inverse"
    p = native.NativePlan(n, b, tt, td, norm, native.FLOW_LDS_FUSED, (elems, stagger))
    if tt == "r2c":
        h = rng.standard_normal((b, n)).astype(np.float32)
        y = torch.full((b, n // 2 + 1), float("nan"), dtype=torch.complex64, device=gpu)
    else:
        m = n // 2 + 1
        h = (rng.standard_normal((b, m)) + 1j * rng.standard_normal((b, m))).astype(np.complex64)
        y = torch.full((b, n), float("nan"), dtype=torch.float32, device=gpu)
    x = torch.from_numpy(h).to(gpu)
    p.execute(x.data_ptr(), y.data_ptr(), torch.cuda.current_stream(gpu).cuda_stream)
    ref = _reference(h, tt, td, norm, n)
    got = y.cpu().numpy()
    l2 = oracle.rel_l2(got, ref)
    mx = oracle.max_rel_error(got, ref)
    assert l2 <= TOL and mx <= TOL, f"rel_l2={l2:.3e} max_rel={mx:.3e}"


def _fused_cases(count=60, seed=77001):
    """The fused four-step schedule (params[2] = 2) through the C ABI: every
    split it takes (n1, n2 in [128, 512] within a factor 2), C2C both ways
    and the real transforms on it, a ragged or chunked batch, a norm, and
    random queue lag, items per dequeue, Z slots per XCD and workgroups per
    CU (params[3] bits 0-7, 8-15, 16-23, 24-30)."""
    rng = np.random.default_rng(seed)
    splits = ((7, 7), (7, 8), (8, 7), (8, 8), (8, 9), (9, 8), (9, 9))
    out = []
    for i in range(count):
        l1, l2 = splits[int(rng.integers(len(splits)))]
        tt = ("c2c", "c2c", "r2c", "c2r")[int(rng.integers(4))]
        logn = l1 + l2 + (1 if tt != "c2c" else 0)
        b = int(rng.integers(1, min(24, max(1, (1 << 21) >> logn)) + 1))
        td = "forward" if tt == "r2c" else ("inverse" if tt == "c2r" else ("forward", "inverse")[int(rng.integers(2))])
        norm = NORMS[int(rng.integers(4))]
        lag = int(rng.integers(0, 7))
        take = int(rng.integers(0, 4))
        ring = 0 if lag == 0 else lag + 1 + int(rng.integers(0, 4))
        bpc = int(rng.integers(0, 5))
        chunk = (0, 0, 2, 5)[int(rng.integers(4))]
        word = lag | (take << 8) | (ring << 16) | (bpc << 24)
        out.append(pytest.param(i, tt, td, norm, 1 << logn, b, 1 << l1, chunk, word,
                                id=f"{i}-{tt}-{td}-{norm}-N{1 << logn}-B{b}-n1_{1 << l1}-c{chunk}-w{word:x}"))
    return out


def _real4_cases(count=80, seed=31337):
    """R2C / C2R on the four-step with the stitch and the pre-twiddle inside
    the passes (schedule 0): a random valid split of the half-length core
    (both passes 16..1024 points), a random norm, a ragged batch, and random
    batch chunks."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        tt = ("r2c", "c2r")[int(rng.integers(2))]
        logn = int(rng.integers(9, 21))
        logc = logn - 1
        l1 = int(rng.integers(max(4, logc - 10), min(10, logc - 4) + 1))
        b = int(rng.integers(1, min(24, max(1, (1 << 22) >> logn)) + 1))
        chunk = (0, 0, 1, 2, 3, 5)[int(rng.integers(6))]
        norm = NORMS[int(rng.integers(4))]
        td = "forward" if tt == "r2c" else "inverse"
        out.append(pytest.param(i, tt, td, norm, 1 << logn, b, 1 << l1, chunk,
                                id=f"{i}-{tt}-{norm}-N{1 << logn}-B{b}-n1_{1 << l1}-c{chunk}"))
    return out


@pytest.mark.parametrize("case,tt,td,norm,n,b,n1,chunk", _real4_cases())
def test_random_real_four_step(gpu, case, tt, td, norm, n, b, n1, chunk):
    """Every bin written (outputs start as NaN), against numpy, through the
    C ABI, with the two fused passes per chunk."""
    rng = np.random.default_rng(13000 + case)
    p = native.NativePlan(n, b, tt, td, norm, native.FLOW_FOUR_STEP, (n1, chunk, 0))
    chunks = -(-b // chunk) if chunk and chunk < b else 1
    assert p.info.launches == 2 * chunks
    if tt == "r2c":
        h = rng.standard_normal((b, n)).astype(np.float32)
        y = torch.full((b, n // 2 + 1), float("nan"), dtype=torch.complex64, device=gpu)
    else:
        h = (rng.standard_normal((b, n // 2 + 1)) + 1j * rng.standard_normal((b, n // 2 + 1))).astype(np.complex64)
        y = torch.full((b, n), float("nan"), dtype=torch.float32, device=gpu)
    x = torch.from_numpy(h).to(gpu)
    p.execute(x.data_ptr(), y.data_ptr(), torch.cuda.current_stream(gpu).cuda_stream)
    got = y.cpu().numpy()
    ref = _reference(h, tt, td, norm, n)
    l2 = oracle.rel_l2(got, ref)
    mx = oracle.max_rel_error(got, ref)
    assert l2 <= TOL and mx <= TOL, f"rel_l2={l2:.3e} max_rel={mx:.3e}"


@pytest.mark.parametrize("case,tt,td,norm,n,b,n1,chunk,word", _fused_cases())
def test_random_fused_schedule(gpu, case, tt, td, norm, n, b, n1, chunk, word):
    rng = np.random.default_rng(11000 + case)
    p = native.NativePlan(n, b, tt, td, norm, native.FLOW_FOUR_STEP, (n1, chunk, 2, word))
    if tt == "r2c":
        h = rng.standard_normal((b, n)).astype(np.float32)
        y = torch.full((b, n // 2 + 1), float("nan"), dtype=torch.complex64, device=gpu)
    else:
        m = n // 2 + 1 if tt == "c2r" else n
        h = (rng.standard_normal((b, m)) + 1j * rng.standard_normal((b, m))).astype(np.complex64)
        y = torch.full((b, n), float("nan"), dtype=torch.float32 if tt == "c2r" else torch.complex64, device=gpu)
    x = torch.from_numpy(h).to(gpu)
    p.execute(x.data_ptr(), y.data_ptr(), torch.cuda.current_stream(gpu).cuda_stream)
    got = y.cpu().numpy()
    assert p.sync_overruns() == 0
    ref = _reference(h, tt, td, norm, n)
    l2 = oracle.rel_l2(got, ref)
    mx = oracle.max_rel_error(got, ref)
    assert l2 <= TOL and mx <= TOL, f"rel_l2={l2:.3e} max_rel={mx:.3e}"
