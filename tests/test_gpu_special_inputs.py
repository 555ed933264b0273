"""Special inputs, round trips and torch.fft equivalence through the plan API
(the cases of reference tests/test_inverse_c2c.py:107-180 and
tests/test_real_flow_hw.py:138-216), at the reference's shapes and at
shapes that take each flow of this library: LDS single-pass, the four-step
(N >= 2^16; real transforms from 2^17, with the stitch or pre-twiddle fused
into its passes) and a stage flow.

Inputs (reference test_inverse_c2c.py:60-82): an impulse at index 0, a
constant, a high-dynamic-range signal (magnitudes e^U(-3, 3), uniform
phases) and iid N(0, 1).  Every result is checked against numpy's float64
FFT to relative L2 <= 1e-5 and the reference's peak-normalised worst element
<= 1e-5."""
import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import DeviceProfile, ExecutionPlan, execute_fft_plan, plan_fft, run_fft

pytestmark = pytest.mark.gpu

TOL = 1e-5
KINDS = ("impulse", "constant", "hdr", "random")
PROF = DeviceProfile.load().hash()  # plans from the MI355X selector table


def make_c64(kind, n, b, seed):
    rng = np.random.default_rng(seed)
    if kind == "impulse":
        a = np.zeros((b, n), np.complex128)
        a[:, 0] = 1.0
    elif kind == "constant":
        a = np.full((b, n), 0.75 - 0.25j)
    elif kind == "hdr":
        a = np.exp(rng.uniform(-3, 3, (b, n))) * np.exp(1j * rng.uniform(0, 2 * np.pi, (b, n)))
    else:
        a = rng.standard_normal((b, n)) + 1j * rng.standard_normal((b, n))
    return a.astype(np.complex64)


def make_f32(kind, n, b, seed):
    rng = np.random.default_rng(seed)
    if kind == "impulse":
        a = np.zeros((b, n))
        a[:, 0] = 1.0
    elif kind == "constant":
        a = np.full((b, n), 0.75)
    elif kind == "hdr":
        a = np.exp(rng.uniform(-3, 3, (b, n))) * np.sign(rng.standard_normal((b, n)))
    else:
        a = rng.standard_normal((b, n))
    return a.astype(np.float32)


def check(got, ref, label):
    l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
    assert l2 <= TOL and mx <= TOL, f"{label}: rel_l2={l2:.3e} max_rel={mx:.3e}"


def mkplan(executed, n, b, tt="c2c", td="forward", norm="backward"):
    return ExecutionPlan(n=n, batch=b, direction="dit", precision="fp32", selection_source="table",
                         reason="test", fallback=False, executed=executed, block=256, params={},
                         transform_type=tt, transform_direction=td, norm=norm)


# (runner, n, b): the reference's shape on the planner's choice, and each flow
C2C_SHAPES = [(None, 512, 2), ("fft_lds_fused_batch", 4096, 4), ("fft_four_step_batch", 1 << 16, 2),
              ("fft_dif_radix4_batch", 2048, 2)]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("executed,n,b", C2C_SHAPES)
def test_inverse_special_inputs(gpu, kind, executed, n, b):
    x = make_c64(kind, n, b, seed=7)
    plan = plan_fft("dit", n, batch=b, profile_hash=PROF, transform_direction="inverse") if executed is None else \
        mkplan(executed, n, b, td="inverse")
    y = execute_fft_plan(plan, torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, np.fft.ifft(x.astype(np.complex128), axis=-1), f"inverse {kind} {plan.executed} N={n}")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("executed,n,b", C2C_SHAPES)
def test_forward_special_inputs(gpu, kind, executed, n, b):
    x = make_c64(kind, n, b, seed=8)
    plan = plan_fft("dit", n, batch=b, profile_hash=PROF) if executed is None else mkplan(executed, n, b)
    y = execute_fft_plan(plan, torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, np.fft.fft(x.astype(np.complex128), axis=-1), f"forward {kind} {plan.executed} N={n}")


REAL_SHAPES = [(None, 256, 16), ("fft_lds_fused_batch", 1 << 14, 4), ("fft_four_step_batch", 1 << 17, 2),
               ("fft_dit_batch", 1024, 4)]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("executed,n,b", REAL_SHAPES)
def test_r2c_special_inputs(gpu, kind, executed, n, b):
    x = make_f32(kind, n, b, seed=91)
    plan = plan_fft("dit", n, batch=b, profile_hash=PROF, transform_type="r2c") if executed is None else \
        mkplan(executed, n, b, tt="r2c")
    y = execute_fft_plan(plan, torch.from_numpy(x).to(gpu)).cpu().numpy()
    check(y, np.fft.rfft(x.astype(np.float64), axis=-1), f"r2c {kind} {plan.executed} N={n}")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("executed,n,b", REAL_SHAPES)
def test_c2r_of_special_spectra(gpu, kind, executed, n, b):
    """C2R of the spectra of the special real signals: the constant's is a
    lone DC bin, the impulse's is flat."""
    x = make_f32(kind, n, b, seed=92).astype(np.float64)
    h = np.fft.rfft(x, axis=-1).astype(np.complex64)
    plan = plan_fft("dit", n, batch=b, profile_hash=PROF, transform_type="c2r", transform_direction="inverse") \
        if executed is None else mkplan(executed, n, b, tt="c2r", td="inverse")
    y = execute_fft_plan(plan, torch.from_numpy(h).to(gpu)).cpu().numpy()
    check(y, np.fft.irfft(h.astype(np.complex128), n=n, axis=-1), f"c2r {kind} {plan.executed} N={n}")


@pytest.mark.parametrize("decomposition", ["dit", "dif"])
@pytest.mark.parametrize("n,b", [(256, 1), (1024, 16), (1 << 16, 2), (1 << 20, 1)])
def test_round_trip_identity(gpu, decomposition, n, b):
    """forward then inverse under "backward" gives the input back
    (reference test_inverse_c2c.py:121-137)."""
    x = torch.from_numpy(make_c64("random", n, b, seed=11)[0 if b == 1 else slice(None)]).to(gpu)
    fwd = plan_fft(decomposition, n, batch=b, profile_hash=PROF)
    inv = plan_fft(decomposition, n, batch=b, profile_hash=PROF, transform_direction="inverse")
    y = execute_fft_plan(inv, execute_fft_plan(fwd, x))
    check(y.cpu().numpy(), x.cpu().numpy().astype(np.complex128), f"round trip {decomposition} N={n} B={b}")


@pytest.mark.parametrize("n,b", [(256, 64), (4096, 1), (1 << 18, 2)])
def test_real_round_trip_identity(gpu, n, b):
    x = torch.from_numpy(make_f32("hdr", n, b, seed=12)[0 if b == 1 else slice(None)]).to(gpu)
    h = execute_fft_plan(plan_fft("dit", n, batch=b, profile_hash=PROF, transform_type="r2c"), x)
    c2r = plan_fft("dit", n, batch=b, profile_hash=PROF, transform_type="c2r", transform_direction="inverse")
    y = execute_fft_plan(c2r, h)
    check(y.cpu().numpy(), x.cpu().numpy().astype(np.float64), f"real round trip N={n} B={b}")


@pytest.mark.parametrize("n,b", [(256, 2), (2048, 16), (1 << 17, 2)])
def test_default_norms_match_torch_fft(gpu, n, b):
    """norm="backward" is torch.fft's default: the forward and inverse C2C,
    R2C and C2R plans equal torch.fft.fft / ifft / rfft / irfft (rocFFT here)
    to the same bound (reference test_inverse_c2c.py:169-180)."""
    x = torch.from_numpy(make_c64("random", n, b, seed=19)).to(gpu)
    r = torch.from_numpy(make_f32("random", n, b, seed=20)).to(gpu)
    cases = [
        (plan_fft("dit", n, batch=b, profile_hash=PROF), x, torch.fft.fft(x)),
        (plan_fft("dit", n, batch=b, profile_hash=PROF, transform_direction="inverse"), x, torch.fft.ifft(x)),
        (plan_fft("dit", n, batch=b, profile_hash=PROF, transform_type="r2c"), r, torch.fft.rfft(r)),
    ]
    h = torch.fft.rfft(r)
    c2r = plan_fft("dit", n, batch=b, profile_hash=PROF, transform_type="c2r", transform_direction="inverse")
    cases.append((c2r, h, torch.fft.irfft(h, n=n)))
    for plan, inp, ref in cases:
        y = execute_fft_plan(plan, inp)
        check(y.cpu().numpy(), ref.cpu().numpy().astype(np.complex128 if ref.is_complex() else np.float64),
              f"{plan.transform_type} {plan.transform_direction} vs torch.fft N={n}")


@pytest.mark.parametrize("n,b", [(128, 1), (1024, 16)])
def test_one_shot_matches_plan_reuse_inverse_ortho(gpu, n, b):
    """run_fft and a reused plan give the same bits (reference
    test_inverse_c2c.py:139-151)."""
    x = torch.from_numpy(make_c64("random", n, b, seed=13)[0 if b == 1 else slice(None)]).to(gpu)
    plan = plan_fft("dit", n, batch=b, profile_hash=PROF, transform_direction="inverse", norm="ortho")
    reused = execute_fft_plan(plan, x)
    once, report = run_fft(x, "dit", profile_hash=PROF, transform_direction="inverse", norm="ortho")
    assert report.executed == plan.executed and report.transform_direction == "inverse"
    assert torch.equal(once, reused)
