"""The LDS kernel's staged form (LDS_FUSED params[2] = 1): for fewer than
16 threads per transform, a workgroup's rows come in and go out through LDS
with consecutive lanes on consecutive elements (C2C; R2C, whose bin rows
of N/2 + 1 values leave through a flat LDS array; C2R, whose bin rows come
in through one and are paired with their mirrors there).  Only the path
between HBM and the Stockham registers changes: its results must match the
unstaged kernel's to a few units in the last place (the two instantiations
may contract products into FMAs differently, which moves the last bit) and
the oracle to the parity bound, at every length, thread width, direction,
norm and batch (ragged last workgroups included); and the library refuses
the form where it does not exist."""
import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import ExecutionPlan, execute_fft_plan, native

pytestmark = pytest.mark.gpu

TOL = 1e-5


def staged_cases():
    out = []
    for logn in range(0, 8):
        for e in (4, 8, 16):
            le = min(e.bit_length() - 1, logn)
            if logn - le < 4 and (logn > 0 or e == 16):
                out.append((1 << logn, e))
    return out


def plan(n, b, elems, stage, td="forward", norm="backward", tt="c2c"):
    params = {"elems": elems}
    if stage:
        params["stage"] = 1
    return ExecutionPlan(n=n, batch=b, direction="dit", precision="fp32", selection_source="table",
                         reason="test", fallback=False, executed="fft_lds_fused" + ("_batch" if b > 1 else ""),
                         block=256, params=params, transform_type=tt, transform_direction=td, norm=norm)


def real_cases():
    # (N, elems): core N/2 of fewer than 16 threads at `elems` per thread
    return [(2 * c, e) for c, e in staged_cases()]


@pytest.mark.parametrize("n,elems", real_cases(), ids=[f"N{n}-e{e}" for n, e in real_cases()])
@pytest.mark.parametrize("b", [1, 3, 255, 4099])
def test_staged_real_equals_unstaged_and_numpy(gpu, n, elems, b):
    rng = np.random.default_rng(n * 7 + b)
    r = rng.standard_normal((b, n)).astype(np.float32)
    rt = torch.from_numpy(r if b > 1 else r[0]).to(gpu)
    for norm in ("backward", "ortho", "forward"):
        h = execute_fft_plan(plan(n, b, elems, 1, tt="r2c", norm=norm), rt)
        h0 = execute_fft_plan(plan(n, b, elems, 0, tt="r2c", norm=norm), rt)
        d = (h - h0).abs().max().item() / max(h0.abs().max().item(), 1e-30)
        assert d <= 4e-7, f"r2c N={n} e={elems} B={b} {norm}: staged differs by {d:.2e}"
        ref = np.fft.rfft(r.astype(np.float64), norm=norm)
        got = h.cpu().numpy().reshape(b, n // 2 + 1)
        l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
        assert l2 <= TOL and mx <= TOL, f"r2c N={n} e={elems} B={b} {norm}: rel_l2={l2:.3e} max={mx:.3e}"
        # C2R of the spectrum, with nonzero DC and Nyquist imaginary parts (ignored)
        hs = h0.clone()
        hs[..., 0] += 0.5j
        hs[..., -1] -= 0.25j
        y = execute_fft_plan(plan(n, b, elems, 1, td="inverse", tt="c2r", norm=norm), hs)
        y0 = execute_fft_plan(plan(n, b, elems, 0, td="inverse", tt="c2r", norm=norm), hs)
        d = (y - y0).abs().max().item() / max(y0.abs().max().item(), 1e-30)
        assert d <= 4e-7, f"c2r N={n} e={elems} B={b} {norm}: staged differs by {d:.2e}"
        ref = np.fft.irfft(h0.cpu().numpy().reshape(b, -1).astype(np.complex128), n=n, norm=norm)
        got = y.cpu().numpy().reshape(b, n)
        l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
        assert l2 <= TOL and mx <= TOL, f"c2r N={n} e={elems} B={b} {norm}: rel_l2={l2:.3e} max={mx:.3e}"


@pytest.mark.parametrize("n,elems", staged_cases(), ids=[f"N{n}-e{e}" for n, e in staged_cases()])
@pytest.mark.parametrize("b", [1, 3, 255, 257, 4099])
def test_staged_equals_unstaged_and_the_oracle(gpu, n, elems, b):
    rng = np.random.default_rng(n * 1000 + b)
    x = (rng.standard_normal((b, n)) + 1j * rng.standard_normal((b, n))).astype(np.complex64)
    xt = torch.from_numpy(x if b > 1 else x[0]).to(gpu)
    for td, norm in (("forward", "backward"), ("inverse", "backward"), ("inverse", "ortho"), ("forward", "forward")):
        staged = execute_fft_plan(plan(n, b, elems, 1, td, norm), xt)
        plain = execute_fft_plan(plan(n, b, elems, 0, td, norm), xt)
        d = (staged - plain).abs().max().item() / max(plain.abs().max().item(), 1e-30)
        assert d <= 4e-7, f"N={n} e={elems} B={b} {td} {norm}: staged differs from unstaged by {d:.2e}"
        ref = oracle.c2c(x.astype(np.complex128), td, norm)
        got = staged.cpu().numpy().reshape(b, n)
        l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
        assert l2 <= TOL and mx <= TOL, f"N={n} e={elems} B={b} {td} {norm}: rel_l2={l2:.3e} max={mx:.3e}"


def test_staged_large_batch_rows_at_the_ends(gpu):
    """A launch of many workgroups: the first, a middle and the last rows."""
    n, b = 16, 1 << 20
    g = torch.Generator(gpu).manual_seed(3)
    x = torch.randn((b, n), dtype=torch.complex64, device=gpu, generator=g)
    y = execute_fft_plan(plan(n, b, 4, 1), x)
    plain = execute_fft_plan(plan(n, b, 4, 0), x)
    assert (y - plain).abs().max().item() <= 4e-7 * plain.abs().max().item()
    rows = [0, b // 2 + 7, b - 1]
    ref = np.fft.fft(x[rows].cpu().numpy().astype(np.complex128))
    assert oracle.rel_l2(y[rows].cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("n,elems,tt", [(64, 4, "c2c"), (256, 16, "c2c"), (128, 4, "r2c"), (512, 16, "c2r"),
                                        (2048, 32, "c2c")])
def test_staged_refused_where_it_does_not_exist(gpu, n, elems, tt):
    """16 or more threads per transform of the core, or 32 elements per
    thread: the C ABI refuses params[2] = 1 (MFFT_ERR_UNSUPPORTED,
    ValueError here), and params[2] = 2 (MFFT_ERR_VALUE)."""
    td = "inverse" if tt == "c2r" else "forward"
    with pytest.raises(ValueError, match="staged"):
        native.NativePlan(n, 4, tt, td, "backward", native.FLOW_LDS_FUSED, (elems, 0, 1))
    with pytest.raises(ValueError, match="staged"):
        native.NativePlan(16, 4, "c2c", "forward", "backward", native.FLOW_LDS_FUSED, (4, 0, 2))


def test_runner_keywords_reach_the_staged_form(gpu):
    from kunlunxin_fft_amd import runner

    x = torch.randn((1024, 32), dtype=torch.complex64, device=gpu, generator=torch.Generator(gpu).manual_seed(9))
    ref = np.fft.fft(x.cpu().numpy().astype(np.complex128))
    for kw in ({"stage": 1}, {"stage": 1, "stagger": 1}, {}):
        y = runner.fft_lds_fused_batch(x, 4, **kw)
        assert oracle.rel_l2(y.cpu().numpy(), ref) <= TOL, kw
    y1 = runner.fft_lds_fused(x[0].contiguous(), 8, stage=1)
    assert oracle.rel_l2(y1.cpu().numpy(), ref[0]) <= TOL
