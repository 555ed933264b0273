"""The standalone real-flow epilogues (runner.r2c_stitch / c2r_pre /
c2r_unpack over mfft_r2c_stitch / mfft_c2r_pre / mfft_c2r_unpack;
reference runner.py:1687-1767) on the GPU: around this library's own C2C
core they give the oracle's R2C and C2R (numpy rfft / irfft in float64),
every norm's scale; they agree with the host references (*_ref) on the same
inputs; and the C ABI refuses bad sizes and overlapping buffers before any
launch."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import execute_fft_plan, native, norm_scale, plan_fft, runner

pytestmark = pytest.mark.gpu

TOL = 1e-5


def check(got, ref, label):
    l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
    assert l2 <= TOL and mx <= TOL, f"{label}: rel_l2={l2:.3e} max_rel={mx:.3e}"


def core(z, inverse=False):
    """The half-length complex core through this library's own plans."""
    b = 1 if z.dim() == 1 else int(z.shape[0])
    plan = plan_fft("dit", int(z.shape[-1]), batch=b, transform_direction="inverse" if inverse else "forward",
                    norm="none")
    return execute_fft_plan(plan, z)


SHAPES = [(4, 1), (8, 3), (64, 1), (1024, 4), (4096, 2), (1 << 16, 2), (1 << 20, 1)]


@pytest.mark.parametrize("n,b", SHAPES)
def test_r2c_stitch_around_the_core(gpu, n, b):
    rng = np.random.default_rng(7 + n + b)
    x = rng.standard_normal((b, n)).astype(np.float32)
    xin = x[0] if b == 1 else x
    z = core(torch.from_numpy(xin).to(gpu).view(torch.complex64))  # packed pairs x[2m] + i x[2m+1]
    X = runner.r2c_stitch(z, n).cpu().numpy()
    assert X.shape == ((n // 2 + 1,) if b == 1 else (b, n // 2 + 1))
    check(X, np.fft.rfft(xin.astype(np.float64), axis=-1), f"r2c_stitch N={n} B={b}")
    assert np.all(X[..., 0].imag == 0) and np.all(X[..., n // 2].imag == 0)
    ref = runner.r2c_stitch_ref(z.cpu(), n).numpy()
    assert oracle.rel_l2(X, ref) <= 1e-6


# every norm up to 2^12, the default norm at the large shapes
C2R_CASES = [(n, b, norm) for n, b in SHAPES for norm in ("none", "forward", "backward", "ortho")
             if n < (1 << 16) or norm == "backward"]


@pytest.mark.parametrize("n,b,norm", C2R_CASES)
def test_c2r_pre_core_unpack(gpu, n, b, norm):
    """c2r_pre -> forward core -> c2r_unpack with scale 2 * norm_scale(N,
    inverse, norm) gives numpy.fft.irfft under that norm; the imaginary parts
    of the DC and Nyquist bins are ignored."""
    rng = np.random.default_rng(11 + n + b)
    h = (rng.standard_normal((b, n // 2 + 1)) + 1j * rng.standard_normal((b, n // 2 + 1))).astype(np.complex64)
    hin = h[0] if b == 1 else h
    xh = torch.from_numpy(hin).to(gpu)
    z = runner.c2r_pre(xh, n)
    assert z.shape == ((n // 2,) if b == 1 else (b, n // 2)) and z.dtype == torch.complex64
    u = core(z)
    y = runner.c2r_unpack(u, n, 2.0 * norm_scale(n, "inverse", norm)).cpu().numpy()
    h64 = hin.astype(np.complex128).copy()
    h64[..., 0] = h64[..., 0].real
    h64[..., n // 2] = h64[..., n // 2].real
    # the inverse is unscaled under "none" and "forward" (norm_scale), numpy's "forward"
    np_norm = {"none": "forward", "forward": "forward", "backward": "backward", "ortho": "ortho"}[norm]
    check(y, np.fft.irfft(h64, n=n, axis=-1, norm=np_norm), f"c2r N={n} B={b} norm={norm}")
    zr = runner.c2r_pre_ref(xh.cpu(), n).numpy()
    assert oracle.rel_l2(z.cpu().numpy(), zr) <= 1e-6
    yr = runner.c2r_unpack_ref(u.cpu(), n, 2.0 * norm_scale(n, "inverse", norm)).numpy()
    assert oracle.rel_l2(y, yr) <= 1e-6


def test_epilogue_contract_errors(gpu):
    z = torch.zeros(32, dtype=torch.complex64, device=gpu)
    with pytest.raises(ValueError, match="last dim"):
        runner.r2c_stitch(z, 128)
    with pytest.raises(ValueError, match="last dim"):
        runner.c2r_pre(z, 128)  # needs N/2+1 = 65
    with pytest.raises(TypeError, match="complex64"):
        runner.c2r_unpack(z.real.contiguous(), 64)
    with pytest.raises(ValueError, match="N >= 4"):
        runner.r2c_stitch(torch.zeros(1, dtype=torch.complex64, device=gpu), 2)
    with pytest.raises(ValueError, match="power of two"):
        runner.r2c_stitch(z, 64, block=1000)
    with pytest.raises(ValueError, match="rank"):
        runner.r2c_stitch(torch.zeros((1, 2, 32), dtype=torch.complex64, device=gpu), 64)


def test_epilogue_c_abi_refuses_before_launch(gpu):
    lib = native.load()
    a = torch.zeros(4096, dtype=torch.complex64, device=gpu)
    b = torch.full((4096,), 7.0, dtype=torch.complex64, device=gpu)
    st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    pa, pb = ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr())
    assert lib.mfft_r2c_stitch(pa, pb, 2, 1, ctypes.c_float(1.0), st) == native.ERR_VALUE  # N < 4
    assert lib.mfft_c2r_pre(pa, pb, 96, 1, st) == native.ERR_VALUE  # not a power of two
    assert lib.mfft_c2r_unpack(pa, pb, 1 << 21, 1, ctypes.c_float(1.0), st) == native.ERR_VALUE  # beyond 2^20
    assert lib.mfft_r2c_stitch(pa, pb, 64, 0, ctypes.c_float(1.0), st) == native.ERR_VALUE  # batch 0
    assert lib.mfft_r2c_stitch(pa, ctypes.c_void_p(a.data_ptr() + 64), 64, 1, ctypes.c_float(1.0), st) \
        == native.ERR_VALUE  # overlapping
    assert lib.mfft_r2c_stitch(pa, pb, 64, 1, ctypes.c_float(float("inf")), st) == native.ERR_VALUE
    assert lib.mfft_c2r_pre(None, pb, 64, 1, st) == native.ERR_VALUE
    torch.cuda.synchronize()
    assert bool((b == 7.0).all())
