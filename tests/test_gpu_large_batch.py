"""Batches past 2^31 elements (16 GiB and more per buffer) through every flow.

A row offset computed in 32 bits wraps once a buffer holds more than 2^31
complex values (2^32 floats for a real signal), so each case runs one plan
whose input or output crosses that mark.  The kernels index rows with 64-bit
offsets and lanes with offsets under 2^23 bytes; these cases check that the
rows past the mark land where they belong.  Every output starts as NaN and
must be fully written; sampled rows on both sides of the mark (the first, the
middle, the last, and the rows around element 2^31) are checked against numpy
in float64 to the north-star gate (rel-L2 and peak-normalised worst element
<= 1e-5).  The largest case holds 48 GiB of device memory at once.
"""
import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import native

pytestmark = pytest.mark.gpu

TOL = 1e-5
MARK_BYTES = 1 << 34  # element 2^31 of a complex64 buffer, 2^32 of a float32 one

# (id, N, batch, transform type, direction, flow, params)
CASES = [
    ("lds-c2c", 1024, (1 << 21) + 1, "c2c", "forward", native.FLOW_LDS_FUSED, (16, 0)),
    ("lds-c2c-inverse-e32", 4096, (1 << 19) + 3, "c2c", "inverse", native.FLOW_LDS_FUSED, (32, 1)),
    ("lds-r2c", 2048, (1 << 21) + 1, "r2c", "forward", native.FLOW_LDS_FUSED, ()),
    ("lds-c2r", 2048, (1 << 21) + 1, "c2r", "inverse", native.FLOW_LDS_FUSED, ()),
    ("fourstep-c2c", 1 << 20, (1 << 11) + 1, "c2c", "forward", native.FLOW_FOUR_STEP, (1024, 0, 0, 0)),
    ("fourstep-c2c-chunked-rev", 1 << 20, (1 << 11) + 1, "c2c", "forward", native.FLOW_FOUR_STEP,
     (1024, 1000, 0, 1)),
    ("fourstep-c2c-persistent", 1 << 17, (1 << 14) + 5, "c2c", "forward", native.FLOW_FOUR_STEP, (256, 0, 1, 0)),
    ("fourstep-c2c-narrow", 1 << 20, (1 << 11) + 1, "c2c", "inverse", native.FLOW_FOUR_STEP, (1024, 0, 3, 1)),
    ("fourstep-c2r-narrow", 1 << 20, (1 << 12) + 1, "c2r", "inverse", native.FLOW_FOUR_STEP, (512, 0, 3, 0)),
    ("fourstep-r2c", 1 << 20, (1 << 12) + 1, "r2c", "forward", native.FLOW_FOUR_STEP, (1024, 0, 0, 0)),
    ("fourstep-c2r", 1 << 20, (1 << 12) + 1, "c2r", "inverse", native.FLOW_FOUR_STEP, (512, 0, 0, 0)),
    ("radix4-dit", 1 << 16, (1 << 15) + 1, "c2c", "forward", native.FLOW_RADIX4_DIT, ()),
    ("mfma", 4096, (1 << 19) + 1, "c2c", "forward", native.FLOW_DENSE_MFMA, ()),
]


def _in_shape(tt, n, b):
    return (b, n // 2 + 1) if tt == "c2r" else (b, n)


def _out_shape(tt, n, b):
    return (b, n // 2 + 1) if tt == "r2c" else (b, n)


def _reference(h, tt, td, n):
    if tt == "r2c":
        return np.fft.rfft(h.astype(np.float64), axis=-1)
    if tt == "c2r":
        return np.fft.irfft(h.astype(np.complex128), n=n, axis=-1)
    hd = h.astype(np.complex128)
    return np.fft.fft(hd, axis=-1) if td == "forward" else np.fft.ifft(hd, axis=-1)


def _bytes(shape, complex_):
    return shape[0] * shape[1] * (8 if complex_ else 4)


@pytest.mark.parametrize("cid,n,b,tt,td,flow,params", CASES, ids=[c[0] for c in CASES])
def test_batch_past_2_31_elements(gpu, cid, n, b, tt, td, flow, params):
    ish, osh = _in_shape(tt, n, b), _out_shape(tt, n, b)
    in_complex, out_complex = tt != "r2c", tt != "c2r"
    # the input or the output crosses byte 2^34 (element 2^31 of complex64, 2^32 of float32)
    assert max(_bytes(ish, in_complex), _bytes(osh, out_complex)) > MARK_BYTES
    # rows around that byte in each buffer, and the ends and the middle
    marks = [MARK_BYTES // (shape[1] * (8 if cx else 4)) for shape, cx in ((ish, in_complex), (osh, out_complex))]
    rows = sorted({r for m in marks for r in (m - 1, m, m + 1) if 0 <= r < b} | {0, 1, b // 2, b - 2, b - 1})
    print(f"large batch {cid}: N={n} B={b} {tt} {td} rows {rows}", flush=True)
    p = native.NativePlan(n, b, tt, td, "backward", flow, params)
    g = torch.Generator(device=gpu)
    g.manual_seed(7000 + n + b)
    x = torch.randn(ish, dtype=torch.complex64 if in_complex else torch.float32, device=gpu, generator=g)
    y = torch.full(osh, float("nan"), dtype=torch.complex64 if out_complex else torch.float32, device=gpu)
    try:
        p.execute(x.data_ptr(), y.data_ptr(), torch.cuda.current_stream(gpu).cuda_stream)
        torch.cuda.synchronize(gpu)
        assert not bool(torch.isnan(y).any()), "an output element was never written"
        idx = torch.tensor(rows, device=gpu)
        h = x.index_select(0, idx).cpu().numpy()
        got = y.index_select(0, idx).cpu().numpy()
    finally:
        del x, y, p
        torch.cuda.empty_cache()
    ref = _reference(h, tt, td, n)
    l2 = oracle.rel_l2(got, ref)
    mx = oracle.max_rel_error(got, ref)
    assert l2 <= TOL and mx <= TOL, f"rows {rows}: rel_l2={l2:.3e} max_rel={mx:.3e}"
