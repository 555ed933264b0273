"""Several host threads using the library at once.

ctypes releases the GIL around every C call, so plan creation, executes and
error reporting really do run concurrently here.  Eight threads, each with
its own stream (default priority), create plans of different flows through
the C ABI and through plan_fft, execute them three times each on their own
stream, and check every result against numpy in float64 (rel-L2 and
peak-normalised worst element <= 1e-5).  A ninth thread keeps asking for
invalid plans meanwhile: each of its errors must carry its own message (the
last-error text is per thread), and the others' plans are unaffected.
Dropped plans are released from several threads at once at the end.
"""
import threading

import numpy as np
import pytest
import torch

import oracle
from kunlunxin_fft_amd import DeviceProfile, execute_fft_plan, native, plan_fft
from kunlunxin_fft_amd.runner import release_retired_plans

pytestmark = pytest.mark.gpu

TOL = 1e-5
# (N, batch, transform type, direction, flow, params)
CASES = [
    (2048, 64, "c2c", "forward", native.FLOW_LDS_FUSED, ()),
    (4096, 16, "r2c", "forward", native.FLOW_LDS_FUSED, ()),
    (1 << 17, 4, "c2c", "inverse", native.FLOW_FOUR_STEP, (256, 0, 0, 1)),
    (1 << 18, 3, "r2c", "forward", native.FLOW_FOUR_STEP, (512, 0, 0, 0)),
    (1 << 17, 2, "c2r", "inverse", native.FLOW_FOUR_STEP, (256, 1, 0, 0)),
    (4096, 8, "c2c", "forward", native.FLOW_RADIX2_DIT, ()),
    (1 << 14, 4, "c2c", "inverse", native.FLOW_RADIX4_DIF, ()),
    (1024, 32, "c2c", "forward", native.FLOW_DENSE_MFMA, ()),
]


def _input(rng, tt, n, b):
    if tt == "r2c":
        return rng.standard_normal((b, n)).astype(np.float32)
    m = n // 2 + 1 if tt == "c2r" else n
    return (rng.standard_normal((b, m)) + 1j * rng.standard_normal((b, m))).astype(np.complex64)


def _reference(h, tt, td, n):
    if tt == "r2c":
        return np.fft.rfft(h.astype(np.float64), axis=-1)
    if tt == "c2r":
        return np.fft.irfft(h.astype(np.complex128), n=n, axis=-1)
    hd = h.astype(np.complex128)
    return np.fft.fft(hd, axis=-1) if td == "forward" else np.fft.ifft(hd, axis=-1)


def _out(tt, n, b, dev):
    if tt == "r2c":
        return torch.full((b, n // 2 + 1), float("nan"), dtype=torch.complex64, device=dev)
    if tt == "c2r":
        return torch.full((b, n), float("nan"), dtype=torch.float32, device=dev)
    return torch.full((b, n), float("nan"), dtype=torch.complex64, device=dev)


def test_threads_share_the_library(gpu):
    prof = DeviceProfile.load().hash()
    start = threading.Barrier(len(CASES) + 1)
    stop = threading.Event()
    failures = []
    bad_messages = []

    def worker(i):
        try:
            n, b, tt, td, flow, params = CASES[i]
            rng = np.random.default_rng(4100 + i)
            h = _input(rng, tt, n, b)
            ref = _reference(h, tt, td, n)
            s = torch.cuda.Stream(device=gpu)
            start.wait(timeout=60)
            with torch.cuda.stream(s):
                x = torch.from_numpy(h).to(gpu)
                p = native.NativePlan(n, b, tt, td, "backward", flow, params)
                for rep in range(3):
                    y = _out(tt, n, b, gpu)
                    p.execute(x.data_ptr(), y.data_ptr(), s.cuda_stream)
                    got = y.cpu().numpy()  # synchronises with s
                    l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
                    if not (l2 <= TOL and mx <= TOL):
                        failures.append(f"case {i} C ABI rep {rep}: rel_l2={l2:.3e} max_rel={mx:.3e}")
                del p
                plan = plan_fft("dit", n, batch=b, profile_hash=prof, transform_type=tt,
                                transform_direction=td if tt == "c2c" else None)
                for rep in range(3):
                    got = execute_fft_plan(plan, x).cpu().numpy()
                    l2, mx = oracle.rel_l2(got, ref), oracle.max_rel_error(got, ref)
                    if not (l2 <= TOL and mx <= TOL):
                        failures.append(f"case {i} plan_fft rep {rep}: rel_l2={l2:.3e} max_rel={mx:.3e}")
        except Exception as e:  # noqa: BLE001
            failures.append(f"case {i}: {e!r}")

    def bad_plans():
        start.wait(timeout=60)
        while not stop.is_set():
            try:
                native.NativePlan(1000, 1)
                bad_messages.append("no error for n=1000")
            except ValueError as e:
                if "power of two" not in str(e):
                    bad_messages.append(str(e))
            try:
                native.NativePlan(1024, 0)
                bad_messages.append("no error for batch=0")
            except ValueError as e:
                if "batch" not in str(e):
                    bad_messages.append(str(e))

    # daemon threads: a stuck one fails the test below instead of holding the process
    threads = [threading.Thread(target=worker, args=(i,), daemon=True) for i in range(len(CASES))]
    noisy = threading.Thread(target=bad_plans, daemon=True)
    for t in threads + [noisy]:
        t.start()
    for t in threads:
        t.join(timeout=120)
    stop.set()
    noisy.join(timeout=30)
    assert not any(t.is_alive() for t in threads + [noisy]), "a thread did not finish"
    assert not failures, failures
    assert not bad_messages, bad_messages[:5]

    # dropped plans released from several threads at once
    rel = [threading.Thread(target=release_retired_plans, daemon=True) for _ in range(4)]
    for t in rel:
        t.start()
    for t in rel:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in rel), "a release did not finish"
    assert native.retired_count() == 0
