"""Write tests/golden/kat.npz: the reference's known-answer cases, as data.

Every input below restates a known-answer test of the reference, and every
expected output comes from a closed form or from the float64 DFT matrix
(numpy), never from the code under test:

* ``bitrev8``       bit_reverse(i, 3) for i < 8 -> {0,4,2,6,1,5,3,7}
                    (src/host/fft_check.cpp:43-54)
* ``kat_in_<N>`` / ``kat_out_<N>``  input re = sin(0.1 i + 1.3),
                    im = cos(0.2 i + 0.7) and its DFT, N in {8..4096}
                    (src/host/fft_check.cpp:56-76; gate rel < 1e-10)
* ``impulse256``    delta at 0 -> all ones (tests/test_fft.py:196-203)
* ``tone256``       exp(2*pi*i*5*n/256) -> 256 at bin 5 (test_fft.py:205-211)
* ``sentinel1024``  x = (1..N) - i*(1..N); DC bin = sum (scripts/smoke.py:72-94)
* ``c1_in`` / ``c1_out``  the reference's headline case: N=2048, B=1, seed
                    102026 + 10*N + B, real/imag iid N(0,1) complex64 and
                    its float64 FFT (scripts/issue10_wp3_holdout.py:127-140)
* ``rfft_in_<N>`` / ``rfft_out_<N>`` / ``irfft_out_<N>``  real input, its
                    half spectrum, and irfft of that half spectrum with the
                    DC/Nyquist imaginary parts set to 7.0 (ignored, as in
                    tests/test_real_transforms.py:335-347)

Run: python tests/golden/make_golden.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def dft_matrix(n, sign=-1.0):
    k = np.arange(n)
    return np.exp(sign * 2j * np.pi * np.outer(k, k) / n)


def main():
    out = {}
    out["bitrev8"] = np.array([0, 4, 2, 6, 1, 5, 3, 7], dtype=np.int64)
    for n in (8, 16, 64, 256, 1024, 4096):
        i = np.arange(n, dtype=np.float64)
        x = np.sin(0.1 * i + 1.3) + 1j * np.cos(0.2 * i + 0.7)
        out[f"kat_in_{n}"] = x
        out[f"kat_out_{n}"] = dft_matrix(n) @ x
    n = 256
    imp = np.zeros(n, np.complex128)
    imp[0] = 1.0
    out["impulse256_in"] = imp
    out["impulse256_out"] = np.ones(n, np.complex128)
    tone = np.exp(2j * np.pi * 5 * np.arange(n) / n)
    out["tone256_in"] = tone
    t = np.zeros(n, np.complex128)
    t[5] = n
    out["tone256_out"] = t
    n = 1024
    base = np.arange(1.0, n + 1.0)
    out["sentinel1024_in"] = base - 1j * base
    out["sentinel1024_dc"] = np.array([base.sum() - 1j * base.sum()])
    n, b = 2048, 1
    rng = np.random.default_rng(102026 + 10 * n + b)
    c1 = (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex64)
    out["c1_in"] = c1
    out["c1_out"] = dft_matrix(n) @ c1.astype(np.complex128)
    for n in (8, 256):
        rng = np.random.default_rng(7 + n)
        xr = rng.standard_normal(n)
        half = dft_matrix(n)[: n // 2 + 1] @ xr
        out[f"rfft_in_{n}"] = xr
        out[f"rfft_out_{n}"] = half
        h = half.copy()
        h[0] = h[0].real + 7.0j
        h[-1] = h[-1].real + 7.0j
        full = np.concatenate([h.real[:1], h[1:-1], h.real[-1:], np.conj(h[1:-1][::-1])])
        out[f"irfft_in_{n}"] = h
        out[f"irfft_out_{n}"] = (dft_matrix(n, +1.0) @ full).real / n
    np.savez_compressed(os.path.join(HERE, "kat.npz"), **out)
    print("wrote", os.path.join(HERE, "kat.npz"))


if __name__ == "__main__":
    main()
