"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against something that does not share its
code: the reference's own compiled CPU FFT (oracle/_ref, bit-exact when it
was built), the known-answer fixtures of tests/golden (closed forms and the
float64 DFT matrix), numpy.fft, and mathematical invariants.  A plausible
mistake -- a dropped twiddle, a wrong sign, a transposed index, a missing
conjugate or scale -- fails at least one of these.
"""
import numpy as np
import pytest

import oracle


def test_bit_reverse_kat(golden):
    assert [oracle.bit_reverse(i, 3) for i in range(8)] == list(golden["bitrev8"])


@pytest.mark.parametrize("n", [8, 16, 64, 256, 1024, 4096])
@pytest.mark.parametrize("dif", [False, True])
def test_core_matches_kat(golden, n, dif):
    x = golden[f"kat_in_{n}"]
    ref = golden[f"kat_out_{n}"]
    got = oracle.fft_dif(x) if dif else oracle.fft_dit(x)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    assert rel < 1e-10  # fft_check.cpp:67 gate


@pytest.mark.parametrize("n", [1, 2, 4, 8, 32])
def test_core_matches_bruteforce_dft(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    np.testing.assert_allclose(oracle.fft_dit(x), oracle.naive_dft(x), atol=1e-12)
    np.testing.assert_allclose(oracle.fft_dif(x), oracle.naive_dft(x), atol=1e-12)
    np.testing.assert_allclose(oracle.naive_dft(x, inverse=True), np.fft.ifft(x) * n, atol=1e-12)


@pytest.mark.parametrize("n", [2, 128, 2048, 65536])
def test_core_matches_numpy(n):
    rng = np.random.default_rng(n + 1)
    x = rng.standard_normal((3, n)) + 1j * rng.standard_normal((3, n))
    ref = np.fft.fft(x)
    assert oracle.rel_l2(oracle.fft_dit(x), ref) < 1e-14
    assert oracle.rel_l2(oracle.fft_dif(x), ref) < 1e-14


@pytest.mark.parametrize("n", [8, 256, 4096])
def test_core_bit_exact_with_reference_build(n):
    if oracle.reference_lib() is None:
        pytest.skip("oracle/_ref not built (reference tree absent at build time)")
    rng = np.random.default_rng(n)
    x = rng.standard_normal((2, n)) + 1j * rng.standard_normal((2, n))
    assert np.array_equal(oracle.fft_dit(x), oracle.reference_fft(x, dif=False))
    assert np.array_equal(oracle.fft_dif(x), oracle.reference_fft(x, dif=True))


def test_reference_build_bit_reverse():
    lib = oracle.reference_lib()
    if lib is None:
        pytest.skip("oracle/_ref not built")
    assert [lib.ref_bit_reverse(i, 5) for i in range(32)] == [oracle.bit_reverse(i, 5) for i in range(32)]


def test_known_signals(golden):
    np.testing.assert_allclose(oracle.fft_dit(golden["impulse256_in"]), golden["impulse256_out"], atol=1e-12)
    np.testing.assert_allclose(oracle.fft_dit(golden["tone256_in"]), golden["tone256_out"], atol=1e-9)
    y = oracle.fft_dit(golden["sentinel1024_in"])
    assert abs(y[0] - golden["sentinel1024_dc"][0]) < 1e-6
    np.testing.assert_allclose(oracle.fft_dit(golden["c1_in"]), golden["c1_out"], rtol=0, atol=1e-9)


@pytest.mark.parametrize("norm", oracle.NORMS)
@pytest.mark.parametrize("direction", ["forward", "inverse"])
def test_c2c_semantics_match_numpy(norm, direction):
    n = 64
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, n)) + 1j * rng.standard_normal((2, n))
    got = oracle.c2c(x, direction, norm)
    if direction == "forward":
        ref = np.fft.fft(x, norm="backward" if norm == "none" else norm)
    elif norm in ("none", "forward"):
        ref = np.fft.ifft(x, norm="backward") * n
    else:
        ref = np.fft.ifft(x, norm=norm)
    np.testing.assert_allclose(got, ref, atol=1e-12)


def test_norm_scale_table():
    n = 16
    assert oracle.norm_scale(n, "forward", "none") == 1.0
    assert oracle.norm_scale(n, "forward", "forward") == 1.0 / n
    assert oracle.norm_scale(n, "forward", "backward") == 1.0
    assert oracle.norm_scale(n, "inverse", "backward") == 1.0 / n
    assert oracle.norm_scale(n, "inverse", "forward") == 1.0
    assert oracle.norm_scale(n, "inverse", "ortho") == 0.25


@pytest.mark.parametrize("n", [8, 256])
def test_real_flows_match_fixtures(golden, n):
    np.testing.assert_allclose(oracle.r2c_dedicated(golden[f"rfft_in_{n}"]), golden[f"rfft_out_{n}"], atol=1e-11)
    np.testing.assert_allclose(oracle.c2r_dedicated(golden[f"irfft_in_{n}"], n), golden[f"irfft_out_{n}"], atol=1e-12)
    np.testing.assert_allclose(oracle.c2r_compat(golden[f"irfft_in_{n}"], n), golden[f"irfft_out_{n}"], atol=1e-12)


@pytest.mark.parametrize("n", [2, 4, 16, 4096])
@pytest.mark.parametrize("norm", oracle.NORMS)
def test_real_flows_match_numpy(n, norm):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((2, n))
    npn = "backward" if norm == "none" else norm
    X = np.fft.rfft(x, norm=npn)
    np.testing.assert_allclose(oracle.r2c_dedicated(x, norm), X, atol=1e-9)
    inv = np.fft.irfft(X, n=n, norm=norm) if norm != "none" else np.fft.irfft(X, n=n) * n
    np.testing.assert_allclose(oracle.c2r_dedicated(X, n, norm), inv, atol=1e-9)


def test_four_step_matches_numpy():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 512)) + 1j * rng.standard_normal((2, 512))
    for n1, n2 in ((16, 32), (32, 16), (8, 64)):
        np.testing.assert_allclose(oracle.four_step(x, n1, n2), np.fft.fft(x), atol=1e-10)
        np.testing.assert_allclose(oracle.four_step(x, n1, n2, "inverse"), np.fft.ifft(x) * 512, atol=1e-10)


def test_max_rel_error_closed_form():
    ref = np.array([3 + 4j, 0j])
    assert oracle.max_rel_error(ref, ref) == 0.0
    assert oracle.max_rel_error(np.array([3 + 4.5j, 0.1 + 0j]), ref) == pytest.approx(0.5 / 5.0)
    assert oracle.max_rel_error(np.array([np.nan, 0j]), ref) == float("inf")
    assert oracle.max_rel_error(np.array([3 + 4j, 1j * np.inf]), ref) == float("inf")


def test_planted_mistakes_are_caught():
    """A wrong sign, a missing conjugate or a dropped scale in a restatement
    must fail the numpy check the oracle is held to."""
    n = 32
    rng = np.random.default_rng(9)
    x = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    ref = np.fft.ifft(x, norm="backward")
    good = oracle.c2c(x, "inverse", "backward")
    assert oracle.rel_l2(good, ref) < 1e-14
    wrong_sign = oracle.fft_dit(x) / n                      # forward instead of inverse
    no_scale = np.conj(oracle.fft_dit(np.conj(x)))           # scale dropped
    one_conj = oracle.fft_dit(np.conj(x)) / n                # output conjugate dropped
    for bad in (wrong_sign, no_scale, one_conj):
        assert oracle.rel_l2(bad, ref) > 1e-3
