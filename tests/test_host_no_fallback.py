"""No CPU fallback: without libmfft.so (or without a GPU) every native entry
raises RuntimeError that says so, in a fresh process where the library was
never loaded.  No GPU needed: the error comes before any device call."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROBE = r"""
import sys
sys.path.insert(0, sys.argv[1])
import __graft_entry__
k = __graft_entry__.load_package()
from kunlunxin_fft_amd import native, runner
native.LIB_PATH = "/nonexistent/libmfft.so"
for name, call in (
        ("load", lambda: native.load()),
        ("native plan", lambda: runner.get_native_plan("fft_lds_fused_batch", 1024, 4, "c2c", "forward",
                                                       "backward", 256, {}, 0)),
        ("device props", lambda: native.device_props(0))):
    try:
        call()
    except RuntimeError as e:
        # the library's absence, or (here, with no GPU) the device's: never a CPU result
        assert "no CPU fallback" in str(e) or "GPU only" in str(e), (name, str(e))
        print("raised", name)
    else:
        print("NO ERROR", name)
"""


def test_missing_library_raises_everywhere():
    r = subprocess.run([sys.executable, "-c", PROBE, ROOT], capture_output=True, text=True, timeout=240, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = r.stdout.split()
    assert "NO" not in lines, r.stdout
    assert r.stdout.count("raised") == 3, r.stdout
