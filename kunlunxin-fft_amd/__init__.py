"""MI355X (gfx950) FFT operator library with the Kunlunxin-FFT plan API.

Drop-in for the reference's ``src.xpu`` package on its complex64 1-D FFT
path: ``plan_fft`` / ``execute_fft_plan`` / ``run_fft`` / ``DeviceProfile``
keep their names, arguments, return types and error classes, while the
execution underneath is hand-written HIP for gfx950 behind the C ABI in
``include/mfft.h`` (``libmfft.so``, loaded through ``native``).

The package directory is ``kunlunxin-fft_amd``; it is imported under the
module name ``kunlunxin_fft_amd`` (``__graft_entry__.load_package()`` or
``importlib`` with ``submodule_search_locations``).

Host-only names (planning, tables, configs) import without torch;
torch-dependent names (runners) resolve lazily on first access, as in the
reference's ``src/xpu/__init__.py:37-81``.
"""
import importlib

from .config import (  # noqa: F401
    ConfigError,
    DesignSpace,
    DeviceProfile,
    Manifest,
    NORMALIZATIONS,
    SizeMatrix,
    TRANSFORM_DIRECTIONS,
    TRANSFORM_TYPES,
    build_manifest,
    git_commit,
    git_dirty,
)
from .entry import (  # noqa: F401
    SUPPORTED_NORMS,
    SUPPORTED_TRANSFORMS,
    SUPPORTED_TRANSFORM_DIRECTIONS,
    ExecutionPlan,
    ExecutionReport,
    execute_fft_plan,
    norm_scale,
    plan_fft,
    run_fft,
)
from .composition import composition_select, load_composition_table  # noqa: F401
from .error_metric import max_rel_error, rel_l2  # noqa: F401
from .selector import Selection, assert_current_environment, load_table, select  # noqa: F401

_TORCH_ATTRS = {
    "bit_reverse_permute": "runner",
    "device_name": "runner",
    "device_ready": "runner",
    "fft_dit": "runner",
    "fft_dif": "runner",
    "fft_dit_batch": "runner",
    "fft_dif_batch": "runner",
    "fft_dit_radix4": "runner",
    "fft_dif_radix4": "runner",
    "fft_dit_radix4_batch": "runner",
    "fft_dif_radix4_batch": "runner",
    "fft_lds_fused": "runner",
    "fft_lds_fused_batch": "runner",
    "fft_four_step": "runner",
    "fft_four_step_batch": "runner",
    "fft_dit_fused": "runner",
    "fft_dit_matrix": "runner",
    "fft_dif_matrix": "runner",
    "fft_dit_matrix_batch": "runner",
    "fft_dif_matrix_batch": "runner",
    "fft_dit_matrix_packet_batch": "runner",
    "fft_dit_grouped": "runner",
    "fft_dif_grouped": "runner",
    "log2_exact": "validate",
    "time_call": "runner",
    "time_call_detailed": "runner",
    "twiddle_tables": "runner",
    "device_context": "context",
    "xpu_context": "context",
    "validate_input": "validate",
}

__all__ = [
    "ConfigError", "DesignSpace", "DeviceProfile", "ExecutionPlan",
    "ExecutionReport", "Manifest", "Selection", "SizeMatrix", "SUPPORTED_NORMS", "SUPPORTED_TRANSFORMS",
    "SUPPORTED_TRANSFORM_DIRECTIONS", "assert_current_environment", "build_manifest",
    "composition_select", "execute_fft_plan", "git_commit", "git_dirty",
    "load_composition_table", "load_table", "max_rel_error", "norm_scale", "plan_fft", "rel_l2",
    "run_fft", "select",
    *sorted(_TORCH_ATTRS),
]


def __getattr__(name):
    if name in _TORCH_ATTRS:
        module = importlib.import_module(f".{_TORCH_ATTRS[name]}", __name__)
        value = getattr(module, name)
        globals()[name] = value
        return value
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


def __dir__():
    return sorted(__all__)
