"""Device guard around every launch (reference src/xpu/context.py:43-66).

``device_context(device)`` makes the tensor's GPU current for the duration of
a launch (``runner.launch`` enters it whenever the tensor's GPU is not the
current one); the native plan is bound to the device that was current when
it was created.  ``xpu_context`` is the reference's name for the same guard.
A missing GPU stack is a RuntimeError, never a silent no-op.
"""
from __future__ import annotations

import contextlib


def device_ready() -> bool:
    try:
        import torch

        return bool(torch.cuda.is_available())
    except Exception:  # noqa: BLE001
        return False


@contextlib.contextmanager
def device_context(device):
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("no ROCm GPU available: the FFT kernels run on the GPU only")
    index = device.index if hasattr(device, "index") else int(device)
    if index is None:
        index = torch.cuda.current_device()
    with torch.cuda.device(index):
        yield index


@contextlib.contextmanager
def xpu_context(device: int = 0):
    """The reference's name for the device guard (context.py:43-66): make
    GPU ``device`` current for the body and restore the previous one after,
    also when the body raises; ``RuntimeError`` without a GPU stack."""
    with device_context(device) as index:
        yield index


def current_device_index() -> int:
    """Index of the current torch GPU (reference context.py:38-40)."""
    import torch

    return torch.cuda.current_device()


def device_name(index: int = 0) -> str:
    """Human-readable device string (reference runner.py:70-91): the
    device name with its architecture, CU count and LDS per CU; ``"cpu"``
    without a GPU."""
    if not device_ready():
        return "cpu"
    import torch

    p = torch.cuda.get_device_properties(index)
    arch = getattr(p, "gcnArchName", "").split(":")[0] or "unknown"
    lds = getattr(p, "shared_memory_per_multiprocessor", 0) or getattr(p, "max_shared_memory_per_multiprocessor", 0)
    return f"{p.name} ({arch}, {p.multi_processor_count} CUs, {lds // 1024} KiB LDS per CU)"
