"""Input validation for the tensor-level runners (reference src/xpu/validate.py).

Every check raises before any launch: ``TypeError`` for non-tensors and
wrong dtypes, ``ValueError`` for rank, contiguity, device, length and block
problems, ``RuntimeError`` when no GPU is present.
"""
from __future__ import annotations


def log2_exact(n: int) -> int:
    if not isinstance(n, int) or n <= 0 or (n & (n - 1)) != 0:
        raise ValueError(f"size must be a positive power of two, got {n}")
    return n.bit_length() - 1


def validate_tensor(x, name: str = "x", *, dtype=None, ranks=(1, 2), last=None,
                    block=None) -> None:
    import torch

    from .context import device_ready

    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(x).__name__}")
    if dtype is not None and x.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {x.dtype}")
    if x.dim() not in ranks:
        raise ValueError(f"{name} must have rank in {ranks}, got {x.dim()} (shape {tuple(x.shape)})")
    if not x.is_contiguous():
        raise ValueError(f"{name} must be contiguous; call .contiguous() first")
    if not device_ready():
        raise RuntimeError("no ROCm GPU available; cannot run the FFT kernels")
    if x.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU (device='cuda'), got device={x.device}")
    if last is not None and x.shape[-1] != last:
        raise ValueError(f"{name} last dim {x.shape[-1]} != expected {last}")
    if block is not None:
        log2_exact(block)


def validate_input(x, name: str = "x", *, allow_n: int | None = None, block: int | None = None,
                   require_complex: bool = True) -> None:
    """Rank-1 contiguous GPU tensor with a power-of-two length, complex64
    unless ``require_complex=False`` (reference validate.py:19-66)."""
    import torch

    validate_tensor(x, name, dtype=torch.complex64 if require_complex else None, ranks=(1,), block=block)
    log2_exact(x.numel())
    if allow_n is not None and x.numel() != allow_n:
        raise ValueError(f"{name} length {x.numel()} != expected {allow_n}")


def validate_batch_input(x, name: str = "x", *, block: int | None = None) -> None:
    """Rank-2 (B, N) complex64 contiguous GPU tensor, power-of-two N."""
    import torch

    validate_tensor(x, name, dtype=torch.complex64, ranks=(2,), block=block)
    log2_exact(int(x.shape[-1]))
    if x.shape[0] < 1:
        raise ValueError(f"{name} batch must be >= 1")


def validate_twiddle(tw, n: int, device) -> None:
    """A caller's twiddle table (reference validate.py:71-84): a ``(cos,
    sin)`` tuple of float32 tensors of length N/2 on the input's device.
    Both tables are checked (the reference's loop returns after the first)."""
    import torch

    if not isinstance(tw, tuple) or len(tw) != 2:
        raise TypeError("twiddle must be a (cos, sin) tuple from twiddle_tables()")
    for t, nm in zip(tw, ("cos", "sin")):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"twiddle {nm} must be a torch.Tensor")
        if t.dtype != torch.float32:
            raise TypeError(f"twiddle {nm} must be float32, got {t.dtype}")
        if t.device != device:
            raise ValueError(f"twiddle {nm} device {t.device} != input device {device}")
        if t.numel() != n >> 1:
            raise ValueError(f"twiddle {nm} length {t.numel()} != N/2 ({n >> 1})")
