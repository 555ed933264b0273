"""Live environment fingerprint (reference src/xpu/envcheck.py).

A selector table is only valid on the device / runtime / compiler stack it
was measured on.  ``collect()`` gathers, from this process: torch and its
HIP version, the device's gfx architecture, CU count and LDS size, the HIP
driver and runtime versions, and this library's ABI version.  Anything
missing (no GPU, library not built) makes the fingerprint unknown (None), and
the selector then fails closed to M0.  Scope is the card family: no
per-card identity is hashed, so every MI355X on the same stack shares one
fingerprint.  Cached per process.
"""
from __future__ import annotations

import hashlib
import json
from functools import lru_cache

REQUIRED = ("torch", "hip", "gfx_arch", "multiprocessor_count", "max_shared_mem",
            "driver", "runtime", "abi")
SCOPE = "card-family"


@lru_cache(maxsize=4)
def collect():
    """Fingerprint dict of device 0, or None when it cannot be determined."""
    try:
        import torch

        if not torch.cuda.is_available():
            return None
        from . import native

        props = native.device_props(0)
        env = {
            "torch": torch.__version__,
            "hip": getattr(torch.version, "hip", None),
            "gfx_arch": props["gcn_arch_name"].split(":")[0],
            "multiprocessor_count": int(props["multiprocessor_count"]),
            "max_shared_mem": int(props["shared_mem_per_block"]),
            "driver": int(props["driver_version"]),
            "runtime": int(props["runtime_version"]),
            "abi": int(props["abi_version"]),
        }
    except Exception:  # noqa: BLE001 -- unknown environment fails closed
        return None
    if any(env.get(k) in (None, "", 0) for k in REQUIRED):
        return None
    return env


def env_hash(env=None):
    """16-hex hash of a fingerprint dict; None when the environment is unknown."""
    if env is None:
        env = collect()
    if env is None:
        return None
    blob = json.dumps(env, sort_keys=True, separators=(",", ":"))
    return hashlib.sha256(blob.encode()).hexdigest()[:16]


def current_env_hash():
    return env_hash(collect())
