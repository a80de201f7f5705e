"""Build provenance and the device/backend guard for the ROCm backend.

``build_info()`` plays the role of ``repop.build_info()`` (recorded by the
reference's audit replay, src/pretrain/cli/audit_replay.py:1508-1511) and
``require_backend`` the role of ``_require_repop_backend``
(audit_replay.py:1114-1141): a ``cuda`` device must be served by a GPU
backend that is actually compiled in, never by a silent fallback.  On
PyTorch-ROCm ``torch.device("cuda")`` is the AMD GPU, so a build whose
backends list ``rocm`` serves it when torch is a HIP build.
"""

from __future__ import annotations

import torch

from . import _lib


def build_info() -> dict:
    """{"commit", "backends", "rocm_arch_list", ...} of the loaded library.

    ``commit`` (12 hex digits, or "unknown" for a build outside a git
    checkout), ``dirty`` and ``sources_blake2b`` are the values stamped into
    the library when it was built, never read from the tree at run time: a
    deployed library without its checkout still names its build, and a
    rebuilt checkout cannot lend its commit to an older library."""
    native = _lib.native_build_info()
    return {
        "commit": native.get("commit", "unknown"),
        "dirty": native.get("dirty"),
        "sources_blake2b": native.get("sources_blake2b", "unknown"),
        "backends": list(native.get("backends", [])),
        "rocm_arch_list": native.get("arch", ""),
        "cuda_arch_list": "",
        "contract": native.get("contract", ""),
        "library": str(_lib.lib_path()),
    }


_UNSET = object()


def require_backend(dev: torch.device, info: dict, hip_version=_UNSET) -> None:
    """Raise unless ``info`` names a backend that can serve ``dev``.

    ``hip_version`` defaults to ``torch.version.hip`` (None on a CUDA or CPU
    build of torch); CPU is always allowed (it is the reference's own CPU
    path, not served by this package).
    """
    if hip_version is _UNSET:
        hip_version = torch.version.hip
    backends = info.get("backends", [])
    if dev.type == "cuda":
        served = "cuda" in backends or ("rocm" in backends and hip_version is not None)
        if not served:
            raise RuntimeError(
                f"--device {dev} requested but this build has no CUDA/ROCm backend "
                f"(build_info: commit={info.get('commit')!r}, backends={backends!r}, "
                f"torch.version.hip={hip_version!r}). Build libotx_attn.so on a "
                "PyTorch-ROCm install, or pass --device cpu to verify on CPU kernels explicitly."
            )
    elif dev.type == "mps":
        if "metal" not in backends:
            raise RuntimeError(
                f"--device {dev} requested but this build has no Metal backend "
                f"(build_info: commit={info.get('commit')!r}, backends={backends!r})."
            )


def require_device_available(device: str) -> torch.device:
    """The device-availability gate of audit_replay.py:1494-1506, ROCm-aware."""
    dev = torch.device(device)
    if dev.type == "cuda" and not torch.cuda.is_available():
        raise RuntimeError(
            f"--device {device} requested but CUDA is not available on this host "
            "(on ROCm: no HIP device visible). Pass --device cpu explicitly if a CPU "
            "replay is really intended."
        )
    return dev


# Environment that is part of the reproducibility contract on ROCm, captured
# next to the reference's CUDA keys (src/pretrain/train/loop.py:100-129 records
# CUBLAS_WORKSPACE_CONFIG and TORCH_CUDA_ARCH_LIST plus every REPOP* variable).
CONTRACT_ENV_KEYS = ("CUBLAS_WORKSPACE_CONFIG", "TORCH_CUDA_ARCH_LIST", "PYTORCH_ROCM_ARCH", "HIP_VISIBLE_DEVICES")


def capture_contract_env(environ=None) -> dict:
    """Every REPOP* / OTX* variable plus the contract keys that are set (values
    verbatim; unset keys stay unrecorded, as in loop.py:_capture_repop_env)."""
    import os

    environ = os.environ if environ is None else environ
    env = {k: v for k, v in environ.items() if k.startswith(("REPOP", "OTX"))}
    for k in CONTRACT_ENV_KEYS:
        v = environ.get(k)
        if v:
            env[k] = v
    return env
