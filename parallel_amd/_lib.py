"""ctypes binding of the gfx950 C-ABI library (``include/moe_mi355x.h``).

The library is loaded after ``import torch`` on purpose: torch ships its own
``libamdhip64.so`` with SONAME ``libamdhip64.so.7``, and loading ours second
makes the dynamic linker reuse that copy, so torch streams and device pointers
are valid in our kernels.  A second HIP runtime in the process is detected and
refused.  There is no CPU fallback: every op raises if the library is absent.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

# MOE_MI355X_LIB selects another build of the same library (A/B comparisons).
LIB_PATH = Path(os.environ.get("MOE_MI355X_LIB") or Path(__file__).resolve().parent / "lib" / "libmoe_mi355x.so")
ABI_VERSION = 4

MOE_OK = 0
MOE_ERR_INVALID = -1
MOE_ERR_UNSUPPORTED = -2
MOE_ERR_LAUNCH = -3
MOE_ERR_WORKSPACE = -4

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/moe_mi355x.h one to one.
SIGNATURES: dict[str, tuple] = {
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_abi_version": (_I, []),
    "moe_router_logits_fwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "moe_router_fwd_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "moe_router_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _SZ, _P]),
    "moe_router_logits_bwd_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "moe_router_logits_bwd": (_I, [_P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _P, _SZ, _P]),
    "moe_router_topk_fwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "moe_router_topk_bwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P, _I, _P, _P]),
    "moe_router_topk_bwd_bf16": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _P, _P]),
    "moe_router_bf16_logits_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P, _P]),
    "moe_router_aux_bwd_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P, _P]),
    "moe_aux_loss_workspace_bytes": (_SZ, [_I64, _I64]),
    "moe_aux_loss_fwd": (_I, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "moe_aux_loss_bwd": (_I, [_P, _P, _P, _P, _I64, _I64, _P, _I, _P]),
    "moe_permute_workspace_bytes": (_SZ, [_I64, _I64]),
    "moe_permute_fwd": (_I, [_P, _I64, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "moe_permute_fwd_noalloc": (_I, [_P, _I64, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P]),
    "moe_f32_grouped_gemm": (_I, [_P, _P, _P, _I64, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64,
                                  _I64, _I64, _I, _P]),
    "moe_f32_swiglu_fwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "moe_f32_swiglu_bwd": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "moe_f32_combine_fwd": (_I, [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _P]),
    "moe_f32_combine_bwd": (_I, [_P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _P]),
    "moe_f32_permute_bwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "moe_dispatch_meta": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P]),
    "moe_permute_bwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "moe_combine_fwd": (_I, [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _P]),
    "moe_combine_bwd": (_I, [_P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _P]),
    "moe_combine_router_bwd": (_I, [_P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P,
                                    _I64, _I, _I, _P, _P]),
    "moe_grouped_gemm_swiglu_fwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "moe_grouped_gemm_fwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "moe_grouped_gemm_dgrad": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "moe_grouped_gemm_dgrad_swiglu_bwd": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "moe_grouped_gemm_wgrad": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _I, _I, _P]),
    "moe_grouped_gemm_wgrad_bucket": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I, _I, _P]),
    "moe_rmsnorm_fwd": (_I, [_P, _P, _I64, _I64, ctypes.c_float, _P, _P, _P]),
    "moe_rmsnorm_bwd_workspace_bytes": (_SZ, [_I64, _I64]),
    "moe_rmsnorm_bwd": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "moe_router_aux_fwd_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "moe_router_aux_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _SZ, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class MoeKernelError(RuntimeError):
    """A HIP launch failed inside the library."""


def _hip_runtimes_mapped() -> set[str]:
    try:
        with open("/proc/self/maps") as f:
            return {line.split()[-1] for line in f if "libamdhip64" in line and "/" in line}
    except OSError:
        return set()


def load() -> ctypes.CDLL:
    """Loads (once) and returns the library, raising if it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the gfx950 kernels with "
                "`python -m parallel_amd.build` (there is no CPU fallback)"
            )
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.moe_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {lib.moe_abi_version()}, expected {ABI_VERSION}: rebuild it")
        runtimes = {os.path.realpath(p) for p in _hip_runtimes_mapped()}
        if len(runtimes) > 1:
            raise RuntimeError(
                "two HIP runtimes are mapped into this process "
                f"({sorted(runtimes)}); import torch before parallel_amd"
            )
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    """Maps a library status to the reference's exception types."""
    if rc == MOE_OK:
        return
    msg = load().moe_last_error().decode(errors="replace")
    if rc in (MOE_ERR_INVALID, MOE_ERR_UNSUPPORTED, MOE_ERR_WORKSPACE):
        raise ValueError(f"{what}: {msg}")
    raise MoeKernelError(f"{what}: {msg} (status {rc})")


class KernelTimer:
    """Optional per-entry-point HIP event timing on torch's current stream.

    When enabled, every ``call`` (or, with ``only`` set, every call whose tag
    is in ``only``) records a start/end event pair around the entry point on
    the current stream (the stream the kernels are launched on);
    ``durations_ms()`` resolves them after a synchronisation.  An event pair
    costs several microseconds of stream time, so a timed region should
    instrument only the launches it needs."""

    def __init__(self):
        self.enabled = False
        self.only: set[str] | None = None
        self.events: dict[str, list] = {}

    def reset(self) -> None:
        self.events = {}

    def durations_ms(self) -> dict[str, list[float]]:
        return {k: [a.elapsed_time(b) for a, b in v] for k, v in self.events.items()}


TIMER = KernelTimer()


def call(name: str, *args, tag: str | None = None) -> None:
    """Calls an int-returning entry point and raises on a non-zero status.

    ``tag`` names the launch for KernelTimer (one entry point serves several
    GEMMs of different shapes)."""
    if TIMER.enabled and (TIMER.only is None or (tag or name) in TIMER.only):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        check(getattr(load(), name)(*args), name)
        end.record()
        TIMER.events.setdefault(tag or name, []).append((start, end))
        return
    check(getattr(load(), name)(*args), name)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on the tensor's device."""
    return torch.cuda.current_stream(t.device).cuda_stream
