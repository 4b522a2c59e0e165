"""ctypes binding of libmoe_mi355x.so (the C ABI declared in include/moe_mi355x.h).

The library is the only compute path: when it is missing or cannot be loaded every
operation raises ``MoeLibraryError`` (there is no CPU or PyTorch fallback). ``torch`` is
imported first so the HIP runtime torch ships is the one the library binds to.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library links against)

LIB_PATH = Path(os.environ.get("MOE_MI355X_LIB", Path(__file__).resolve().parent / "libmoe_mi355x.so"))

ABI_VERSION = 3  # MOE_ABI_VERSION of include/moe_mi355x.h that SIGNATURES describes
MOE_OK = 0
MOE_EINVAL = 1
MOE_EHIP = 2
WEIGHTS_BF16 = 0
WEIGHTS_FP8_E4M3 = 1
ROUND_PRODUCT = 1
EXACT_PRODUCT = 2
NOALLOC_SCRATCH_BYTES = 16 << 20  # MOE_NOALLOC_SCRATCH_BYTES: moe_block_forward_noalloc's limit

_P = ctypes.c_void_p
_I = ctypes.c_int
_LL = ctypes.c_longlong
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES: dict[str, tuple] = {
    "moe_abi_version": (_I, []),
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_reload_tuning": (None, []),
    "moe_tile_rows": (_I, [_I]),
    "moe_max_tiles": (_I, [_I, _I, _I, _I, _I]),
    "moe_router_logits": (_I, [_P, _I, _I, _P, _I, _P, _P]),
    "moe_route_topk": (_I, [_P, _LL, _I, _I, _I, _P, _P, _P, _P]),
    "moe_sort_scratch_bytes": (_SZ, [_I, _I]),
    "moe_sort": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P, _P]),
    "moe_grouped_gate_up": (
        _I, [_P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _I, _I, _P, _P, _P, _I, _P, _P]),
    "moe_grouped_down": (
        _I, [_P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _I, _I, _P, _P, _I, _P, _P, _P]),
    "moe_combine": (_I, [_P, _P, _I, _I, _I, _P, _P, _LL, _P, _P, _I, _P]),
    "moe_decode_fits": (_I, [_I, _I, _I, _I, _I, _I]),
    "moe_decode_router": (_I, [_P, _I, _I, _P, _I, _P, _P, _I, _P, _P, _P]),
    "moe_decode_gate_up": (
        _I, [_P, _I, _I, _I, _I, _I, _P, _I, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P,
             _P]),
    "moe_decode_down": (
        _I, [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P, _I, _P, _P, _I, _P, _I, _P, _P]),
    "moe_experts_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "moe_experts_forward": (
        _I,
        [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _SZ, _P],
    ),
    "moe_block_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I, _I]),
    "moe_block_forward": (
        _I,
        [_P, _I, _I, _I, _I, _I, _I, _P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _P, _I,
         _P, _P, _P, _P, _P, _SZ, _P],
    ),
    "moe_block_forward_noalloc": (
        _I,
        [_P, _I, _I, _I, _I, _I, _I, _P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _P, _I,
         _P, _P, _P, _P, _P],
    ),
    "moe_add_rmsnorm": (_I, [_P, _P, _P, _I, _I, _F, _P, _P, _P]),
    "moe_block_forward_add_rms": (
        _I,
        [_P, _P, _P, _F, _I, _I, _I, _I, _I, _I, _P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _I,
         _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
    ),
}


class MoeLibraryError(RuntimeError):
    """The native library is missing, failed to load, or a launch failed."""


_lib = None


def load() -> ctypes.CDLL:
    """The loaded library (loaded once); raises ``MoeLibraryError`` if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise MoeLibraryError(
            f"{LIB_PATH} is not built: run `python __graft_entry__.py build` (or build.py) first"
        )
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        raise MoeLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.moe_abi_version() != ABI_VERSION:
        raise MoeLibraryError(
            f"{LIB_PATH} implements ABI {lib.moe_abi_version()}, this binding ABI {ABI_VERSION}: "
            "rebuild it"
        )
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Raise for a non-zero status: ValueError for an unsupported argument, else MoeLibraryError."""
    if rc == MOE_OK:
        return
    msg = (load().moe_last_error() or b"").decode(errors="replace")
    if rc == MOE_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise MoeLibraryError(f"{what}: {msg}")


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_of(t) -> int:
    """The current HIP stream of ``t``'s device, as the C ABI's ``void* stream``."""
    return torch.cuda.current_stream(t.device).cuda_stream


_WORKSPACES: dict = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A workspace of at least ``nbytes`` for calls on ``device``'s current stream.

    One workspace is kept per (device, stream) and reused (it is scratch: no call needs its
    contents cleared). Calls on one stream run in order, so they never share it
    concurrently."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, torch.cuda.current_stream(device).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, 256, 0 if ws is None else 2 * ws.numel())
        ws = torch.empty(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws
