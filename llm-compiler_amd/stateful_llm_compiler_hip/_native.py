"""ctypes binding of ``libslc_hip.so`` (the C ABI declared in include/slc_hip.h).

The library is loaded lazily on first use and never replaced by anything
else: if it is missing or fails to load, every kernel entry point raises
``NativeLibraryError``.  There is no PyTorch or CPU fallback behind these
functions.
"""

from __future__ import annotations

import ctypes
import os
import threading
from collections import OrderedDict
from pathlib import Path

import torch

LIBRARY_PATH = Path(
    os.environ.get(
        "SLC_HIP_LIBRARY",
        str(Path(__file__).resolve().parent / "libslc_hip.so"),
    )
)

SLC_F32 = 0
SLC_F16 = 1
SLC_BF16 = 2
SLC_I32 = 3
SLC_I64 = 4

# slc_softmax_order
SOFTMAX_ORDERS = {"online": 0, "exact": 1}
# Workgroup tiles of the prefill-sized linear (SLC_TILE_* in slc_hip.h).
LINEAR_TILES = {"auto": 0, "t128x128": 1, "t128x64": 2, "t64x128": 3, "t64x64": 4, "t32x64": 5,
                "r128x128": 6, "r256x128": 7, "r128x64": 8, "r64x64": 9,
                "s256x128": 10}

# slc_split: decode attention's length-balanced split-sequence variant
SPLIT_BALANCED = -1

_DTYPE_TAGS = {
    torch.float32: SLC_F32,
    torch.float16: SLC_F16,
    torch.bfloat16: SLC_BF16,
    torch.int32: SLC_I32,
    torch.int64: SLC_I64,
}

# Every exported symbol with its ctypes signature.  The tests check that this
# table and include/slc_hip.h list the same entry points.
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "slc_hip_version": (_I, []),
    "slc_hip_last_error": (ctypes.c_char_p, []),
    "slc_hip_set_timing_events": (None, [_P, _P]),
    "slc_hip_set_timing_repeats": (None, [ctypes.c_int]),
    "slc_hip_kv_store": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _L, _P],
    ),
    "slc_hip_embedding": (_I, [_P, _P, _P, _I, _L, _L, _L, _P, _P]),
    "slc_hip_add": (_I, [_P, _P, _P, _I, _L, _P]),
    "slc_hip_swiglu": (_I, [_P, _P, _P, _I, _L, _P]),
    "slc_hip_rope_table": (_I, [_P, _P, _P, _P, _I, _L, _L, _L, _L, _P]),
    "slc_hip_kv_advance": (_I, [_P, _P, _L, _L, _L, _P, _P]),
    "slc_hip_argmax_workspace_size": (_L, [_L]),
    "slc_hip_argmax": (_I, [_P, _P, _I, _L, _L, _L, _P, _L, _P, _L, _P]),
    "slc_hip_norm_linear_group": (
        _I,
        [_P, _L, _P, _F, _L, _L, _I] + [_P, _P, _P, _L, _L] * 3 + [_I, _P],
    ),
    "slc_hip_norm_linear_swiglu": (_I, [_P, _L, _P, _F, _L, _L, _L, _P, _P, _P, _L, _I, _P]),
    "slc_hip_linear_residual": (_I, [_P, _L, _L, _L, _L, _P, _P, _P, _L, _P, _L, _I, _P]),
    "slc_hip_rope_kv_store": (_I, [_P] * 11 + [_L, _I] + [_L] * 6 + [_L] * 16 + [_P, _L, _P]),
    "slc_hip_linear_group": (
        _I, [_P, _L, _L, _L, _I] + [_P, _P, _P, _L, _L] * 3 + [_I, _P]),
    "slc_hip_linear_swiglu": (_I, [_P, _L, _L, _L, _L, _P, _P, _P, _L, _I, _P]),
    "slc_hip_rope_decode_attention": (
        _I, [_P] * 11 + [_I, _P, _P, _L, _P, _L, _I] + [_L] * 6 + [_L] * 15 + [_F, _I, _P]),
    "slc_hip_decode_attention_workspace_size": (
        _L,
        [_L, _L, _L, _L, _L, _I, _L],
    ),
    "slc_hip_decode_attention": (
        _I,
        [_P, _P, _P, _P, _I, _P, _I, _P, _P, _L, _P, _L, _I]
        + [_L] * 15
        + [_F, _L, _I, _P],
    ),
    "slc_hip_decode_attention_noalloc": (
        _I,
        [_P, _P, _P, _P, _I, _P, _I, _P, _I] + [_L] * 15 + [_F, _L, _I, _P],
    ),
    "slc_hip_paged_decode_attention": (
        _I,
        [_P, _P, _P, _P, _L, _L, _L, _L, _P, _I, _P, _I, _P, _P, _L, _P, _L, _I]
        + [_L] * 13 + [_F, _L, _I, _P],
    ),
    "slc_hip_paged_rope_decode_attention": (
        _I,
        [_P] * 7 + [_P, _L, _L, _L, _L, _P, _P, _P, _P, _I, _P, _P, _L, _P, _L, _I]
        + [_L] * 4 + [_L] * 15 + [_F, _I, _P],
    ),
    "slc_hip_paged_kv_store": (
        _I,
        [_P, _P, _P, _L, _L, _L, _L, _L, _L, _P, _P, _P, _P, _I] + [_L] * 10 + [_P],
    ),
    "slc_hip_decode_attention_exact_max_tokens": (_L, [_L, _I]),
    "slc_hip_decode_attention_counter_count": (_L, [_L, _L]),
    "slc_hip_rms_norm": (
        _I,
        [_P, _P, _P, _I, _I, _I, _I, _L, _L, _L, _L, _F, _I, _I, _P],
    ),
    "slc_hip_linear": (
        _I,
        [_P, _P, _P, _P, _I, _L, _L, _L, _L, _L, _P],
    ),
    "slc_hip_linear_tile": (
        _I,
        [_P, _P, _P, _P, _I, _L, _L, _L, _L, _L, _I, _P],
    ),
    "slc_hip_prefill_attention_classes": (
        _I,
        [_P, _P, _P, _P, _I, _P, _P, _I, _L, _L, _L, _L, _L, _I] + [_L] * 15 + [_F, _I, _P],
    ),
    "slc_hip_prefill_mask_tile_count": (_L, [_L, _L]),
    "slc_hip_prefill_mask_tiles": (_I, [_P, _I, _L, _L, _L, _L, _L, _P, _P]),
    "slc_hip_prefill_attention": (
        _I,
        [_P, _P, _P, _P, _I, _P, _I, _L, _L, _L, _L, _L, _I] + [_L] * 15 + [_F, _I, _P],
    ),
    "slc_hip_rope": (
        _I,
        [_P] * 6 + [_I] + [_L] * 5 + [_L] * 16 + [_P],
    ),
}


class NativeLibraryError(RuntimeError):
    """The gfx950 kernel library is missing or could not be loaded."""


class KernelLaunchError(RuntimeError):
    """A C entry point rejected its arguments or a launch failed."""


_lock = threading.Lock()
_library: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """Load (once) and return the kernel library; raise if it is unavailable."""

    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is not None:
            return _library
        if not LIBRARY_PATH.exists():
            raise NativeLibraryError(
                f"{LIBRARY_PATH} does not exist; build it with "
                "`python llm-compiler_amd/stateful_llm_compiler_hip/build.py` "
                "(or __graft_entry__.build())"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH))
        except OSError as error:
            raise NativeLibraryError(
                f"cannot load {LIBRARY_PATH}: {error}"
            ) from error
        for name, (restype, argtypes) in SIGNATURES.items():
            function = getattr(lib, name)
            function.restype = restype
            function.argtypes = argtypes
        _library = lib
        return lib


def dtype_tag(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_TAGS[dtype]
    except KeyError as error:
        raise ValueError(f"unsupported dtype {dtype}") from error


def current_stream(device: torch.device) -> int:
    """Raw hipStream_t of PyTorch's current stream on ``device``."""

    return torch.cuda.current_stream(device).cuda_stream


def check(status: int, what: str) -> None:
    if status != 0:
        message = library().slc_hip_last_error().decode(errors="replace")
        raise KernelLaunchError(f"{what} failed (status {status}): {message}")


def softmax_order_tag(order: str) -> int:
    try:
        return SOFTMAX_ORDERS[order]
    except KeyError as error:
        raise ValueError(f"softmax order must be one of {sorted(SOFTMAX_ORDERS)}, got {order!r}") from error


class DeviceWorkspace:
    """Caller-owned device memory of the kernels that combine work across
    workgroups: one zero-filled int32 counter array, shared by every kernel
    kind (each kernel leaves its counters zero again), and scratch buffers
    per kernel kind for partial results.  Kernels that run in order (one
    stream, or one captured graph) can share a workspace; kernels that may run
    concurrently need separate ones.  Buffers that were outgrown stay alive (a
    captured graph may still hold their address)."""

    def __init__(self, device: torch.device | str) -> None:
        self.device = torch.device(device)
        self._counters: torch.Tensor | None = None
        self._scratch: dict[str, torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []

    def counters(self, count: int) -> torch.Tensor:
        """Zeroed int32 counters, at least ``count`` (and at least 1) of them."""

        current = self._counters
        if current is None or current.numel() < count:
            if current is not None:
                self._retired.append(current)
            size = max(int(count), 2 * (current.numel() if current is not None else 0), 64)
            self._counters = torch.zeros(size, dtype=torch.int32, device=self.device)
        return self._counters

    def scratch(self, name: str, nbytes: int) -> torch.Tensor | None:
        """Scratch bytes of a kernel kind (no initial contents), or None."""

        if nbytes <= 0:
            return None
        buffer = self._scratch.get(name)
        if buffer is None or buffer.numel() < nbytes:
            if buffer is not None:
                self._retired.append(buffer)
            size = max(int(nbytes), 2 * (buffer.numel() if buffer is not None else 0))
            buffer = torch.empty(size, dtype=torch.uint8, device=self.device)
            self._scratch[name] = buffer
        return buffer


# Workspaces of raw stream handles, least recently used first.  A server that
# keeps creating streams would otherwise grow this without bound; past
# MAX_STREAM_WORKSPACES the least recently used entry is dropped (its memory
# returns to PyTorch's caching allocator, which reuses it in stream order).
# A graph captured on a stream without an explicit workspace keeps using that
# stream's workspace: callers that capture on more streams than the bound at
# once pass their own DeviceWorkspace instead.
MAX_STREAM_WORKSPACES = 64
_stream_workspaces: "OrderedDict[tuple[int, int], DeviceWorkspace]" = OrderedDict()


def stream_workspace(device: torch.device) -> DeviceWorkspace:
    """The workspace of PyTorch's current stream on ``device``, for callers
    that do not own one (calls on one stream never overlap)."""

    stream = current_stream(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, stream)
    with _lock:
        workspace = _stream_workspaces.get(key)
        if workspace is None:
            workspace = DeviceWorkspace(torch.device("cuda", index))
            _stream_workspaces[key] = workspace
            while len(_stream_workspaces) > MAX_STREAM_WORKSPACES:
                _stream_workspaces.popitem(last=False)
        else:
            _stream_workspaces.move_to_end(key)
    return workspace
