"""ctypes binding of libflicker_hip.so (the C ABI declared in include/flicker_hip.h).

The library is the only compute path of this package: if it has not been built the
first call raises ``HipLibraryMissing`` -- there is no CPU or PyTorch fallback.
"""

from __future__ import annotations

import ctypes
import functools
import pathlib

import torch

LIB_PATH = pathlib.Path(__file__).resolve().with_name("libflicker_hip.so")

_p, _i, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
_ip = ctypes.POINTER(ctypes.c_int)

# name -> (restype, argtypes); one entry per function of include/flicker_hip.h
SIGNATURES = {
    "flk_abi_version": (_i, []),
    "flk_status_string": (ctypes.c_char_p, [_i]),
    "flk_qk_prep": (_i, [_p, _i64, _i64, _p, _p, _i64, _p, _p, _i, _f, _i, _i, _i, _i,
                         _p, _p, _p, _i64, _i64, _p]),
    "flk_qk_prep_f32": (_i, [_p, _i64, _i64, _p, _p, _i64, _p, _p, _i, _i, _i, _i, _p, _p, _p, _i64, _i64, _p]),
    "flk_qk_prep_ids": (_i, [_p, _i64, _i64, _p, _i64, _i, _ip, _f, _p, _p, _i, _f, _i, _i, _i, _i,
                             _p, _p, _p, _i64, _i64, _p]),
    "flk_attend": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "flk_attend_to": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i64, _i64, _i64, _p]),
    "flk_attend_split_to": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i64, _i64, _i64, _i, _p, _i64, _p]),
    "flk_attend_split_static_to": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i64, _i64, _i64, _i, _p]),
    "flk_attend_balanced_to": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i64, _i64, _i64, _p, _i64, _p]),
    "flk_attend_balanced_plan": (_i, [_i, _i, _i, _ip, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]),
    "flk_attend_plan": (_i, [_i, _i, _i, _ip, ctypes.POINTER(ctypes.c_int64)]),
    "flk_attend_kernel": (ctypes.c_char_p, [_i, _i, _i]),
    "flk_rope_embed": (_i, [_p, _i64, _i64, _i, _ip, _f, _p, _p]),
    "flk_lane_pair": (_i, [_p, _i64, _i, _p, _p, _p]),
    "flk_rope_lanes": (_i, [_p, _i64, _i64, _i, _ip, _f, _p, _p, _p]),
    "flk_absmax_rows": (_i, [_p, _i64, _i64, _i64, _p, _p]),
    "flk_absmax_cols": (_i, [_p, _i64, _i64, _i64, _i, _p, _p]),
    "flk_smooth_factors": (_i, [_p, _p, _i64, _p, _p, _p]),
    "flk_quantize_weight": (_i, [_p, _i64, _p, _i, _i, _p, _p, _p]),
    "flk_quantize_act": (_i, [_p, _i64, _p, _i, _i, _p, _p, _p]),
    "flk_quantize_act_modulated": (_i, [_p, _i64, _p, _p, _i64, _i, _p, _i, _i, _p, _p, _p, _i64, _p]),
    "flk_quantize_act_modulated_pair": (_i, [_p, _i64, _p, _p, _i64, _i, _p, _i, _p, _p, _p, _i64,
                                             _p, _i64, _p, _p, _i64, _i, _p, _i, _p, _p, _p, _i64, _i, _p]),
    "flk_w8a8_gemm": (_i, [_p, _p, _p, _p, _i, _i, _i, _p, _i64, _p, _p]),
    "flk_w8a8_qk_prep": (_i, [_p, _p, _p, _p, _i, _p, _p, _i64, _p, _p, _i, _f, _i, _i, _i, _i,
                              _p, _p, _p, _i64, _i64, _p]),
    "flk_w8a8_qk_prep_pair": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i64,
                                   _p, _p, _p, _p, _p, _p, _p, _p, _i, _i64,
                                   _i, _i64, _i, _f, _i, _i, _i, _p, _p, _p, _i64, _p]),
}

ABI_VERSION = 1
FLK_OK, FLK_E_INVALID, FLK_E_ALIGN, FLK_E_UNSUPPORTED, FLK_E_SCRATCH = 0, -1, -2, -3, -4
ATTEND_STATIC_SCRATCH_BYTES = 34078720   # FLK_ATTEND_STATIC_SCRATCH_BYTES


class HipLibraryMissing(RuntimeError):
    """libflicker_hip.so is not built (run ``python -m flicker_amd.build``)."""


class HipKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


_LIB = None


def lib() -> ctypes.CDLL:
    """Load the library once and attach the argument types of every entry point."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise HipLibraryMissing(
                f"{LIB_PATH} is missing: build it with `python -m flicker_amd.build` "
                "(flicker_amd has no fallback compute path)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = handle.flk_abi_version()
        if version != ABI_VERSION:
            raise HipLibraryMissing(f"{LIB_PATH} has ABI {version}, expected {ABI_VERSION}; rebuild it")
        _LIB = handle
    return _LIB


def status_string(status: int) -> str:
    return lib().flk_status_string(status).decode()


def check(status: int, what: str) -> None:
    if status != FLK_OK:
        raise HipKernelError(f"{what} failed with status {status}: {status_string(status)}")


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on the tensor's device (the integer handle,
    without building a torch Stream object per call)."""
    return torch._C._cuda_getCurrentRawStream(t.device.index)


def device_of(*tensors) -> torch.device:
    """The one GPU that every given tensor (None entries skipped) lives on."""
    devices = {t.device for t in tensors if t is not None}
    if len(devices) != 1:
        raise ValueError(f"the operands of one call must share one GPU, got {sorted(map(str, devices))}")
    device = devices.pop()
    if device.type != "cuda":
        raise ValueError(f"operands are on {device}; flicker_amd runs its kernels on the GPU only")
    return device


def run(name: str, tensors, *args) -> None:
    """Call entry point ``name`` with the tensors' GPU current -- a HIP launch goes to the
    current device, whatever device the tensors live on -- and raise on a non-zero status."""
    device = device_of(*tensors)
    fn = getattr(lib(), name)
    if torch.cuda.current_device() == device.index:
        check(fn(*args), name)
        return
    with torch.cuda.device(device):
        check(fn(*args), name)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


@functools.lru_cache(maxsize=1024)
def attend_plan(batch: int, heads: int, length: int) -> tuple[int, int]:
    """(splits, workspace bytes) that flk_attend_plan picks for an attend of this shape (a
    pure function of the shape, so cached)."""
    splits, nbytes = ctypes.c_int(0), ctypes.c_int64(0)
    check(lib().flk_attend_plan(batch, heads, length, ctypes.byref(splits), ctypes.byref(nbytes)),
          "flk_attend_plan")
    return splits.value, nbytes.value


@functools.lru_cache(maxsize=1024)
def attend_kernel_name(batch: int, heads: int, length: int) -> str:
    """Name of the kernel flk_attend / flk_attend_to launch for this shape."""
    return lib().flk_attend_kernel(batch, heads, length).decode()


@functools.lru_cache(maxsize=1024)
def attend_balanced_plan(batch: int, heads: int, length: int) -> tuple[int, int, int]:
    """(grid, workspace bytes, counters offset) of flk_attend_balanced_to for a shape; grid 0
    when the shape has fewer 256-query tiles than CUs (a pure function of the shape)."""
    grid, nbytes, off = ctypes.c_int(0), ctypes.c_int64(0), ctypes.c_int64(0)
    check(lib().flk_attend_balanced_plan(batch, heads, length, ctypes.byref(grid), ctypes.byref(nbytes),
                                         ctypes.byref(off)), "flk_attend_balanced_plan")
    return grid.value, nbytes.value, off.value


_BALANCED_WORKSPACE: dict = {}


def balanced_workspace(device: torch.device, stream: int, nbytes: int, counters_offset: int) -> torch.Tensor:
    """The balanced attend's workspace for one (device, stream): allocated zeroed on first use
    and kept, since its hand-off counters carry each call's epoch and need no reset.  One per
    stream, so that calls on different streams never share one.  Under graph capture a fresh
    workspace is taken from the capture's pool and its counters are zeroed by a captured fill
    (a fill kernel, not a memset node), so no garbage in the pool can pass for a live count."""
    if torch.cuda.is_current_stream_capturing():
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        ws[counters_offset:].zero_()
        return ws
    key = (device.index, stream)
    ws = _BALANCED_WORKSPACE.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _BALANCED_WORKSPACE[key] = ws
    return ws


def int_array(values) -> ctypes.Array:
    values = [int(v) for v in values]
    return (ctypes.c_int * len(values))(*values)
