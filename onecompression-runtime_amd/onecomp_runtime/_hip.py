"""ctypes binding of ``libonecomp_hip.so``, the C ABI declared in
``include/onecomp_hip.h``.

Every device entry point takes raw device pointers, element counts and the
caller's current HIP stream; this module only converts torch tensors to those
arguments and maps status codes to the exception types the reference raises
(``ValueError`` for bad shapes/arguments, ``NotImplementedError`` for valid but
unimplemented layouts, ``RuntimeError`` for runtime failures).

There is no fallback: if the library is missing, or a tensor is not on a HIP
device, the call raises.
"""
from __future__ import annotations

import ctypes
import functools
import os
import threading
from pathlib import Path

import torch

OC_OK = 0
OC_ERR_INVALID_ARGUMENT = 1
OC_ERR_SHAPE = 2
OC_ERR_UNSUPPORTED = 3
OC_ERR_WORKSPACE = 4
OC_ERR_HIP = 5

OC_DTYPE_F16 = 1
OC_DTYPE_BF16 = 2
OC_DTYPE_F32 = 3
OC_DTYPE_U8 = 4
OC_DTYPE_I32 = 5

OC_ZERO_V1 = 1
OC_ZERO_V2 = 2

OC_REGIME_AUTO = 0
OC_REGIME_SPLITK = 1
OC_REGIME_TILED = 2
OC_REGIME_DOT = 3

LIB_PATH = Path(
    os.environ.get("ONECOMP_HIP_LIB", Path(__file__).resolve().parent / "_lib" / "libonecomp_hip.so")
)

_DTYPE_CODES = {
    torch.float16: OC_DTYPE_F16,
    torch.bfloat16: OC_DTYPE_BF16,
    torch.float32: OC_DTYPE_F32,
    torch.uint8: OC_DTYPE_U8,
    torch.int32: OC_DTYPE_I32,
}

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); must match include/onecomp_hip.h.
SIGNATURES = {
    "oc_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "oc_last_error": (ctypes.c_char_p, []),
    "oc_version": (ctypes.c_int, []),
    "oc_int4_plan_groups": (
        ctypes.c_int,
        [_P, _I32, _I32, _P, _I64, _P, _P, _P, _P],
    ),
    "oc_int4_prepare": (
        ctypes.c_int,
        [_P, _I32, _I32, _P, _I32, _I32, _P, _I32, _P, _I32, _P, _P, _P, _P],
    ),
    "oc_int4_export": (
        ctypes.c_int,
        [_P, _P, _P, _I32, _I32, _I32, _P, _I32, _I32, _I32, _P, _P, _P, _P],
    ),
    "oc_int8_prepare": (
        ctypes.c_int,
        [_P, _I32, _I32, _P, _I32, _I32, _P, _I32, _P, _I32, _P, _P, _P, _P],
    ),
    "oc_int8_gemm": (
        ctypes.c_int,
        [_P, _I64, _I32, _I32, _I32, _P, _P, _I32, _P, _I32, _I32, _I32, _P, _P, _P, _I32,
         _P, _I64, _P, _SZ, _P],
    ),
    "oc_int8_gemm_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I32]),
    "oc_int8_export": (
        ctypes.c_int,
        [_P, _P, _P, _I32, _I32, _I32, _P, _I32, _I32, _I32, _P, _P, _P, _P],
    ),
    "oc_int8_dequant_tiled": (
        ctypes.c_int,
        [_P, _P, _I32, _P, _P, _I32, _I32, _I32, _I32, _P, _I32, _P],
    ),
    "oc_int4_dequant_tiled": (
        ctypes.c_int,
        [_P, _P, _I32, _P, _P, _I32, _I32, _I32, _I32, _P, _I32, _P],
    ),
    "oc_unpack_rows": (ctypes.c_int, [_P, _I32, _I32, _I32, _I32, _P, _P]),
    "oc_int4_dequant": (
        ctypes.c_int,
        [_P, _P, _I32, _P, _I32, _P, _I32, _I32, _I32, _I32, _P, _I32, _P],
    ),
    "oc_int4_gemm": (
        ctypes.c_int,
        [_P, _I64, _I32, _I32, _I32, _P, _P, _I32, _P, _I32, _I32, _I32, _P, _P, _P, _I32,
         _P, _I64, _P, _SZ, _I32, _P],
    ),
    "oc_int4_gemm_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "oc_int4_gemm_noalloc": (
        ctypes.c_int,
        [_P, _I64, _I32, _I32, _I32, _P, _P, _I32, _P, _I32, _I32, _I32, _P, _P, _P, _I32,
         _P, _I64, _I32, _P],
    ),
    "oc_int4_gemm_noalloc_scratch_bytes": (_SZ, []),
    "oc_rtn_dequant": (
        ctypes.c_int,
        [_P, _I32, _I32, _P, _I32, _P, _I32, _I32, _I32, _P, _I32, _P],
    ),
    "oc_rtn_linear": (
        ctypes.c_int,
        [_P, _I64, _I32, _I32, _I32, _P, _I32, _P, _I32, _P, _I32, _I32, _I32, _P, _I32, _P,
         _I64, _P],
    ),
    "oc_rtn_embedding": (
        ctypes.c_int,
        [_P, _I64, _P, _I64, _I32, _P, _I32, _P, _I32, _I32, _I32, _P, _I32, _P, _P],
    ),
    "oc_dsv4_dequant": (
        ctypes.c_int,
        [_P, _I32, _I32, _I32, _I32, _P, _I32, _P, _I32, _I32, _I64, _I64, _P, _I32, _P],
    ),
    "oc_dsv4_gemm": (
        ctypes.c_int,
        [_P, _I64, _I32, _I32, _I32, _P, _I32, _I32, _P, _I32, _P, _I32, _I32, _I64, _I64, _I32,
         _P, _I32, _P, _I64, _P, _SZ, _P],
    ),
    "oc_dsv4_gemm_workspace_bytes": (_SZ, [_I32, _I32, _I32]),
    "oc_rtn_conv1d": (
        ctypes.c_int,
        [_P, _I32, _I32, _I32, _I32, _P, _I32, _P, _I32, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
         _I32, _P, _I32, _P, _P, _SZ, _P],
    ),
    "oc_rtn_conv1d_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I32]),
    "oc_rtn_tile_prepare": (ctypes.c_int, [_P, _I32, _I32, _I32, _P, _P, _I32, _I32, _P, _P, _P, _P]),
    "oc_rtn_conv1d_prepared": (
        ctypes.c_int,
        [_P, _I32, _I32, _I32, _I32, _P, _I32, _P, _I32, _P, _I32, _I32, _P, _P, _I32, _I32, _I32, _I32, _I32,
         _I32, _I32, _P, _I32, _P, _P, _SZ, _P],
    ),
    "oc_rtn_transpose_prepare": (ctypes.c_int, [_P, _I32, _I32, _I32, _P, _P, _I32, _P, _P, _P, _P]),
    "oc_rtn_tile_prepare_t": (ctypes.c_int, [_P, _I32, _I32, _I32, _P, _P, _I32, _I32, _I32, _P, _P, _P, _P]),
    "oc_rtn_conv_transpose1d_prepared": (
        ctypes.c_int,
        [_P, _I32, _I32, _I32, _I32, _P, _P, _P, _I32, _I32, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
         _P, _I32, _P, _P, _SZ, _P],
    ),
    "oc_rtn_conv_transpose1d": (
        ctypes.c_int,
        [_P, _I32, _I32, _I32, _I32, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
         _P, _I32, _P, _P, _SZ, _P],
    ),
    "oc_rtn_conv_transpose1d_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "oc_moe_route": (ctypes.c_int, [_P, _I32, _I32, _I32, _P, _P, _P]),
    "oc_int4_moe_gemm": (
        ctypes.c_int,
        [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _I32, _P, _I32, _I32, _I32, _P, _P,
         _P, _I64, _P],
    ),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load the shared library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"onecomp_runtime HIP library not found at {LIB_PATH}; build it with "
                    "`make -C onecompression-runtime_amd` (hipcc, gfx950)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def last_error() -> str:
    return lib().oc_last_error().decode()


def check(status: int, what: str) -> None:
    """Map a C status code to the reference's exception types."""
    if status == OC_OK:
        return
    msg = f"{what}: {lib().oc_status_string(status).decode()}: {last_error()}"
    if status in (OC_ERR_INVALID_ARGUMENT, OC_ERR_SHAPE):
        raise ValueError(msg)
    if status == OC_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def require_device(*tensors: torch.Tensor | None) -> torch.device:
    """All given tensors must live on one HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "onecomp_runtime HIP kernels need tensors on a HIP device "
                f"(got a tensor on {t.device}); there is no CPU fallback"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor given")
    return dev


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = torch._C._cuda_getCurrentRawStream


def stream_of(device: torch.device | int) -> int:
    """Raw handle of torch's current HIP stream on ``device``."""
    idx = device if isinstance(device, int) else (
        device.index if device.index is not None else torch.cuda.current_device())
    return _raw_stream(idx)


class _Workspace:
    """Scratch of the GEMM calls (counter area, gathered activations, split-K
    partials), one buffer per (device, stream).

    Calls on one stream run in order, so they can share a buffer (each call
    overwrites what it reads and leaves the counter area zero); calls on
    different streams may overlap in time, so every stream gets its own.
    A graph captured on a stream keeps that stream's buffer address: graphs
    replayed concurrently must be captured on distinct streams. Buffers grow
    on demand; outgrown ones stay allocated, since a captured graph may still
    hold their address. The first call on a stream allocates, so run each
    layer once on the capture stream (or eagerly on it) before a capture if
    the capture must not allocate.
    """

    def __init__(self) -> None:
        self._bufs: dict[tuple[int, int], torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []

    def get(self, device: torch.device | int, nbytes: int, stream: int | None = None) -> torch.Tensor | None:
        if nbytes == 0:
            return None
        idx = device if isinstance(device, int) else (
            device.index if device.index is not None else torch.cuda.current_device())
        key = (idx, _raw_stream(idx) if stream is None else stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                self._retired.append(buf)
            # zero-filled: the counter area must start at zero
            buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=torch.device("cuda", idx))
            self._bufs[key] = buf
        return buf


workspace = _Workspace()


@functools.lru_cache(maxsize=4096)
def gemm_workspace_bytes(M: int, N: int, K_phys: int, group_rows: int, has_kmap: bool, regime: int) -> int:
    return int(lib().oc_int4_gemm_workspace_bytes(M, N, K_phys, group_rows, int(has_kmap), regime))


def gemm_workspace(device: torch.device | int, M: int, N: int, K_phys: int, group_rows: int,
                   has_kmap: bool, regime: int, stream: int | None = None, wbits: int = 4):
    if wbits == 8:
        nbytes = gemm8_workspace_bytes(M, N, K_phys, group_rows, has_kmap)
    else:
        nbytes = gemm_workspace_bytes(M, N, K_phys, group_rows, has_kmap, regime)
    return workspace.get(device, nbytes, stream), nbytes


@functools.lru_cache(maxsize=4096)
def gemm8_workspace_bytes(M: int, N: int, K_phys: int, group_rows: int, has_kmap: bool) -> int:
    return int(lib().oc_int8_gemm_workspace_bytes(M, N, K_phys, group_rows, int(has_kmap)))
