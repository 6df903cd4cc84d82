"""ctypes binding of ``libtilemaxsim.so`` (the C ABI declared in ``include/tilemaxsim.h``).

The library is loaded lazily on first use and is REQUIRED: there is no CPU or
PyTorch fallback, so a missing or unloadable library raises immediately.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtilemaxsim.so")

TMS_OK = 0
TMS_ERR_INVALID = 1
TMS_ERR_UNSUPPORTED = 2
TMS_ERR_HIP = 3

TMS_DTYPE_F16 = 0
TMS_DTYPE_BF16 = 1
TMS_DTYPE_F32 = 2
TMS_QUERY_F32 = 0x100  # OR-ed into a 16-bit dtype: Q is fp32 (split into two 16-bit terms, not rounded)
TMS_CODES_I16 = 0x200  # OR-ed into a PQ dtype: int16 codes
TMS_CODES_I32 = 0x400  # OR-ed into a PQ dtype: int32 codes
TMS_READ_PROBE_SINK_WORDS = 524288  # words of the sink tms_read_probe writes
TMS_LDS_PROBE_WAVES = 4096  # waves of one tms_lds_probe launch (one cycle count each)
TMS_MAXSIM_TOPK_COUNTER_WORDS = 144  # 32-bit words of tms_maxsim_topk's zeroed ticket block
TMS_MFMA_PROBE_SINK_WORDS = 131072  # words of the sink tms_mfma_probe writes

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int

# name -> argtypes (restype is int for every entry point except tms_last_error)
SIGNATURES = {
    "tms_version": [],
    "tms_set_rerank_limit": [_i64],
    "tms_maxsim_dense": [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _int, _c_void_p, _c_void_p],
    "tms_maxsim_masked": [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64, _i64, _int, _c_void_p, _c_void_p],
    "tms_maxsim_varlen": [_c_void_p, _i64, _i64, _c_void_p, _i64, _c_void_p, _i64, _int, _c_void_p, _c_void_p],
    "tms_maxsim_varlen_padded": [_c_void_p, _i64, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _int, _c_void_p,
                                 _c_void_p],
    "tms_maxsim_dense_batched": [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i64, _int, _c_void_p, _c_void_p],
    "tms_pq_build_lut": [_c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _int, _c_void_p, _c_void_p],
    "tms_pq_score_lut": [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p],
    "tms_pq_score_lut_ex": [_c_void_p, _i64, _i64, _i64, _c_void_p, _int, _i64, _i64, _c_void_p, _c_void_p],
    "tms_pq_score": [_c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _int, _c_void_p, _i64, _i64, _c_void_p, _c_void_p],
    "tms_topk": [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p],
    "tms_topk_workspace_size": [_i64, _i64, _i64],
    "tms_topk_noalloc": [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p],
    "tms_maxsim_topk": [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _int, _i64, _c_void_p, _c_void_p, _c_void_p,
                        _c_void_p, _c_void_p],
    "tms_read_probe": [_c_void_p, _i64, _c_void_p, _i64, _c_void_p],
    "tms_lds_probe": [_int, _c_void_p, _i64, _c_void_p, _i64, _c_void_p],
    "tms_mfma_probe": [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p],
    "tms_residual_decompress": [_c_void_p, _c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p, _int, _c_void_p,
                                _c_void_p],
    "tms_maxsim_residual": [_c_void_p, _i64, _i64, _c_void_p, _i64, _c_void_p, _int, _c_void_p, _c_void_p, _i64,
                            _c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p],
    "tms_maxsim_varlen_batched": [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _int,
                                  _c_void_p, _c_void_p],
    "tms_pq_score_batched": [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _i64, _int, _c_void_p, _i64, _i64,
                             _c_void_p, _c_void_p],
    "tms_maxsim_residual_batched": [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _c_void_p, _int, _c_void_p,
                                    _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p],
}
RESTYPES = {"tms_topk_workspace_size": ctypes.c_int64, "tms_set_rerank_limit": ctypes.c_int64}

_lib = None
_lock = threading.Lock()


class TileMaxSimError(RuntimeError):
    """The HIP runtime reported an error inside the library."""


def load() -> ctypes.CDLL:
    """Load the shared library (once). Raises ImportError if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m tilemaxsim_amd.build` "
                "(tilemaxsim_amd has no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue  # calling it raises AttributeError
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        lib.tms_last_error.argtypes = []
        lib.tms_last_error.restype = ctypes.c_char_p
        _lib = lib
    return _lib


@contextlib.contextmanager
def rerank_limit(tiles: int):
    """Within the block, dense calls whose documents span at most ``tiles`` 16-token tiles
    take the small-batch kernel (0: none do; ``tms_set_rerank_limit``). Process-wide."""
    lib = load()
    prev = lib.tms_set_rerank_limit(int(tiles))
    try:
        yield prev
    finally:
        lib.tms_set_rerank_limit(prev)


def check(status: int) -> None:
    """Turn a non-zero C status into the matching Python exception."""
    if status == TMS_OK:
        return
    msg = load().tms_last_error().decode(errors="replace")
    if status == TMS_ERR_INVALID:
        raise ValueError(msg)
    if status == TMS_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise TileMaxSimError(msg)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float16:
        return TMS_DTYPE_F16
    if dt == torch.bfloat16:
        return TMS_DTYPE_BF16
    if dt == torch.float32:
        return TMS_DTYPE_F32
    raise TypeError(f"tilemaxsim_amd kernels take float16, bfloat16 or float32 embeddings, got {dt}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on the tensor's device (through torch's raw
    stream query where this torch has it: a fraction of a microsecond against about 2 us
    for building a Stream object)."""
    if _raw_stream is not None:
        idx = t.device.index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(t.device).cuda_stream


class _Current:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


_CURRENT = _Current()


def on_device(dev: torch.device):
    """``torch.cuda.device(dev)``, or a no-op context when ``dev`` is already current."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return _CURRENT
    return torch.cuda.device(dev)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
