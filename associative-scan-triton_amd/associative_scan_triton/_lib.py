"""ctypes binding of libassocscan (include/assocscan.h).

This is the only door from Python to the device code.  There is no
fallback: if the shared library is missing or a tensor is not on a HIP
device, the call raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

from associative_scan_triton._build import LIB_PATH

ASC_F32, ASC_F16, ASC_BF16 = 0, 1, 2
ASC_CU_I32, ASC_CU_I64 = 0, 1
ABI_VERSION = 6

_DTYPES = {
  torch.float32: ASC_F32,
  torch.float16: ASC_F16,
  torch.bfloat16: ASC_BF16,
}

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_D = ctypes.c_double

# name -> argtypes, mirroring include/assocscan.h
_U = ctypes.c_uint

SIGNATURES = {
  "asc_abi_version": [],
  "asc_scan_workspace_bytes": [_L, _L, _L, _I, _I],
  "asc_scan_workspace_walk": [_L, _L, _L, _I, _I],
  "asc_set_lookback_spin_limit": [_U],
  "asc_strerror": [_I],
  "asc_scan_fwd": [_P, _P, _P, _P, _P, _I, _L, _L, _L, _I, _I, _P, _L, _P],
  "asc_scan_fwd_noalloc": [_P, _P, _P, _P, _P, _I, _L, _L, _L, _I, _I, _P],
  "asc_scan_bwd": [_P, _P, _P, _P, _P, _P, _I, _L, _L, _L, _I, _I, _P, _L, _P],
  "asc_scan_checkpoint_elems": [_L, _L, _I],
  "asc_scan_checkpoints": [_P, _P, _P, _I, _L, _L, _L, _I, _I, _P],
  "asc_scan_bwd_recompute": [_P, _L, _P, _P, _P, _P, _P, _P, _I, _L, _L, _L, _I, _I, _P, _L, _P],
  "asc_scan_bwd_rowgrad": [_P, _L, _P, _P, _P, _P, _P, _I, _L, _L, _L, _I, _I, _P, _L, _P],
  "asc_scan_bidi_fwd": [_P, _P, _P, _P, _P, _P, _P, _I, _L, _L, _L, _I, _P, _L, _P],
  "asc_scan_bidi_bwd": [_P] * 11 + [_I, _L, _L, _L, _I, _P, _L, _P],
  "asc_scan_bidi_bwd_rowgrad": [_P, _L, _P, _L] + [_P] * 9 + [_I, _L, _L, _L, _I, _P, _L, _P],
  "asc_shift_pad": [_P, _P, _P, _I, _L, _L, _L, _I, _D, _I, _I, _P],
  "asc_shift_pad_strided": [_P, _L, _L, _P, _L, _L, _P, _I, _L, _L, _L, _I, _D, _I, _I, _P],
}
# walks a workspace buys (asc_scan_workspace_walk)
WALK_LOOKBACK = 1
WALK_CHAINED = 2

RESTYPES = {
  "asc_strerror": ctypes.c_char_p,
  "asc_scan_workspace_bytes": ctypes.c_int64,
  "asc_scan_checkpoint_elems": ctypes.c_int64,
  "asc_set_lookback_spin_limit": ctypes.c_uint,
}

_lib = None
_lock = threading.Lock()


class AscError(RuntimeError):
  """A libassocscan entry point returned a non-zero status."""


def load(path: Path | str | None = None) -> ctypes.CDLL:
  """Loads libassocscan once; raises if it has not been built."""
  global _lib
  if _lib is not None and path is None:
    return _lib
  with _lock:
    if _lib is not None and path is None:
      return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
      raise RuntimeError(
        f"{p} is missing: build it first "
        "(python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(str(p))
    for name, argtypes in SIGNATURES.items():
      fn = getattr(lib, name)
      fn.argtypes = argtypes
      fn.restype = RESTYPES.get(name, ctypes.c_int)
    if lib.asc_abi_version() != ABI_VERSION:
      raise RuntimeError(
        f"libassocscan ABI {lib.asc_abi_version()} != expected {ABI_VERSION}")
    if path is None:
      _lib = lib
    return lib


def check(status: int) -> None:
  if status != 0:
    msg = load().asc_strerror(status).decode()
    raise AscError(f"libassocscan error {status}: {msg}")


def dtype_code(t: torch.Tensor) -> int:
  try:
    return _DTYPES[t.dtype]
  except KeyError:
    raise TypeError(
      f"unsupported dtype {t.dtype}; expected float32, float16 or bfloat16"
    ) from None


def cu_code(cu: torch.Tensor) -> int:
  if cu.dtype == torch.int32:
    return ASC_CU_I32
  if cu.dtype == torch.int64:
    return ASC_CU_I64
  raise TypeError(f"cu_seqlens must be int32 or int64, got {cu.dtype}")


def require_device(*tensors: torch.Tensor) -> torch.device:
  """All tensors must live on the same HIP device; returns it."""
  dev = None
  for t in tensors:
    if t is None:
      continue
    if t.device.type != "cuda":
      raise ValueError(
        "associative_scan_triton runs on HIP devices only; got a tensor on "
        f"{t.device}")
    if dev is None:
      dev = t.device
    elif t.device != dev:
      raise ValueError(f"tensors on different devices: {dev} and {t.device}")
  return dev


def ptr(t: torch.Tensor | None) -> int | None:
  return None if t is None else t.data_ptr()


def stream_of(dev: torch.device) -> int:
  return torch.cuda.current_stream(dev).cuda_stream
