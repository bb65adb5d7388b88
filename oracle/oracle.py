"""CPU oracle for the chunked linear-recurrence scan -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or the timed CPU baseline).
The product package never imports it.

Two independent restatements of the reference's algorithm:

* ``liboracle.so`` (scan_oracle.c): sequential fp64 loops per segment,
  compiled with -ffp-contract=off.  Functions ``scan_fwd``, ``scan_bwd``,
  ``shift_pad`` below call it.
* pure numpy (``np_scan_fwd``, ``np_scan_bwd``, ``np_shift_pad``):
  vectorised over channels, sequential over time, also one rounding per
  operation -- the exact method of the reference's gold label
  (tests/test_scan_dtypes.py:26-38).

Both follow these reference lines: _kernels.py:6-16 (combine op),
:54-81 and :115-168 (masking, reverse indexing, gate product),
:226-287 (backward shifts, pads and d_gates), _shift_pad.py:18-55 and
:140-165 (shift_pad), tests/test_scan_kernels.py:873-918 (hand-derived
backward).  How each function is pinned (golden vectors, closed forms,
brute-force autograd) is listed in tests/test_oracle.py.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
  """Compiles liboracle.so with the committed Makefile."""
  import subprocess
  subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
  return LIB_PATH


def _load():
  global _lib
  if _lib is None:
    if not LIB_PATH.exists():
      build()
    lib = ctypes.CDLL(str(LIB_PATH))
    P, L, I, D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
    lib.oracle_scan_fwd.argtypes = [P, P, P, P, P, L, L, L, I]
    lib.oracle_scan_bwd.argtypes = [P, P, P, P, P, P, L, L, L, I]
    lib.oracle_shift_pad.argtypes = [P, P, P, L, L, L, D, I, I]
    lib.oracle_fwd_bwd_f32io.argtypes = [P, P, P, P, P, P, P, L, L, L, I]
    lib.oracle_max_threads.argtypes = []
    for f in ("oracle_scan_fwd", "oracle_scan_bwd", "oracle_shift_pad",
              "oracle_fwd_bwd_f32io", "oracle_max_threads"):
      getattr(lib, f).restype = ctypes.c_int
    _lib = lib
  return _lib


def _f64(a) -> np.ndarray:
  return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def _cu(cu) -> np.ndarray:
  return np.ascontiguousarray(np.asarray(cu, dtype=np.int64))


def _ptr(a: np.ndarray | None):
  return None if a is None else a.ctypes.data


def _rows(shape, C):
  """(C, T) of an array of `shape` holding C flat rows."""
  n = int(np.prod(shape))
  C = int(C if C is not None else (shape[0] if len(shape) == 2 else 1))
  assert n % C == 0, (shape, C)
  return C, n // C


# ---------------------------------------------------------------------------
# C oracle
# ---------------------------------------------------------------------------

def scan_fwd(g, x, cu, reverse=False, channels=None, gate_prod=False):
  """fp64 sequential forward scan.  Returns h (and A if gate_prod)."""
  g, x, cu = _f64(g), _f64(x), _cu(cu)
  C, T = _rows(x.shape, channels)
  h = np.zeros_like(x)
  a = np.zeros_like(x) if gate_prod else None
  st = _load().oracle_scan_fwd(_ptr(g), _ptr(x), _ptr(h), _ptr(a), _ptr(cu),
                               len(cu) - 1, C, T, int(reverse))
  if st:
    raise ValueError("malformed cu_seqlens for the oracle")
  return (h, a) if gate_prod else h


def scan_bwd(dy, g, h, cu, causal=True, channels=None):
  """fp64 backward; returns (dx, dg) = (d_tokens, d_gates)."""
  dy, g, h, cu = _f64(dy), _f64(g), _f64(h), _cu(cu)
  C, T = _rows(dy.shape, channels)
  dx = np.zeros_like(dy)
  dg = np.zeros_like(dy)
  st = _load().oracle_scan_bwd(_ptr(dy), _ptr(g), _ptr(h), _ptr(dx), _ptr(dg),
                               _ptr(cu), len(cu) - 1, C, T, int(causal))
  if st:
    raise ValueError("malformed cu_seqlens for the oracle")
  return dx, dg


def shift_pad(data, cu, pad, backward=True, wrap=True):
  data, cu = _f64(data), _cu(cu)
  assert data.ndim == 2
  C, L = data.shape
  out = np.zeros_like(data)
  st = _load().oracle_shift_pad(_ptr(data), _ptr(out), _ptr(cu), len(cu) - 1,
                                C, L, float(pad), int(backward), int(wrap))
  if st:
    raise ValueError("boundary position out of range")
  return out


def fwd_bwd_f32io(g, x, dy, cu, channels, threads=1, out=None):
  """CPU baseline: fp32 storage, fp64 accumulation; returns (h, dx, dg).

  `out` may pass preallocated (h, dx, dg) float32 arrays of x's shape.
  """
  g = np.ascontiguousarray(g, dtype=np.float32)
  x = np.ascontiguousarray(x, dtype=np.float32)
  dy = np.ascontiguousarray(dy, dtype=np.float32)
  cu = _cu(cu)
  C, T = _rows(x.shape, channels)
  if out is None:
    h, dx, dg = np.empty_like(x), np.empty_like(x), np.empty_like(x)
  else:
    h, dx, dg = out
    for a in out:
      assert a.dtype == np.float32 and a.shape == x.shape and a.flags.c_contiguous
  st = _load().oracle_fwd_bwd_f32io(
    _ptr(g), _ptr(x), _ptr(dy), _ptr(h), _ptr(dx), _ptr(dg), _ptr(cu),
    len(cu) - 1, C, T, int(threads))
  if st:
    raise ValueError("malformed cu_seqlens for the oracle")
  return h, dx, dg


def max_threads() -> int:
  return int(_load().oracle_max_threads())


# ---------------------------------------------------------------------------
# numpy oracle (independent second restatement)
# ---------------------------------------------------------------------------

def np_scan_fwd(g, x, cu, reverse=False, channels=None):
  g, x, cu = _f64(g), _f64(x), _cu(cu)
  C, T = _rows(x.shape, channels)
  g2, x2 = g.reshape(C, T), x.reshape(C, T)
  h = np.zeros((C, T))
  for s in range(len(cu) - 1):
    b, e = int(cu[s]), int(cu[s + 1])
    if e <= b:
      continue
    ts = range(b, e) if not reverse else range(e - 1, b - 1, -1)
    prev = None
    for t in ts:
      h[:, t] = x2[:, t] if prev is None else g2[:, t] * h[:, prev] + x2[:, t]
      prev = t
  return h.reshape(x.shape)


def np_scan_bwd(dy, g, h, cu, causal=True, channels=None):
  dy, g, h, cu = _f64(dy), _f64(g), _f64(h), _cu(cu)
  C, T = _rows(dy.shape, channels)
  dy2, g2, h2 = dy.reshape(C, T), g.reshape(C, T), h.reshape(C, T)
  dx = np.zeros((C, T))
  dg = np.zeros((C, T))
  for s in range(len(cu) - 1):
    b, e = int(cu[s]), int(cu[s + 1])
    if e <= b:
      continue
    ts = range(e - 1, b - 1, -1) if causal else range(b, e)
    prev = None
    for t in ts:
      dx[:, t] = dy2[:, t] if prev is None else dy2[:, t] + dx[:, prev] * g2[:, prev]
      nb = t - 1 if causal else t + 1
      edge = (t == b) if causal else (t == e - 1)
      dg[:, t] = (0.0 if edge else h2[:, nb]) * dx[:, t]
      prev = t
  return dx.reshape(dy.shape), dg.reshape(dy.shape)


def np_shift_pad(data, cu, pad, backward=True, wrap=True):
  data, cu = _f64(data), _cu(cu)
  C, L = data.shape
  if wrap:
    out = np.roll(data, 1 if backward else -1, axis=-1)
  else:
    idx = np.arange(L) + (-1 if backward else 1)
    out = data[:, np.clip(idx, 0, L - 1)]
  mask = np.zeros(L, dtype=bool)
  pos = cu[:-1] if backward else cu[1:] - 1
  mask[pos] = True
  out = out.copy()
  out[:, mask] = pad
  return out


# ---------------------------------------------------------------------------
# the reference's own CPU method, in torch (timed as a CPU baseline)
# ---------------------------------------------------------------------------

def torch_fwd_bwd_f64(g, x, dy, cu):
  """Forward and backward in torch fp64, a loop over time vectorised over
  the channels: the forward is the reference's gold label
  (tests/test_scan_dtypes.py:26-38, bench/bench_accuracy.py:40-49), the
  backward its hand-derived reverse recurrence
  (tests/test_scan_kernels.py:873-897).  Takes and returns [C, T] torch
  tensors (h, dx, dg), per segment of cu."""
  import torch
  g = torch.as_tensor(g).to(torch.float64)
  x = torch.as_tensor(x).to(torch.float64)
  dy = torch.as_tensor(dy).to(torch.float64)
  h = torch.zeros_like(x)
  dx = torch.zeros_like(x)
  dg = torch.zeros_like(x)
  cu = [int(v) for v in cu]
  for s in range(len(cu) - 1):
    b, e = cu[s], cu[s + 1]
    if e <= b:
      continue
    h[:, b] = x[:, b]
    for t in range(b + 1, e):
      h[:, t] = g[:, t] * h[:, t - 1] + x[:, t]
    dx[:, e - 1] = dy[:, e - 1]
    for t in range(e - 2, b - 1, -1):
      dx[:, t] = dy[:, t] + dx[:, t + 1] * g[:, t + 1]
    dg[:, b + 1:e] = h[:, b:e - 1] * dx[:, b + 1:e]
  return h, dx, dg


def default_threads() -> int:
  return max(1, min(os.cpu_count() or 1, 16))
