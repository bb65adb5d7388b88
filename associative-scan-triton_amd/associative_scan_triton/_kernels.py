"""The combine op and launchable kernel objects with the reference's call
convention.

The reference exposes its Triton kernels and callers launch them as
``kernel[grid](gates_ptr=..., ...)`` (tests and benches do, e.g.
test_scan_kernels.py:74-83, bench_kernels.py:89-136).  The objects below
accept the same subscript-then-call form and keyword names, and launch the
gfx950 kernels of libassocscan.  Grid layouts follow the reference:
``forward_scan_chunked`` and ``backward_scan_fused_single_chunk`` take
``(num_seq, num_chunks, C)``; ``forward_scan_onepass_pipelined`` and
``backward_scan_fused`` take ``(num_seq, C)``.  Compile-time parameters that
only steer Triton code generation (CHUNK_SIZE, NUM_CHUNKS, NUM_STAGES) are
accepted and ignored: every launch scans whole segments.
"""

from __future__ import annotations

import torch

from associative_scan_triton import _ops


def op(fl, xl, fr, xr):
  """First-order linear recurrence combine (_kernels.py:6-16).

  ``(fl, xl)`` followed by ``(fr, xr)`` composes to
  ``(fr * fl, fr * xl + xr)``; works on Python floats and tensors.
  """
  f = fr * fl
  x = fr * xl + xr
  return f, x


def _cu_slice(cu: torch.Tensor, num_seq: int) -> torch.Tensor:
  # The reference kernels take num_seq from the grid (program axis 0).
  if num_seq + 1 > cu.numel():
    raise ValueError(
      f"grid asks for {num_seq} sequences but cu_seqlens has {cu.numel()} entries")
  return cu[: num_seq + 1]


class _Launchable:
  """``kernel[grid](**kwargs)`` front-end for one libassocscan entry point."""

  def __init__(self, name: str, fn, channel_axis: int):
    self.__name__ = name
    self._fn = fn
    self._channel_axis = channel_axis

  def __getitem__(self, grid):
    grid = tuple(grid)

    def launch(*args, **kwargs):
      return self._fn(grid[0], grid[self._channel_axis], *args, **kwargs)

    return launch

  def __repr__(self) -> str:
    return f"<libassocscan kernel {self.__name__}>"


def _fwd_launch(num_seq, num_channels, gates_ptr, tokens_ptr, tokens_out_ptr,
                cu_seqlens_ptr, REVERSE, CHUNK_SIZE, TESTING, INPLACE,  # noqa: N803
                NUM_CHUNKS=None, NUM_STAGES=None):  # noqa: N803
  del CHUNK_SIZE, NUM_CHUNKS, NUM_STAGES
  out = tokens_ptr if INPLACE else tokens_out_ptr
  _ops.scan_fwd(
    gates_ptr, tokens_ptr, out, _cu_slice(cu_seqlens_ptr, num_seq),
    reverse=bool(REVERSE), gate_prod_out=gates_ptr if TESTING else None,
    num_channels=num_channels,
  )


def _bwd_launch(num_seq, num_channels, grad_ptr, gates_ptr, states_ptr,
                d_tokens_ptr, d_gates_ptr, cu_seqlens_ptr, CHUNK_SIZE,  # noqa: N803
                CAUSAL, NUM_CHUNKS=None, NUM_STAGES=None):  # noqa: N803
  del CHUNK_SIZE, NUM_CHUNKS, NUM_STAGES
  _ops.scan_bwd(
    grad_ptr, gates_ptr, states_ptr, d_tokens_ptr, d_gates_ptr,
    _cu_slice(cu_seqlens_ptr, num_seq), causal=bool(CAUSAL),
    num_channels=num_channels,
  )


# _kernels.py:19-81 (grid (num_seq, num_chunks, C); channel on axis 2)
forward_scan_chunked = _Launchable("forward_scan_chunked", _fwd_launch, 2)
# _kernels.py:84-168 (grid (num_seq, C))
forward_scan_onepass_pipelined = _Launchable(
  "forward_scan_onepass_pipelined", _fwd_launch, 1)
# _kernels.py:171-287 (grid (num_seq, C))
backward_scan_fused = _Launchable("backward_scan_fused", _bwd_launch, 1)
# _kernels.py:290-374 (grid (num_seq, 1, C))
backward_scan_fused_single_chunk = _Launchable(
  "backward_scan_fused_single_chunk", _bwd_launch, 2)
