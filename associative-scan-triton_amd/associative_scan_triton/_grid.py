"""Launch-grid helpers (integer host logic, same results as the reference).

Reference: _grid.py:4-70.  The grid tuple is part of the public ``args``
dict, ``(num_seq, num_chunks, no_channels)``.  On MI355X the kernels do not
need ``num_chunks`` (one wavefront walks a whole segment), but the tuple is
still produced and validated so that callers written for the reference keep
working unchanged.
"""

from __future__ import annotations


def next_power_of_2(n: int) -> int:
  """Smallest power of 2 >= n (bit smearing; 0 -> 0, as _grid.py:4-14)."""
  n -= 1
  n |= n >> 1
  n |= n >> 2
  n |= n >> 4
  n |= n >> 8
  n |= n >> 16
  n |= n >> 32
  n += 1
  return n


def get_grid(
  no_seq: int, max_seqlen: int, chunk_size: int, no_channels: int
) -> tuple[int, int, int]:
  """Returns ``(no_seq - 1, next_pow2(ceil(max_seqlen / chunk)), C)``.

  ``no_seq`` is ``len(cu_seqlens)``.  Asserts an even chunk size with the
  reference message (_grid.py:17-34).
  """
  assert chunk_size % 2 == 0, "chunk size must be divisible by 2"
  num_chunks = (max_seqlen + chunk_size - 1) // chunk_size
  num_chunks = next_power_of_2(num_chunks)
  return (no_seq - 1, num_chunks, no_channels)


def get_num_stages(num_chunks: int, kernel: str = "fwd") -> int:
  """Pipelining depth the reference picks (_grid.py:37-54).

  Kept for API compatibility; the HIP kernels choose their own unrolling.
  """
  if num_chunks <= 1:
    return 1
  if kernel == "fwd":
    return 1 if num_chunks <= 4 else 3
  return 2 if num_chunks <= 4 else 3


def get_static_grid(
  max_seqlen: int, chunk_size: int, no_channels: int
) -> tuple[int, int]:
  """Batch-independent part ``(num_chunks, no_channels)`` (_grid.py:57-70)."""
  return get_grid(2, max_seqlen, chunk_size, no_channels)[1:]
