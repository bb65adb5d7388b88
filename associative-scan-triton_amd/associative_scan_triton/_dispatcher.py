"""Host dispatch for direct (non-autograd) scan calls.

Same signatures and semantics as the reference dispatcher
(_dispatcher.py:12-117).  The reference picks a single-chunk or a pipelined
multi-chunk Triton kernel from ``grid[1]``; on MI355X one kernel family
covers every length (a wavefront walks the whole segment with a register
carry), so ``CHUNK_SIZE`` and ``NUM_STAGES`` are accepted and ignored.
Results do not depend on them; the reference's single-chunk kernel is only
defined when ``CHUNK_SIZE`` covers the longest segment, and there the two
agree.
"""

from __future__ import annotations

import torch

from associative_scan_triton import _ops


def forward_scan_full(
  gates: torch.Tensor,
  tokens: torch.Tensor,
  cu_seqlens: torch.Tensor,
  grid: tuple,
  REVERSE: bool,  # noqa: N803
  CHUNK_SIZE: int,  # noqa: N803
  TESTING: bool = True,  # noqa: N803
  NUM_STAGES: int | None = None,  # noqa: N803
  tokens_out: torch.Tensor | None = None,
) -> None:
  """Forward scan, in place or into ``tokens_out`` (_dispatcher.py:12-70).

  ``tokens_out is None`` writes h back into ``tokens``; ``TESTING`` writes the
  running gate product into ``gates`` (the reference default is True).
  """
  assert (
    len(cu_seqlens) - 1 == grid[0]
  ), "cu_seqlens do not match grid configuration"
  del CHUNK_SIZE, NUM_STAGES
  out = tokens if tokens_out is None else tokens_out
  _ops.scan_fwd(
    gates, tokens, out, cu_seqlens, reverse=bool(REVERSE),
    gate_prod_out=gates if TESTING else None, num_channels=grid[2],
  )


def backward_scan_fused_full(
  grad: torch.Tensor,
  gates: torch.Tensor,
  states: torch.Tensor,
  d_tokens_out: torch.Tensor,
  d_gates_out: torch.Tensor,
  cu_seqlens: torch.Tensor,
  grid: tuple,
  CHUNK_SIZE: int,  # noqa: N803
  CAUSAL: bool,  # noqa: N803
  NUM_STAGES: int | None = None,  # noqa: N803
) -> None:
  """Fused backward into preallocated outputs (_dispatcher.py:73-117)."""
  del CHUNK_SIZE, NUM_STAGES
  _ops.scan_bwd(
    grad, gates, states, d_tokens_out, d_gates_out, cu_seqlens,
    causal=bool(CAUSAL), num_channels=grid[2],
  )
