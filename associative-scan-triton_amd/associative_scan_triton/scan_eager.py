"""Eager autograd scans (reference: scan_eager.py:20-210).

Same public functions, argument meaning, saved tensors and gradient order
as the reference.  Differences are internal: the bidirectional scan runs
both branches in one launch forward and one launch backward instead of two
each.
"""

from __future__ import annotations

import torch

from associative_scan_triton import _ops


def _unpack_args(args: dict):
  return args["cu_seqlens"], args["chunk_size"], args["grid"]


class ScanCausal(torch.autograd.Function):
  """Causal (unidirectional) scan with autograd (scan_eager.py:20-64)."""

  @staticmethod
  def forward(ctx, gates, tokens, args) -> torch.Tensor:
    shape = gates.shape
    assert tokens.shape == shape
    assert gates.is_contiguous()
    assert tokens.is_contiguous()
    cu_seqlens, chunk_size, grid = _unpack_args(args)
    assert (
      len(cu_seqlens) - 1 == grid[0]
    ), "cu_seqlens do not match grid configuration"
    need_backward = gates.requires_grad or tokens.requires_grad

    out_tokens = torch.empty_like(tokens)
    _ops.scan_fwd(gates, tokens, out_tokens, cu_seqlens, reverse=False,
                  num_channels=grid[2])

    if need_backward:
      ctx.grid = grid
      ctx.cu_seqlens = cu_seqlens
      ctx.chunk_size = chunk_size
      ctx.save_for_backward(out_tokens, gates)
    return out_tokens

  @staticmethod
  def backward(ctx, grad_output):
    states, gates = ctx.saved_tensors
    # A gradient constant along time (out.sum()) is read one value per row
    # instead of being materialised (the reference's .contiguous(),
    # scan_eager.py:61); any other layout is made contiguous.
    d_tokens = torch.empty_like(states)
    d_gates = torch.empty_like(gates)
    _ops.scan_bwd_any(grad_output, gates, states, d_tokens, d_gates,
                      ctx.cu_seqlens, causal=True, num_channels=ctx.grid[2])
    return d_gates, d_tokens, None


def scan_causal(
  gates: torch.Tensor,
  tokens: torch.Tensor,
  args: dict,
) -> torch.Tensor:
  """Causal associative scan ``h[t] = gates[t]*h[t-1] + tokens[t]``.

  Args:
    gates: [C, B*L] gate values
    tokens: [C, B*L] token values
    args: dict with keys "cu_seqlens" ([B+1] cumulative lengths),
      "chunk_size" (int) and "grid" ((num_seq, num_chunks, no_channels)).

  Returns:
    scanned tokens, [C, B*L]
  """
  return ScanCausal.apply(gates, tokens, args)


class ScanBidirectionalBranched(torch.autograd.Function):
  """Two branches in opposite directions (scan_eager.py:93-178)."""

  @staticmethod
  def forward(ctx, gates_fwd, tokens_fwd, gates_bwd, tokens_bwd, args,
              testing=False):
    shape = gates_fwd.shape
    assert tokens_fwd.shape == shape
    assert tokens_bwd.shape == shape
    assert gates_fwd.is_contiguous()
    assert gates_bwd.is_contiguous()
    assert tokens_fwd.is_contiguous()
    assert tokens_bwd.is_contiguous()
    cu_seqlens, chunk_size, grid = _unpack_args(args)
    assert (
      len(cu_seqlens) - 1 == grid[0]
    ), "cu_seqlens do not match grid configuration"
    need_backward = (
      gates_fwd.requires_grad or tokens_fwd.requires_grad
      or gates_bwd.requires_grad or tokens_bwd.requires_grad
    )

    out_tokens_fwd = torch.empty_like(tokens_fwd)
    out_tokens_bwd = torch.empty_like(tokens_bwd)
    _ops.scan_bidi_fwd(gates_fwd, tokens_fwd, gates_bwd, tokens_bwd,
                       out_tokens_fwd, out_tokens_bwd, cu_seqlens,
                       num_channels=grid[2])

    if need_backward:
      ctx.grid = grid
      ctx.cu_seqlens = cu_seqlens
      ctx.chunk_size = chunk_size
      ctx.testing = testing
      ctx.save_for_backward(
        out_tokens_fwd, out_tokens_bwd, gates_fwd, gates_bwd
      )
    # an output that receives no gradient arrives as None (a zero gradient
    # read as one value, not a materialised zeros tensor)
    ctx.set_materialize_grads(False)
    return out_tokens_fwd, out_tokens_bwd

  @staticmethod
  def backward(ctx, grad_output_fwd, grad_output_bwd):
    states_fwd, states_bwd, gates_fwd, gates_bwd = ctx.saved_tensors
    # gradients constant along time (out.sum()) are read one value per row;
    # any other layout is made contiguous, as the reference does
    d_tokens_fwd = torch.empty_like(states_fwd)
    d_gates_fwd = torch.empty_like(gates_fwd)
    d_tokens_bwd = torch.empty_like(states_bwd)
    d_gates_bwd = torch.empty_like(gates_bwd)
    _ops.scan_bidi_bwd_any(grad_output_fwd, grad_output_bwd, gates_fwd,
                           gates_bwd, states_fwd, states_bwd, d_tokens_fwd,
                           d_gates_fwd, d_tokens_bwd, d_gates_bwd,
                           ctx.cu_seqlens, num_channels=ctx.grid[2])
    return (
      d_gates_fwd,
      d_tokens_fwd,
      d_gates_bwd,
      d_tokens_bwd,
      None,  # args
      None,  # testing
    )


def scan_bidirectional_branched(
  gates_fwd: torch.Tensor,
  tokens_fwd: torch.Tensor,
  gates_bwd: torch.Tensor,
  tokens_bwd: torch.Tensor,
  args: dict,
  testing: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
  """Bidirectional branched scan: causal over the forward pair, reverse over
  the backward pair.  ``testing`` is accepted and, as in the reference
  (scan_eager.py:137), has no effect on the results.

  Returns:
    (scanned_tokens_fwd, scanned_tokens_bwd)
  """
  return ScanBidirectionalBranched.apply(
    gates_fwd, tokens_fwd, gates_bwd, tokens_bwd, args, testing
  )
