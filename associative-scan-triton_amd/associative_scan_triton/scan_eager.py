"""Eager autograd scans (reference: scan_eager.py:20-210).

Same public functions, argument meaning, saved tensors and gradient order
as the reference.  Differences are internal: the bidirectional scan runs
both branches in one launch forward and one launch backward instead of two
each.

Addition: ``recompute_states=True`` (default False) keeps the forward's
inputs and one fp32 checkpoint per 4096 fp32 / 8192 fp16-bf16 elements of
each row for the backward instead of the scanned output, which the
backward then recomputes chunk by chunk in registers (no [C, T] tensor of
states is kept alive between the forward and the backward; the backward's
HBM traffic is unchanged).  Results agree with the default mode to the
dtype's rounding.  The reference lists this as future work (the
recompute-states backward; it saves the outputs, scan_eager.py:42-47).
"""

from __future__ import annotations

import torch

from associative_scan_triton import _ops


def _unpack_args(args: dict):
  return args["cu_seqlens"], args["chunk_size"], args["grid"]


class ScanCausal(torch.autograd.Function):
  """Causal (unidirectional) scan with autograd (scan_eager.py:20-64)."""

  @staticmethod
  def forward(ctx, gates, tokens, args, recompute_states=False) -> torch.Tensor:
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
      ctx.recompute = bool(recompute_states)
      if ctx.recompute:
        ckpt = _checkpoints(gates, tokens, out_tokens, cu_seqlens, False, grid[2])
        ctx.save_for_backward(gates, tokens, ckpt)
      else:
        ctx.save_for_backward(out_tokens, gates)
    return out_tokens

  @staticmethod
  def backward(ctx, grad_output):
    if ctx.recompute:
      gates, tokens, ckpt = ctx.saved_tensors
      d_tokens = torch.empty_like(tokens)
      d_gates = torch.empty_like(gates)
      _ops.scan_bwd_recompute(grad_output, gates, tokens, ckpt, d_tokens,
                              d_gates, ctx.cu_seqlens, causal=True,
                              num_channels=ctx.grid[2])
      return d_gates, d_tokens, None, None
    states, gates = ctx.saved_tensors
    # A gradient constant along time (out.sum()) is read one value per row
    # instead of being materialised (the reference's .contiguous(),
    # scan_eager.py:61); any other layout is made contiguous.
    d_tokens = torch.empty_like(states)
    d_gates = torch.empty_like(gates)
    _ops.scan_bwd_any(grad_output, gates, states, d_tokens, d_gates,
                      ctx.cu_seqlens, causal=True, num_channels=ctx.grid[2])
    return d_gates, d_tokens, None, None


def _checkpoints(gates, tokens, states, cu_seqlens, reverse, num_channels):
  """Checkpoints for the recompute backward, or None when the backward will
  recompute the states with the forward scan instead (few items, unaligned
  tensors)."""
  if not _ops.recompute_in_kernel(gates, tokens, cu_seqlens, num_channels):
    return None
  return _ops.scan_checkpoints(states, cu_seqlens, reverse, num_channels)


def scan_causal(
  gates: torch.Tensor,
  tokens: torch.Tensor,
  args: dict,
  recompute_states: bool = False,
) -> torch.Tensor:
  """Causal associative scan ``h[t] = gates[t]*h[t-1] + tokens[t]``.

  Args:
    gates: [C, B*L] gate values
    tokens: [C, B*L] token values
    args: dict with keys "cu_seqlens" ([B+1] cumulative lengths),
      "chunk_size" (int) and "grid" ((num_seq, num_chunks, no_channels)).
    recompute_states: keep (gates, tokens) and per-chunk checkpoints for the
      backward instead of the output, and recompute the states there.

  Returns:
    scanned tokens, [C, B*L]
  """
  return ScanCausal.apply(gates, tokens, args, recompute_states)


class ScanBidirectionalBranched(torch.autograd.Function):
  """Two branches in opposite directions (scan_eager.py:93-178)."""

  @staticmethod
  def forward(ctx, gates_fwd, tokens_fwd, gates_bwd, tokens_bwd, args,
              testing=False, recompute_states=False):
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
      ctx.recompute = bool(recompute_states)
      if ctx.recompute:
        ckf = _checkpoints(gates_fwd, tokens_fwd, out_tokens_fwd, cu_seqlens,
                           False, grid[2])
        ckb = _checkpoints(gates_bwd, tokens_bwd, out_tokens_bwd, cu_seqlens,
                           True, grid[2])
        ctx.save_for_backward(gates_fwd, tokens_fwd, gates_bwd, tokens_bwd,
                              ckf, ckb)
      else:
        ctx.save_for_backward(
          out_tokens_fwd, out_tokens_bwd, gates_fwd, gates_bwd
        )
    # an output that receives no gradient arrives as None (a zero gradient
    # read as one value, not a materialised zeros tensor)
    ctx.set_materialize_grads(False)
    return out_tokens_fwd, out_tokens_bwd

  @staticmethod
  def backward(ctx, grad_output_fwd, grad_output_bwd):
    if ctx.recompute:
      gf, tf, gb, tb, ckf, ckb = ctx.saved_tensors
      out = [torch.empty_like(t) for t in (gf, tf, gb, tb)]
      _ops.scan_bwd_recompute(grad_output_fwd, gf, tf, ckf, out[1], out[0],
                              ctx.cu_seqlens, causal=True,
                              num_channels=ctx.grid[2])
      _ops.scan_bwd_recompute(grad_output_bwd, gb, tb, ckb, out[3], out[2],
                              ctx.cu_seqlens, causal=False,
                              num_channels=ctx.grid[2])
      return (*out, None, None, None)
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
      None,  # recompute_states
    )


def scan_bidirectional_branched(
  gates_fwd: torch.Tensor,
  tokens_fwd: torch.Tensor,
  gates_bwd: torch.Tensor,
  tokens_bwd: torch.Tensor,
  args: dict,
  testing: bool = True,
  recompute_states: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
  """Bidirectional branched scan: causal over the forward pair, reverse over
  the backward pair.  ``testing`` is accepted and, as in the reference
  (scan_eager.py:137), has no effect on the results; ``recompute_states`` as
  for scan_causal, per branch.

  Returns:
    (scanned_tokens_fwd, scanned_tokens_bwd)
  """
  return ScanBidirectionalBranched.apply(
    gates_fwd, tokens_fwd, gates_bwd, tokens_bwd, args, testing,
    recompute_states
  )
