"""torch.compile-safe scans as torch.library custom ops.

Reference: scan_compiled.py:33-371, which registers ``@triton_op``s.  Here
the same qualnames are registered with ``torch.library.custom_op`` (opaque
to dynamo, so no graph break), each with a fake (meta) implementation and
an autograd formula.

Deliberate difference: the reference forward ops also return
``gates.clone()`` because a triton_op output may not alias an input
(scan_compiled.py:113,240); that copy costs 8 bytes per element of HBM
traffic.  These ops save the gates from the op *inputs* in
``setup_context`` instead, so ``scan_causal_fwd`` returns only the scanned
tokens and ``scan_bidi_fwd`` only the two scanned branches.  The public
functions ``scan_causal_compiled`` and ``scan_bidirectional_branched_compiled``
return exactly what the reference's do.
"""

from __future__ import annotations

import torch

from associative_scan_triton import _ops

# ============================================================
# Causal scan
# ============================================================


@torch.library.custom_op("associative_scan_triton::scan_causal_fwd",
                         mutates_args=())
def scan_causal_fwd_op(
  gates: torch.Tensor,
  tokens: torch.Tensor,
  cu_seqlens: torch.Tensor,
  num_chunks: int,
  no_channels: int,
  chunk_size: int,
) -> torch.Tensor:
  """Causal scan forward; gates and tokens are read-only."""
  out = torch.empty_like(tokens)
  _ops.scan_fwd(gates, tokens, out, cu_seqlens, reverse=False,
                num_channels=no_channels)
  return out


@scan_causal_fwd_op.register_fake
def _(gates, tokens, cu_seqlens, num_chunks, no_channels, chunk_size):
  return torch.empty_like(tokens)


@torch.library.custom_op("associative_scan_triton::scan_causal_bwd",
                         mutates_args=())
def scan_causal_bwd_op(
  grad: torch.Tensor,
  gates: torch.Tensor,
  states: torch.Tensor,
  cu_seqlens: torch.Tensor,
  num_chunks: int,
  no_channels: int,
  chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor]:
  """Causal scan backward; returns (d_gates, d_tokens).  A gradient that
  is constant along time is read one value per row, not materialised."""
  d_tokens = torch.empty_like(states)
  d_gates = torch.empty_like(gates)
  _ops.scan_bwd_any(grad, gates, states, d_tokens, d_gates, cu_seqlens,
                    causal=True, num_channels=no_channels)
  return d_gates, d_tokens


@scan_causal_bwd_op.register_fake
def _(grad, gates, states, cu_seqlens, num_chunks, no_channels, chunk_size):
  return torch.empty_like(gates), torch.empty_like(states)


def _scan_causal_setup_context(ctx, inputs, output) -> None:
  gates, _tokens, cu_seqlens, num_chunks, no_channels, chunk_size = inputs
  ctx.save_for_backward(output, gates)
  ctx.cu_seqlens = cu_seqlens
  ctx.num_chunks = num_chunks
  ctx.no_channels = no_channels
  ctx.chunk_size = chunk_size


def _scan_causal_backward(ctx, grad):
  states, gates = ctx.saved_tensors
  if grad is None:
    grad = states.new_zeros(()).expand_as(states)
  d_gates, d_tokens = scan_causal_bwd_op(
    grad, gates, states, ctx.cu_seqlens,
    ctx.num_chunks, ctx.no_channels, ctx.chunk_size,
  )
  return d_gates, d_tokens, None, None, None, None


scan_causal_fwd_op.register_autograd(
  _scan_causal_backward, setup_context=_scan_causal_setup_context
)

# ============================================================
# Bidirectional branched scan
# ============================================================


@torch.library.custom_op("associative_scan_triton::scan_bidi_fwd",
                         mutates_args=())
def scan_bidi_fwd_op(
  gates_fwd: torch.Tensor,
  tokens_fwd: torch.Tensor,
  gates_bwd: torch.Tensor,
  tokens_bwd: torch.Tensor,
  cu_seqlens: torch.Tensor,
  num_chunks: int,
  no_channels: int,
  chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor]:
  """Both branches in one launch; returns (out_tokens_fwd, out_tokens_bwd)."""
  out_fwd = torch.empty_like(tokens_fwd)
  out_bwd = torch.empty_like(tokens_bwd)
  _ops.scan_bidi_fwd(gates_fwd, tokens_fwd, gates_bwd, tokens_bwd, out_fwd,
                     out_bwd, cu_seqlens, num_channels=no_channels)
  return out_fwd, out_bwd


@scan_bidi_fwd_op.register_fake
def _(gates_fwd, tokens_fwd, gates_bwd, tokens_bwd, cu_seqlens, num_chunks,
      no_channels, chunk_size):
  return torch.empty_like(tokens_fwd), torch.empty_like(tokens_bwd)


@torch.library.custom_op("associative_scan_triton::scan_bidi_bwd",
                         mutates_args=())
def scan_bidi_bwd_op(
  grad_fwd: torch.Tensor,
  grad_bwd: torch.Tensor,
  states_fwd: torch.Tensor,
  states_bwd: torch.Tensor,
  gates_fwd: torch.Tensor,
  gates_bwd: torch.Tensor,
  cu_seqlens: torch.Tensor,
  num_chunks: int,
  no_channels: int,
  chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
  """Backward of both branches in one launch.  Gradients that are constant
  along time are read one value per row, not materialised.

  Returns (d_gates_fwd, d_tokens_fwd, d_gates_bwd, d_tokens_bwd).
  """
  d_tokens_fwd = torch.empty_like(states_fwd)
  d_gates_fwd = torch.empty_like(gates_fwd)
  d_tokens_bwd = torch.empty_like(states_bwd)
  d_gates_bwd = torch.empty_like(gates_bwd)
  _ops.scan_bidi_bwd_any(grad_fwd, grad_bwd, gates_fwd, gates_bwd,
                         states_fwd, states_bwd, d_tokens_fwd, d_gates_fwd,
                         d_tokens_bwd, d_gates_bwd, cu_seqlens,
                         num_channels=no_channels)
  return d_gates_fwd, d_tokens_fwd, d_gates_bwd, d_tokens_bwd


@scan_bidi_bwd_op.register_fake
def _(grad_fwd, grad_bwd, states_fwd, states_bwd, gates_fwd, gates_bwd,
      cu_seqlens, num_chunks, no_channels, chunk_size):
  return (torch.empty_like(gates_fwd), torch.empty_like(states_fwd),
          torch.empty_like(gates_bwd), torch.empty_like(states_bwd))


def _scan_bidi_setup_context(ctx, inputs, output) -> None:
  (gates_fwd, _tokens_fwd, gates_bwd, _tokens_bwd,
   cu_seqlens, num_chunks, no_channels, chunk_size) = inputs
  out_fwd, out_bwd = output
  ctx.save_for_backward(out_fwd, out_bwd, gates_fwd, gates_bwd)
  # an output that receives no gradient arrives as None (read below as one
  # zero value per row), not as a materialised zeros tensor
  ctx.set_materialize_grads(False)
  ctx.cu_seqlens = cu_seqlens
  ctx.num_chunks = num_chunks
  ctx.no_channels = no_channels
  ctx.chunk_size = chunk_size


def _scan_bidi_backward(ctx, grad_fwd, grad_bwd):
  states_fwd, states_bwd, gates_fwd, gates_bwd = ctx.saved_tensors
  # an output without a gradient: a zero gradient constant along time (read
  # as one value per row by the backward, no [C, T] zeros tensor)
  if grad_fwd is None:
    grad_fwd = states_fwd.new_zeros(()).expand_as(states_fwd)
  if grad_bwd is None:
    grad_bwd = states_bwd.new_zeros(()).expand_as(states_bwd)
  d_gates_fwd, d_tokens_fwd, d_gates_bwd, d_tokens_bwd = scan_bidi_bwd_op(
    grad_fwd, grad_bwd, states_fwd, states_bwd, gates_fwd, gates_bwd,
    ctx.cu_seqlens, ctx.num_chunks, ctx.no_channels, ctx.chunk_size,
  )
  return (d_gates_fwd, d_tokens_fwd, d_gates_bwd, d_tokens_bwd,
          None, None, None, None)


scan_bidi_fwd_op.register_autograd(
  _scan_bidi_backward, setup_context=_scan_bidi_setup_context
)

# ============================================================
# Recompute mode: the forward ops also return per-chunk checkpoints, and
# autograd saves (gates, tokens, checkpoints) instead of the outputs; the
# backward ops recompute the states (see scan_eager.py's recompute_states).
# The checkpoints are always produced (their shape depends only on the
# tensors' shapes and dtype), whichever way the backward then recomputes.
# ============================================================


def _ckpt_like(tokens: torch.Tensor, no_channels: int) -> torch.Tensor:
  return tokens.new_empty(_ops.checkpoint_shape(tokens, no_channels),
                          dtype=torch.float32)


@torch.library.custom_op("associative_scan_triton::scan_causal_fwd_rc",
                         mutates_args=())
def scan_causal_fwd_rc_op(
  gates: torch.Tensor,
  tokens: torch.Tensor,
  cu_seqlens: torch.Tensor,
  num_chunks: int,
  no_channels: int,
  chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor]:
  """Causal scan forward; returns (out_tokens, checkpoints)."""
  out = torch.empty_like(tokens)
  _ops.scan_fwd(gates, tokens, out, cu_seqlens, reverse=False,
                num_channels=no_channels)
  return out, _ops.scan_checkpoints(out, cu_seqlens, False, no_channels)


@scan_causal_fwd_rc_op.register_fake
def _(gates, tokens, cu_seqlens, num_chunks, no_channels, chunk_size):
  return torch.empty_like(tokens), _ckpt_like(tokens, no_channels)


@torch.library.custom_op("associative_scan_triton::scan_causal_bwd_rc",
                         mutates_args=())
def scan_causal_bwd_rc_op(
  grad: torch.Tensor,
  gates: torch.Tensor,
  tokens: torch.Tensor,
  checkpoints: torch.Tensor,
  cu_seqlens: torch.Tensor,
  num_chunks: int,
  no_channels: int,
  chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor]:
  """Causal scan backward from the forward's inputs and checkpoints;
  returns (d_gates, d_tokens)."""
  d_tokens = torch.empty_like(tokens)
  d_gates = torch.empty_like(gates)
  _ops.scan_bwd_recompute(grad, gates, tokens, checkpoints, d_tokens, d_gates,
                          cu_seqlens, causal=True, num_channels=no_channels)
  return d_gates, d_tokens


@scan_causal_bwd_rc_op.register_fake
def _(grad, gates, tokens, checkpoints, cu_seqlens, num_chunks, no_channels,
      chunk_size):
  return torch.empty_like(gates), torch.empty_like(tokens)


def _scan_causal_rc_setup_context(ctx, inputs, output) -> None:
  gates, tokens, cu_seqlens, num_chunks, no_channels, chunk_size = inputs
  _out, ckpt = output
  ctx.mark_non_differentiable(ckpt)
  ctx.set_materialize_grads(False)
  ctx.save_for_backward(gates, tokens, ckpt)
  ctx.cu_seqlens = cu_seqlens
  ctx.num_chunks = num_chunks
  ctx.no_channels = no_channels
  ctx.chunk_size = chunk_size


def _scan_causal_rc_backward(ctx, grad, _grad_ckpt):
  gates, tokens, ckpt = ctx.saved_tensors
  if grad is None:
    grad = tokens.new_zeros(()).expand_as(tokens)
  d_gates, d_tokens = scan_causal_bwd_rc_op(
    grad, gates, tokens, ckpt, ctx.cu_seqlens, ctx.num_chunks,
    ctx.no_channels, ctx.chunk_size)
  return d_gates, d_tokens, None, None, None, None


scan_causal_fwd_rc_op.register_autograd(
  _scan_causal_rc_backward, setup_context=_scan_causal_rc_setup_context
)


@torch.library.custom_op("associative_scan_triton::scan_bidi_fwd_rc",
                         mutates_args=())
def scan_bidi_fwd_rc_op(
  gates_fwd: torch.Tensor,
  tokens_fwd: torch.Tensor,
  gates_bwd: torch.Tensor,
  tokens_bwd: torch.Tensor,
  cu_seqlens: torch.Tensor,
  num_chunks: int,
  no_channels: int,
  chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
  """Both branches in one launch; returns (out_tokens_fwd, out_tokens_bwd,
  checkpoints_fwd, checkpoints_bwd)."""
  out_fwd = torch.empty_like(tokens_fwd)
  out_bwd = torch.empty_like(tokens_bwd)
  _ops.scan_bidi_fwd(gates_fwd, tokens_fwd, gates_bwd, tokens_bwd, out_fwd,
                     out_bwd, cu_seqlens, num_channels=no_channels)
  return (out_fwd, out_bwd,
          _ops.scan_checkpoints(out_fwd, cu_seqlens, False, no_channels),
          _ops.scan_checkpoints(out_bwd, cu_seqlens, True, no_channels))


@scan_bidi_fwd_rc_op.register_fake
def _(gates_fwd, tokens_fwd, gates_bwd, tokens_bwd, cu_seqlens, num_chunks,
      no_channels, chunk_size):
  return (torch.empty_like(tokens_fwd), torch.empty_like(tokens_bwd),
          _ckpt_like(tokens_fwd, no_channels),
          _ckpt_like(tokens_bwd, no_channels))


@torch.library.custom_op("associative_scan_triton::scan_bidi_bwd_rc",
                         mutates_args=())
def scan_bidi_bwd_rc_op(
  grad_fwd: torch.Tensor,
  grad_bwd: torch.Tensor,
  gates_fwd: torch.Tensor,
  tokens_fwd: torch.Tensor,
  gates_bwd: torch.Tensor,
  tokens_bwd: torch.Tensor,
  checkpoints_fwd: torch.Tensor,
  checkpoints_bwd: torch.Tensor,
  cu_seqlens: torch.Tensor,
  num_chunks: int,
  no_channels: int,
  chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
  """Backward of both branches from their inputs and checkpoints; returns
  (d_gates_fwd, d_tokens_fwd, d_gates_bwd, d_tokens_bwd)."""
  out = [torch.empty_like(t) for t in
         (gates_fwd, tokens_fwd, gates_bwd, tokens_bwd)]
  _ops.scan_bwd_recompute(grad_fwd, gates_fwd, tokens_fwd, checkpoints_fwd,
                          out[1], out[0], cu_seqlens, causal=True,
                          num_channels=no_channels)
  _ops.scan_bwd_recompute(grad_bwd, gates_bwd, tokens_bwd, checkpoints_bwd,
                          out[3], out[2], cu_seqlens, causal=False,
                          num_channels=no_channels)
  return tuple(out)


@scan_bidi_bwd_rc_op.register_fake
def _(grad_fwd, grad_bwd, gates_fwd, tokens_fwd, gates_bwd, tokens_bwd,
      checkpoints_fwd, checkpoints_bwd, cu_seqlens, num_chunks, no_channels,
      chunk_size):
  return (torch.empty_like(gates_fwd), torch.empty_like(tokens_fwd),
          torch.empty_like(gates_bwd), torch.empty_like(tokens_bwd))


def _scan_bidi_rc_setup_context(ctx, inputs, output) -> None:
  (gates_fwd, tokens_fwd, gates_bwd, tokens_bwd,
   cu_seqlens, num_chunks, no_channels, chunk_size) = inputs
  _of, _ob, ckf, ckb = output
  ctx.mark_non_differentiable(ckf, ckb)
  ctx.set_materialize_grads(False)
  ctx.save_for_backward(gates_fwd, tokens_fwd, gates_bwd, tokens_bwd, ckf, ckb)
  ctx.cu_seqlens = cu_seqlens
  ctx.num_chunks = num_chunks
  ctx.no_channels = no_channels
  ctx.chunk_size = chunk_size


def _scan_bidi_rc_backward(ctx, grad_fwd, grad_bwd, _gcf, _gcb):
  gf, tf, gb, tb, ckf, ckb = ctx.saved_tensors
  if grad_fwd is None:
    grad_fwd = tf.new_zeros(()).expand_as(tf)
  if grad_bwd is None:
    grad_bwd = tb.new_zeros(()).expand_as(tb)
  d = scan_bidi_bwd_rc_op(grad_fwd, grad_bwd, gf, tf, gb, tb, ckf, ckb,
                          ctx.cu_seqlens, ctx.num_chunks, ctx.no_channels,
                          ctx.chunk_size)
  return (*d, None, None, None, None)


scan_bidi_fwd_rc_op.register_autograd(
  _scan_bidi_rc_backward, setup_context=_scan_bidi_rc_setup_context
)

# ============================================================
# Public API (scan_compiled.py:333-371)
# ============================================================


def scan_causal_compiled(
  gates: torch.Tensor,
  tokens: torch.Tensor,
  args: dict,
  recompute_states: bool = False,
) -> torch.Tensor:
  """Drop-in replacement for scan_causal() built on a custom op."""
  cu_seqlens = args["cu_seqlens"]
  chunk_size = args["chunk_size"]
  _num_seq, num_chunks, no_channels = args["grid"]
  if recompute_states:
    return scan_causal_fwd_rc_op(
      gates, tokens, cu_seqlens, num_chunks, no_channels, chunk_size)[0]
  return scan_causal_fwd_op(
    gates, tokens, cu_seqlens, num_chunks, no_channels, chunk_size,
  )


def scan_bidirectional_branched_compiled(
  gates_fwd: torch.Tensor,
  tokens_fwd: torch.Tensor,
  gates_bwd: torch.Tensor,
  tokens_bwd: torch.Tensor,
  args: dict,
  testing: bool = True,
  recompute_states: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
  """Drop-in replacement for scan_bidirectional_branched() on custom ops."""
  del testing
  cu_seqlens = args["cu_seqlens"]
  chunk_size = args["chunk_size"]
  _num_seq, num_chunks, no_channels = args["grid"]
  if recompute_states:
    return scan_bidi_fwd_rc_op(
      gates_fwd, tokens_fwd, gates_bwd, tokens_bwd,
      cu_seqlens, num_chunks, no_channels, chunk_size)[:2]
  return scan_bidi_fwd_op(
    gates_fwd, tokens_fwd, gates_bwd, tokens_bwd,
    cu_seqlens, num_chunks, no_channels, chunk_size,
  )
