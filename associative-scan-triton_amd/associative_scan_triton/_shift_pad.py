"""Segment-aware shift-and-pad (reference: _shift_pad.py:18-165).

``shift_pad`` (eager) and ``shift_pad_compiled`` (custom op
``associative_scan_triton::shift_pad``) both run the same gfx950 kernels,
which read the input through its strides (no copy).
The eager form keeps the reference's zero-length check, with its exact
message, and its torch.roll wrap-around at the row ends; the compiled form,
like the reference's Triton kernel, clamps at the row ends and does no
host-side check (so it never synchronises).
"""

from __future__ import annotations

import torch

from associative_scan_triton import _ops


def shift_pad(
  data: torch.Tensor,
  cu_seqlens: torch.Tensor,
  pad_value: float = 0.0,
  backward: bool = True,
) -> torch.Tensor:
  """Shifts every segment by one position and pads the vacated slot.

  Parameters:
  - data: [C, BL] where C is the number of channels and BL the total length
  - cu_seqlens: cumulative sequence lengths
  - pad_value: value written at segment starts (backward) or ends (forward)
  - backward: True shifts right (out[p] = data[p-1]), False shifts left

  Returns:
  - [C, BL] shifted and padded tensor
  """
  _C, _BL = data.shape
  # Data-dependent check, as in the reference (synchronises the device).
  assert not (
    cu_seqlens[1:] == cu_seqlens[:-1]
  ).any(), "can't shift_pad zero-length seqments"
  # any input strides are read in place; the result is contiguous, as
  # torch.roll's is in the reference
  out = torch.empty_like(data, memory_format=torch.contiguous_format)
  _ops.shift_pad(data, out, cu_seqlens, pad_value, backward, wrap=True)
  return out


@torch.library.custom_op("associative_scan_triton::shift_pad", mutates_args=())
def shift_pad_compiled(
  data: torch.Tensor,
  cu_seqlens: torch.Tensor,
  pad_value: float,
  backward: bool,
) -> torch.Tensor:
  """Compile-compatible shift_pad.

  Args:
      data: [C, BL] tensor
      cu_seqlens: [num_seq + 1] cumulative sequence lengths
      pad_value: value for padding (1.0 for gates, 0.0 for states)
      backward: True = shift right (pad at seq starts),
        False = shift left (pad at seq ends)
  """
  # the reference's kernel reads data through its strides and writes
  # torch.empty_like(data), which keeps the layout of a dense input
  # (_shift_pad.py:140,156-157); so here, with no copy of the input
  out = torch.empty_like(data)
  _ops.shift_pad(data, out, cu_seqlens, pad_value, backward, wrap=False)
  return out


@shift_pad_compiled.register_fake
def _(data, cu_seqlens, pad_value, backward):
  return torch.empty_like(data)
