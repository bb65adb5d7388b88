"""Chunked associative scan for h[t] = g[t]*h[t-1] + x[t] on AMD Instinct
MI355X (gfx950), with varlen packing, a bidirectional variant and
torch.compile support.

Drop-in replacement for the public API of associative-scan-triton 1.0.0
(reference __init__.py:1-36).  Every compute path runs hand-written HIP
kernels from libassocscan.so; there is no Triton and no CPU fallback.
"""

__version__ = "1.0.0"

from associative_scan_triton._kernels import (
  op,
  forward_scan_chunked,
  forward_scan_onepass_pipelined,
  backward_scan_fused,
  backward_scan_fused_single_chunk,
)
from associative_scan_triton._dispatcher import (
  forward_scan_full,
  backward_scan_fused_full,
)
from associative_scan_triton._shift_pad import shift_pad, shift_pad_compiled
from associative_scan_triton._grid import (
  next_power_of_2,
  get_grid,
  get_static_grid,
  get_num_stages,
)
from associative_scan_triton.scan_eager import (
  scan_causal,
  scan_bidirectional_branched,
)
from associative_scan_triton.scan_compiled import (
  scan_causal_compiled,
  scan_bidirectional_branched_compiled,
)

__all__ = [
  # Kernels
  "op",
  "forward_scan_chunked",
  "forward_scan_onepass_pipelined",
  "forward_scan_full",
  "backward_scan_fused",
  "backward_scan_fused_single_chunk",
  "backward_scan_fused_full",
  # Shift-pad
  "shift_pad",
  "shift_pad_compiled",
  # Grid utilities
  "next_power_of_2",
  "get_grid",
  "get_static_grid",
  # High-level API
  "scan_causal",
  "scan_causal_compiled",
  "scan_bidirectional_branched",
  "scan_bidirectional_branched_compiled",
]
