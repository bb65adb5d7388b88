"""Tensor-level launchers over the libassocscan C ABI.

Every public function of the package ends here.  These helpers validate
shapes, dtypes, devices and contiguity on the host (no device sync), derive
the geometry ``(num_seq, C, T)`` and launch on the current stream of the
tensors' device.
"""

from __future__ import annotations

import torch

from associative_scan_triton import _lib

# Problems with few (segment, channel) items run the library's tree walk (or
# its look-back walk when the tensors do not share one 16-byte phase), and
# long chunk-aligned segments its chained walk; all need a workspace, and
# the library says how large (0 = none needed).  False forces the
# workspace-free walks (the walks agree to fp32 rounding).
USE_WORKSPACE = True


def _one_phase(tensors) -> bool:
  """Whether the tensors' addresses agree modulo 16 bytes (the library then
  takes the tree walk, not the look-back walk, for few items)."""
  return bool(tensors) and len({t.data_ptr() % 16 for t in tensors}) == 1


def _walk(lib, S: int, C: int, T: int, dtype_code: int, nbranch: int,
          tensors=()) -> int:
  """The walk a workspace would buy for this geometry (0: none is used).

  For few items the library runs the tree walk, whose results repeat bit
  for bit, when every tensor of the call (`tensors`) has the same address
  modulo 16 bytes, and otherwise the look-back walk, whose last bits can
  vary from run to run (which predecessor a tile meets as inclusive depends
  on timing); under torch.use_deterministic_algorithms(True) the latter is
  not used, and the workspace-free walks, which are bitwise reproducible,
  run instead."""
  if not USE_WORKSPACE:
    return 0
  walk = lib.asc_scan_workspace_walk(S, C, T, dtype_code, nbranch)
  if (walk == _lib.WALK_LOOKBACK and torch.are_deterministic_algorithms_enabled()
      and not _one_phase(tensors)):
    return 0
  return max(walk, 0)


def _workspace(lib, dev: torch.device, S: int, C: int, T: int,
               dtype_code: int, nbranch: int, *tensors):
  """A workspace from torch's caching allocator when the geometry wants one
  (the library clears it on the launch stream), else (None, 0); `tensors`
  are the call's tensors (see _walk)."""
  if not _walk(lib, S, C, T, dtype_code, nbranch, tensors):
    return None, 0
  nbytes = lib.asc_scan_workspace_bytes(S, C, T, dtype_code, nbranch)
  if nbytes <= 0:
    return None, 0
  ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
  return ws, nbytes


def _geometry(t: torch.Tensor, cu: torch.Tensor, num_channels: int | None
              ) -> tuple[int, int, int]:
  """Returns (num_seq, C, T) for a [C, T] (or flat [C*T]) tensor.

  The reference reads the row stride from ``cu_seqlens[num_seq]`` on the
  device (_kernels.py:51,108); here it is the tensor width, and callers must
  keep ``cu_seqlens[-1] == T`` exactly as the reference requires.
  """
  if cu.dim() != 1 or cu.numel() < 1:
    raise ValueError("cu_seqlens must be a 1-D tensor with num_seq + 1 entries")
  num_seq = cu.numel() - 1
  # Addressing is flat (row c starts at c*T), as in the reference kernels, so
  # the channel count comes from the grid when given, else from the rows.
  if num_channels is not None:
    C = int(num_channels)
  else:
    C = t.shape[0] if t.dim() == 2 else 1
  if C <= 0 or t.numel() % C:
    raise ValueError(
      f"a tensor of {t.numel()} elements cannot hold {C} channels")
  return num_seq, C, t.numel() // C


def _check_same(ref: torch.Tensor, *others: torch.Tensor | None) -> None:
  for o in others:
    if o is None:
      continue
    if o.dtype != ref.dtype:
      raise TypeError(f"dtype mismatch: {ref.dtype} vs {o.dtype}")
    if o.numel() != ref.numel():
      raise ValueError(f"size mismatch: {tuple(ref.shape)} vs {tuple(o.shape)}")
    if not o.is_contiguous():
      raise ValueError("all scan tensors must be contiguous")
  if not ref.is_contiguous():
    raise ValueError("all scan tensors must be contiguous")


class _OnDevice:
  """Makes `dev` current for the duration of a launch."""

  def __init__(self, dev: torch.device):
    self.dev = dev
    self.prev = None

  def __enter__(self):
    cur = torch.cuda.current_device()
    if self.dev.index is not None and cur != self.dev.index:
      self.prev = cur
      torch.cuda.set_device(self.dev)
    return self

  def __exit__(self, *exc):
    if self.prev is not None:
      torch.cuda.set_device(self.prev)
    return False


def scan_fwd(gates: torch.Tensor, tokens: torch.Tensor, h_out: torch.Tensor,
             cu: torch.Tensor, reverse: bool,
             gate_prod_out: torch.Tensor | None = None,
             num_channels: int | None = None) -> None:
  """h_out <- scan(gates, tokens); optionally gate_prod_out <- prod(gates)."""
  lib = _lib.load()
  dev = _lib.require_device(gates, tokens, h_out, gate_prod_out, cu)
  _check_same(tokens, gates, h_out, gate_prod_out)
  dt = _lib.dtype_code(tokens)
  cuc = _lib.cu_code(cu)
  cu = cu.contiguous()
  S, C, T = _geometry(tokens, cu, num_channels)
  with _OnDevice(dev):
    # the gate product and in-place calls run the workspace-free walks
    plain = gate_prod_out is None and h_out.data_ptr() != tokens.data_ptr()
    ws, nb = (_workspace(lib, dev, S, C, T, dt, 1, gates, tokens, h_out)
              if plain else (None, 0))
    _lib.check(lib.asc_scan_fwd(
      gates.data_ptr(), tokens.data_ptr(), h_out.data_ptr(),
      _lib.ptr(gate_prod_out), cu.data_ptr(), cuc, S, C, T, dt,
      1 if reverse else 0, _lib.ptr(ws), nb, _lib.stream_of(dev)))


def scan_bwd(grad: torch.Tensor, gates: torch.Tensor, states: torch.Tensor,
             d_tokens: torch.Tensor, d_gates: torch.Tensor, cu: torch.Tensor,
             causal: bool, num_channels: int | None = None) -> None:
  """Fused backward: (d_tokens, d_gates) of a scan given dy, g and h."""
  lib = _lib.load()
  dev = _lib.require_device(grad, gates, states, d_tokens, d_gates, cu)
  _check_same(grad, gates, states, d_tokens, d_gates)
  dt = _lib.dtype_code(grad)
  cuc = _lib.cu_code(cu)
  cu = cu.contiguous()
  S, C, T = _geometry(grad, cu, num_channels)
  with _OnDevice(dev):
    # d_tokens in place of the gradient runs the workspace-free walks
    plain = d_tokens.data_ptr() != grad.data_ptr()
    ws, nb = (_workspace(lib, dev, S, C, T, dt, 1, grad, gates, states,
                         d_tokens, d_gates) if plain else (None, 0))
    _lib.check(lib.asc_scan_bwd(
      grad.data_ptr(), gates.data_ptr(), states.data_ptr(),
      d_tokens.data_ptr(), d_gates.data_ptr(), cu.data_ptr(), cuc, S, C, T,
      dt, 1 if causal else 0, _lib.ptr(ws), nb, _lib.stream_of(dev)))


def row_constant_stride(grad: torch.Tensor, like: torch.Tensor,
                        num_channels: int | None = None) -> int | None:
  """Element stride between rows if `grad` (shaped like `like`) is constant
  along time in every row -- an expanded tensor with time stride 0, as
  autograd passes for out.sum() -- else None."""
  if grad.shape != like.shape or grad.dtype != like.dtype or grad.numel() == 0:
    return None
  if grad.device != like.device:
    return None
  if grad.dim() == 1:
    return 0 if grad.stride(0) == 0 else None
  if grad.dim() != 2 or grad.shape[1] < 2 or grad.stride(1) != 0:
    return None
  if grad.stride(0) == 0:
    return 0
  if num_channels is not None and int(num_channels) != grad.shape[0]:
    return None
  return grad.stride(0)


def scan_bwd_rowgrad(grad: torch.Tensor, row_stride: int, gates: torch.Tensor,
                     states: torch.Tensor, d_tokens: torch.Tensor,
                     d_gates: torch.Tensor, cu: torch.Tensor, causal: bool,
                     num_channels: int | None = None) -> None:
  """Fused backward for a gradient constant along time (one value per row,
  `row_stride` elements apart, read from grad.data_ptr())."""
  lib = _lib.load()
  dev = _lib.require_device(grad, gates, states, d_tokens, d_gates, cu)
  _check_same(states, gates, d_tokens, d_gates)
  if grad.dtype != states.dtype:
    raise TypeError(f"dtype mismatch: {states.dtype} vs {grad.dtype}")
  dt = _lib.dtype_code(states)
  cuc = _lib.cu_code(cu)
  cu = cu.contiguous()
  S, C, T = _geometry(states, cu, num_channels)
  with _OnDevice(dev):
    ws, nb = _workspace(lib, dev, S, C, T, dt, 1, gates, states, d_tokens,
                        d_gates)
    _lib.check(lib.asc_scan_bwd_rowgrad(
      grad.data_ptr(), int(row_stride), gates.data_ptr(), states.data_ptr(),
      d_tokens.data_ptr(), d_gates.data_ptr(), cu.data_ptr(), cuc, S, C, T,
      dt, 1 if causal else 0, _lib.ptr(ws), nb, _lib.stream_of(dev)))


def scan_bwd_any(grad: torch.Tensor, gates: torch.Tensor, states: torch.Tensor,
                 d_tokens: torch.Tensor, d_gates: torch.Tensor,
                 cu: torch.Tensor, causal: bool,
                 num_channels: int | None = None) -> None:
  """Backward for any incoming gradient layout: a gradient that is constant
  along time is read one value per row (no materialised copy) unless the
  geometry runs the look-back walk for few items (tensors of different
  16-byte phases), which needs the full gradient; any other layout is made
  contiguous, as the reference does (scan_eager.py:61)."""
  rs = row_constant_stride(grad, states, num_channels)
  if rs is not None:
    lib = _lib.load()
    cu_c = cu.contiguous()
    S, C, T = _geometry(states, cu_c, num_channels)
    if (_walk(lib, S, C, T, _lib.dtype_code(states), 1) != _lib.WALK_LOOKBACK
        or _one_phase((gates, states, d_tokens, d_gates))):
      scan_bwd_rowgrad(grad, rs, gates, states, d_tokens, d_gates, cu_c,
                       causal, num_channels)
      return
  scan_bwd(grad.contiguous(), gates, states, d_tokens, d_gates, cu, causal,
           num_channels)


def scan_bidi_fwd(gf: torch.Tensor, xf: torch.Tensor, gb: torch.Tensor,
                  xb: torch.Tensor, hf: torch.Tensor, hb: torch.Tensor,
                  cu: torch.Tensor, num_channels: int | None = None) -> None:
  """Both bidirectional branches in one launch."""
  lib = _lib.load()
  dev = _lib.require_device(gf, xf, gb, xb, hf, hb, cu)
  _check_same(xf, gf, gb, xb, hf, hb)
  dt = _lib.dtype_code(xf)
  cuc = _lib.cu_code(cu)
  cu = cu.contiguous()
  S, C, T = _geometry(xf, cu, num_channels)
  with _OnDevice(dev):
    ws, nb = _workspace(lib, dev, S, C, T, dt, 2, gf, xf, gb, xb, hf, hb)
    _lib.check(lib.asc_scan_bidi_fwd(
      gf.data_ptr(), xf.data_ptr(), gb.data_ptr(), xb.data_ptr(),
      hf.data_ptr(), hb.data_ptr(), cu.data_ptr(), cuc, S, C, T, dt,
      _lib.ptr(ws), nb, _lib.stream_of(dev)))


def scan_bidi_bwd(dyf: torch.Tensor, dyb: torch.Tensor, gf: torch.Tensor,
                  gb: torch.Tensor, hf: torch.Tensor, hb: torch.Tensor,
                  dxf: torch.Tensor, dgf: torch.Tensor, dxb: torch.Tensor,
                  dgb: torch.Tensor, cu: torch.Tensor,
                  num_channels: int | None = None) -> None:
  """Backward of both bidirectional branches in one launch."""
  lib = _lib.load()
  dev = _lib.require_device(dyf, dyb, gf, gb, hf, hb, dxf, dgf, dxb, dgb, cu)
  _check_same(dyf, dyb, gf, gb, hf, hb, dxf, dgf, dxb, dgb)
  dt = _lib.dtype_code(dyf)
  cuc = _lib.cu_code(cu)
  cu = cu.contiguous()
  S, C, T = _geometry(dyf, cu, num_channels)
  with _OnDevice(dev):
    ws, nb = _workspace(lib, dev, S, C, T, dt, 2, dyf, dyb, gf, gb, hf, hb,
                        dxf, dgf, dxb, dgb)
    _lib.check(lib.asc_scan_bidi_bwd(
      dyf.data_ptr(), dyb.data_ptr(), gf.data_ptr(), gb.data_ptr(),
      hf.data_ptr(), hb.data_ptr(), dxf.data_ptr(), dgf.data_ptr(),
      dxb.data_ptr(), dgb.data_ptr(), cu.data_ptr(), cuc, S, C, T, dt,
      _lib.ptr(ws), nb, _lib.stream_of(dev)))


def scan_bidi_bwd_rowgrad(dyf: torch.Tensor, rsf: int, dyb: torch.Tensor,
                          rsb: int, gf: torch.Tensor, gb: torch.Tensor,
                          hf: torch.Tensor, hb: torch.Tensor,
                          dxf: torch.Tensor, dgf: torch.Tensor,
                          dxb: torch.Tensor, dgb: torch.Tensor,
                          cu: torch.Tensor,
                          num_channels: int | None = None) -> None:
  """Backward of both branches for gradients constant along time (one value
  per row, `rsf` / `rsb` elements apart, read from dyf / dyb.data_ptr())."""
  lib = _lib.load()
  dev = _lib.require_device(dyf, dyb, gf, gb, hf, hb, dxf, dgf, dxb, dgb, cu)
  _check_same(hf, gf, gb, hb, dxf, dgf, dxb, dgb)
  for d in (dyf, dyb):
    if d.dtype != hf.dtype:
      raise TypeError(f"dtype mismatch: {hf.dtype} vs {d.dtype}")
  dt = _lib.dtype_code(hf)
  cuc = _lib.cu_code(cu)
  cu = cu.contiguous()
  S, C, T = _geometry(hf, cu, num_channels)
  with _OnDevice(dev):
    ws, nb = _workspace(lib, dev, S, C, T, dt, 2, gf, gb, hf, hb, dxf, dgf,
                        dxb, dgb)
    _lib.check(lib.asc_scan_bidi_bwd_rowgrad(
      dyf.data_ptr(), int(rsf), dyb.data_ptr(), int(rsb), gf.data_ptr(),
      gb.data_ptr(), hf.data_ptr(), hb.data_ptr(), dxf.data_ptr(),
      dgf.data_ptr(), dxb.data_ptr(), dgb.data_ptr(), cu.data_ptr(), cuc, S,
      C, T, dt, _lib.ptr(ws), nb, _lib.stream_of(dev)))


def scan_bidi_bwd_any(dyf: torch.Tensor | None, dyb: torch.Tensor | None,
                      gf: torch.Tensor, gb: torch.Tensor, hf: torch.Tensor,
                      hb: torch.Tensor, dxf: torch.Tensor, dgf: torch.Tensor,
                      dxb: torch.Tensor, dgb: torch.Tensor, cu: torch.Tensor,
                      num_channels: int | None = None) -> None:
  """Bidirectional backward for any incoming gradient layouts.  None stands
  for a branch whose output received no gradient (zero).  When both
  gradients are constant along time (stride-0 expanded tensors, or None)
  they are read one value per row, unless the geometry runs the look-back
  walk for few items (tensors of different 16-byte phases); otherwise both
  are made contiguous, as the reference does (scan_eager.py:161,166)."""
  zero = None
  if dyf is None or dyb is None:
    zero = torch.zeros((), dtype=hf.dtype, device=hf.device)
  rsf = 0 if dyf is None else row_constant_stride(dyf, hf, num_channels)
  rsb = 0 if dyb is None else row_constant_stride(dyb, hb, num_channels)
  if rsf is not None and rsb is not None:
    lib = _lib.load()
    cu_c = cu.contiguous()
    S, C, T = _geometry(hf, cu_c, num_channels)
    if (_walk(lib, S, C, T, _lib.dtype_code(hf), 2) != _lib.WALK_LOOKBACK
        or _one_phase((gf, gb, hf, hb, dxf, dgf, dxb, dgb))):
      scan_bidi_bwd_rowgrad(zero if dyf is None else dyf, rsf,
                            zero if dyb is None else dyb, rsb, gf, gb, hf, hb,
                            dxf, dgf, dxb, dgb, cu_c, num_channels)
      return
  dyf = torch.zeros_like(hf) if dyf is None else dyf.contiguous()
  dyb = torch.zeros_like(hb) if dyb is None else dyb.contiguous()
  scan_bidi_bwd(dyf, dyb, gf, gb, hf, hb, dxf, dgf, dxb, dgb, cu,
                num_channels)


# ---------------------------------------------------------------------------
# recompute mode: the backward recomputes the forward states from its inputs
# ---------------------------------------------------------------------------

def checkpoint_shape(tokens: torch.Tensor, num_channels: int | None = None
                     ) -> tuple[int, int]:
  """[C, chunks per row] of the checkpoints of a [C, T] tensor (one fp32
  value per 4096 fp32 / 8192 fp16-bf16 elements of each row)."""
  C = int(num_channels) if num_channels is not None else (
    tokens.shape[0] if tokens.dim() == 2 else 1)
  if C <= 0 or tokens.numel() % C:
    raise ValueError(
      f"a tensor of {tokens.numel()} elements cannot hold {C} channels")
  T = tokens.numel() // C
  chunk = 4096 if tokens.dtype == torch.float32 else 8192
  return C, -(-T // chunk)


def scan_checkpoints(states: torch.Tensor, cu: torch.Tensor, reverse: bool,
                     num_channels: int | None = None) -> torch.Tensor:
  """The forward states the recompute backward starts each chunk from,
  sampled from a finished forward scan's output (see
  asc_scan_checkpoints)."""
  lib = _lib.load()
  dev = _lib.require_device(states, cu)
  _check_same(states)
  dt = _lib.dtype_code(states)
  cuc = _lib.cu_code(cu)
  cu = cu.contiguous()
  S, C, T = _geometry(states, cu, num_channels)
  ck = torch.empty(checkpoint_shape(states, C), dtype=torch.float32,
                   device=dev)
  assert ck.numel() == lib.asc_scan_checkpoint_elems(C, T, dt)
  with _OnDevice(dev):
    _lib.check(lib.asc_scan_checkpoints(
      states.data_ptr(), ck.data_ptr(), cu.data_ptr(), cuc, S, C, T, dt,
      1 if reverse else 0, _lib.stream_of(dev)))
  return ck


def recompute_in_kernel(gates: torch.Tensor, tokens: torch.Tensor,
                        cu: torch.Tensor, num_channels: int | None = None
                        ) -> bool:
  """Whether the recompute mode's backward runs the library's recompute
  kernels: 16-byte aligned tensors and a geometry whose workspace buys the
  chained walk (long segments, rows a whole number of chunks).  Other calls
  recompute the states with the forward scan into a temporary and run the
  plain backward: the library's per-item recompute walk is correct for any
  geometry but, measured on ragged segments shorter than a chunk (cfg3),
  4x slower than the forward plus the plain backward (1.70 against 0.25 +
  0.44 ms), and few-item problems run the look-back walk."""
  if gates.data_ptr() % 16 or tokens.data_ptr() % 16:
    return False
  S, C, T = _geometry(tokens, cu, num_channels)
  lib = _lib.load()
  return lib.asc_scan_workspace_walk(
    S, C, T, _lib.dtype_code(tokens), 1) == _lib.WALK_CHAINED


def scan_bwd_recompute(grad: torch.Tensor, gates: torch.Tensor,
                       tokens: torch.Tensor, ckpt: torch.Tensor | None,
                       d_tokens: torch.Tensor, d_gates: torch.Tensor,
                       cu: torch.Tensor, causal: bool,
                       num_channels: int | None = None) -> None:
  """Backward of a forward scan of (gates, tokens) without its states:
  asc_scan_bwd_recompute recomputes them from the checkpoints when
  recompute_in_kernel() says so (and checkpoints are given); otherwise the
  states are recomputed into a temporary with the forward scan and the plain
  backward runs.  A gradient constant along time is read one value per row;
  None stands for a zero gradient."""
  if grad is None:
    grad = tokens.new_zeros(()).expand_as(tokens)
  if ckpt is None or not recompute_in_kernel(gates, tokens, cu, num_channels):
    h = torch.empty_like(tokens)
    scan_fwd(gates, tokens, h, cu, reverse=not causal,
             num_channels=num_channels)
    scan_bwd_any(grad, gates, h, d_tokens, d_gates, cu, causal, num_channels)
    return
  scan_bwd_recompute_kernel(grad, gates, tokens, ckpt, d_tokens, d_gates, cu,
                            causal, num_channels)


def scan_bwd_recompute_kernel(grad: torch.Tensor, gates: torch.Tensor,
                              tokens: torch.Tensor, ckpt: torch.Tensor,
                              d_tokens: torch.Tensor, d_gates: torch.Tensor,
                              cu: torch.Tensor, causal: bool,
                              num_channels: int | None = None) -> None:
  """asc_scan_bwd_recompute for any geometry it accepts: the chained walk
  when the workspace buys it and every segment edge is chunk-aligned, else
  one workgroup per (segment, channel) item."""
  lib = _lib.load()
  rs = row_constant_stride(grad, tokens, num_channels)
  if rs is None:
    grad = grad.contiguous()
    rs = -1
  dev = _lib.require_device(grad, gates, tokens, ckpt, d_tokens, d_gates, cu)
  _check_same(tokens, gates, d_tokens, d_gates)
  if grad.dtype != tokens.dtype:
    raise TypeError(f"dtype mismatch: {tokens.dtype} vs {grad.dtype}")
  if rs < 0:
    _check_same(tokens, grad)
  dt = _lib.dtype_code(tokens)
  cuc = _lib.cu_code(cu)
  cu = cu.contiguous()
  S, C, T = _geometry(tokens, cu, num_channels)
  if (ckpt.dtype != torch.float32 or not ckpt.is_contiguous()
      or ckpt.numel() != lib.asc_scan_checkpoint_elems(C, T, dt)):
    raise ValueError("checkpoints do not match the tensors "
                     "(see scan_checkpoints)")
  with _OnDevice(dev):
    plain = rs >= 0 or d_tokens.data_ptr() != grad.data_ptr()
    ws, nb = _workspace(lib, dev, S, C, T, dt, 1) if plain else (None, 0)
    _lib.check(lib.asc_scan_bwd_recompute(
      grad.data_ptr(), int(rs), gates.data_ptr(), tokens.data_ptr(),
      ckpt.data_ptr(), d_tokens.data_ptr(), d_gates.data_ptr(), cu.data_ptr(),
      cuc, S, C, T, dt, 1 if causal else 0, _lib.ptr(ws), nb,
      _lib.stream_of(dev)))


def shift_pad(data: torch.Tensor, out: torch.Tensor, cu: torch.Tensor,
              pad_value: float, backward: bool, wrap: bool) -> None:
  """out <- segment-aware shift of a [C, L] tensor; data and out may have
  any (non-negative) strides, out must not overlap itself or data."""
  lib = _lib.load()
  dev = _lib.require_device(data, out, cu)
  if data.dim() != 2:
    raise ValueError(f"shift_pad expects a [C, BL] tensor, got {tuple(data.shape)}")
  if out.shape != data.shape:
    raise ValueError(f"size mismatch: {tuple(data.shape)} vs {tuple(out.shape)}")
  if out.dtype != data.dtype:
    raise TypeError(f"dtype mismatch: {data.dtype} vs {out.dtype}")
  dt = _lib.dtype_code(data)
  cuc = _lib.cu_code(cu)
  cu = cu.contiguous()
  C, L = data.shape
  with _OnDevice(dev):
    _lib.check(lib.asc_shift_pad_strided(
      data.data_ptr(), data.stride(0), data.stride(1), out.data_ptr(),
      out.stride(0), out.stride(1), cu.data_ptr(), cuc, cu.numel() - 1,
      C, L, dt, float(pad_value), 1 if backward else 0, 1 if wrap else 0,
      _lib.stream_of(dev)))
