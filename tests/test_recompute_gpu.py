"""Recompute mode: the backward recomputes the forward states from the
forward's inputs and per-chunk checkpoints instead of reading saved states.

* asc_scan_checkpoints: checkpoint (c, k) is the state adjacent to chunk k
  of row c on the side the forward scan comes from, when it lies in the
  segment of the chunk's first element in scan order, else 0 -- checked bit
  for bit against the states it samples.
* asc_scan_bwd_recompute against the fp64 oracle: d_tokens and d_gates of
  the oracle's states rounded to the storage type (the states a stored
  forward output holds), on the chained walk (aligned segments, one past the
  64-chunk checkpoint), on the per-item walk (unaligned and ragged segments,
  rows that are not a whole number of chunks, no workspace), dense and
  per-row gradients, both directions, with the bounded wait forced, in
  place of the gradient, and twice in a row (bit for bit: both walks
  compose in a fixed order).
* The autograd API with recompute_states=True: the same forward bits, the
  gradients within tolerance of the oracle and of the default mode, eager
  and compiled, causal and bidirectional, the few-item and misaligned
  geometries that recompute the states with the forward scan instead, and
  no [C, T] output kept alive between the forward and the backward.

Reference: scan_eager.py:42-47 (the states the reference saves),
_kernels.py:171-287 (the fused backward run on them).
"""

import numpy as np
import pytest
import torch

import associative_scan_triton as ast
from _helpers import (DEV, check_close, cu_of, grid_args, make, npf,
                      oracle_bwd, oracle_fwd)
from associative_scan_triton import _lib, _ops

pytestmark = pytest.mark.gpu


def _chunk(dtype):
  return 4096 if dtype == torch.float32 else 8192


def _stored(ref: np.ndarray, dtype) -> np.ndarray:
  """fp64 states rounded to the storage type (as a stored output holds)."""
  return npf(torch.from_numpy(ref).to(dtype))


def _ckpt_expected(h: np.ndarray, lens, reverse: bool, chunk: int):
  """The checkpoint definition, restated in numpy from the states."""
  C, T = h.shape
  cu = cu_of(lens)
  seg = np.full(T, -1)
  for s in range(len(lens)):
    seg[cu[s]:cu[s + 1]] = s
  kr = -(-T // chunk)
  out = np.zeros((C, kr))
  for k in range(kr):
    tf = min((k + 1) * chunk, T) - 1 if reverse else k * chunk
    tp = tf + 1 if reverse else tf - 1
    if 0 <= tp < T and seg[tf] >= 0 and seg[tp] == seg[tf]:
      out[:, k] = h[:, tp]
  return out


# name -> (dtype, C, lens in elements or chunk multiples, use workspace)
def _case(name):
  f32, bf16, f16 = torch.float32, torch.bfloat16, torch.float16
  CH4, CH8 = 4096, 8192
  return {
    "chained": (f32, 130, [2 * CH4, CH4, 3 * CH4], True),
    "chained-checkpoint": (f32, 130, [70 * CH4] + [CH4] * 4, True),
    "chained-bf16": (bf16, 130, [CH8, 2 * CH8], True),
    "chained-f16": (f16, 129, [3 * CH8], True),
    "unaligned": (f32, 130, [2 * CH4 + 8, CH4 - 8, 3 * CH4], True),
    "ragged": (f32, 40, [1, 7, 300, 5000, 1029, 16001, 10], True),
    "ragged-bf16": (bf16, 40, [3, 9000, 1, 20000, 4], True),
    "no-workspace": (f32, 130, [2 * CH4, CH4, 3 * CH4], False),
    # more segments than one wave surveys: the per-item walk's first
    # workgroup surveys them in two batches before the chained walk runs
    "chained-300": (f32, 2, [CH4 * (1 + i % 3) for i in range(300)], True),
  }[name]


CASES = ["chained", "chained-checkpoint", "chained-bf16", "chained-f16",
         "unaligned", "ragged", "ragged-bf16", "no-workspace", "chained-300"]


def _run_case(name, causal, grad_kind, spin=None, inplace=False):
  dtype, C, lens, use_ws = _case(name)
  T = sum(lens)
  lib = _lib.load()
  g, x, dy = make(lens, C, dtype, glo=0.5, n=3)
  if grad_kind == "rows":
    dy = torch.randn(C, 1, generator=torch.Generator().manual_seed(4)).to(
      dtype).expand(C, T)
  cu = torch.tensor(cu_of(lens), device=DEV)
  gd, xd = g.to(DEV), x.to(DEV)
  dyd = dy.to(DEV) if grad_kind == "dense" else dy[:, :1].to(DEV).expand(C, T)
  h = torch.empty_like(xd)
  _ops.scan_fwd(gd, xd, h, cu, reverse=not causal)
  ck = _ops.scan_checkpoints(h, cu, reverse=not causal)
  dx, dg = torch.empty_like(xd), torch.empty_like(xd)
  if inplace:
    dyd = dyd.contiguous()
    dx = dyd
  prev_ws = _ops.USE_WORKSPACE
  _ops.USE_WORKSPACE = use_ws
  prev = lib.asc_set_lookback_spin_limit(spin) if spin is not None else None
  try:
    _ops.scan_bwd_recompute_kernel(dyd, gd, xd, ck, dx, dg, cu, causal)
    torch.cuda.synchronize()
  finally:
    _ops.USE_WORKSPACE = prev_ws
    if prev is not None:
      lib.asc_set_lookback_spin_limit(prev)
  return dtype, C, lens, g, x, dy, h, ck, dx, dg


@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "anticausal"])
@pytest.mark.parametrize("grad_kind", ["dense", "rows"])
def test_recompute_backward_parity(name, causal, grad_kind):
  dtype, C, lens, g, x, dy, h, ck, dx, dg = _run_case(name, causal, grad_kind)
  rows = (list(range(C)) if C * sum(lens) <= 4_000_000 else
          sorted({r for r in (0, 1, 64, C - 1) if r < C}))
  h_st = _stored(oracle_fwd(g[rows], x[rows], lens, reverse=not causal), dtype)
  dx_ref, dg_ref = oracle_bwd(dy[rows], g[rows], h_st, lens, causal=causal)
  check_close(dx[rows], dx_ref, dtype, f"{name} dx")
  check_close(dg[rows], dg_ref, dtype, f"{name} dg")
  # the checkpoints are the states they sample, bit for bit
  exp = _ckpt_expected(npf(h[rows]), lens, not causal, _chunk(dtype))
  assert np.array_equal(npf(ck[rows]), exp)
  # and the plain backward on the stored states agrees to rounding
  dx2, dg2 = torch.empty_like(dx), torch.empty_like(dg)
  dyd = dy.to(DEV) if grad_kind == "dense" else dy.contiguous().to(DEV)
  _ops.scan_bwd(dyd, g.to(DEV), h, dx2, dg2,
                torch.tensor(cu_of(lens), device=DEV), causal)
  tol = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)
  sc = max(1.0, float(dx2.float().abs().mean()))
  torch.testing.assert_close(dx.float(), dx2.float(), rtol=tol["rtol"],
                             atol=tol["atol"] * sc)


@pytest.mark.parametrize("name", ["chained", "ragged"])
def test_recompute_backward_is_reproducible(name):
  a = _run_case(name, True, "dense")
  b = _run_case(name, True, "dense")
  assert torch.equal(a[8], b[8]) and torch.equal(a[9], b[9])


@pytest.mark.parametrize("name", ["chained", "chained-checkpoint"])
def test_recompute_chain_bounded_wait_fallback(name):
  """Spin limit 0: a chunk that finds a predecessor's slot empty composes its
  carry from the segment's inputs before it; still the oracle's values."""
  dtype, C, lens, g, x, dy, h, ck, dx, dg = _run_case(name, True, "dense", spin=0)
  rows = [0, 65, C - 1]
  h_st = _stored(oracle_fwd(g[rows], x[rows], lens), dtype)
  dx_ref, dg_ref = oracle_bwd(dy[rows], g[rows], h_st, lens)
  check_close(dx[rows], dx_ref, dtype, "dx")
  check_close(dg[rows], dg_ref, dtype, "dg")


@pytest.mark.parametrize("name", ["chained", "ragged-bf16"])
def test_recompute_backward_in_place_of_gradient(name):
  dtype, C, lens, g, x, dy, h, ck, dx, dg = _run_case(name, True, "dense",
                                                      inplace=True)
  rows = [0, C // 2, C - 1]
  h_st = _stored(oracle_fwd(g[rows], x[rows], lens), dtype)
  dx_ref, dg_ref = oracle_bwd(dy[rows], g[rows], h_st, lens)
  check_close(dx[rows], dx_ref, dtype, "dx over dy")
  check_close(dg[rows], dg_ref, dtype, "dg")


# ---------------------------------------------------------------------------
# autograd API
# ---------------------------------------------------------------------------

API_GEOMS = {
  "chained": (torch.float32, 130, [4096, 2 * 4096]),
  "ragged": (torch.float32, 80, [3000, 17, 5003]),
  "bf16": (torch.bfloat16, 130, [8192, 16384]),
  "few-items": (torch.float32, 3, [70001, 3, 20000]),
}


@pytest.mark.parametrize("geom", sorted(API_GEOMS))
@pytest.mark.parametrize("compiled", [False, True], ids=["eager", "compiled"])
@pytest.mark.parametrize("loss", ["sum", "dense"])
def test_scan_causal_recompute_mode(geom, compiled, loss):
  dtype, C, lens = API_GEOMS[geom]
  fn = ast.scan_causal_compiled if compiled else ast.scan_causal
  g, x, dy = make(lens, C, dtype, glo=0.5, n=3)
  T = sum(lens)
  args = grid_args(lens, C)
  if loss == "sum":
    dy = torch.ones(C, T, dtype=dtype)

  def run(rc):
    gd = g.to(DEV).requires_grad_(True)
    xd = x.to(DEV).requires_grad_(True)
    y = fn(gd, xd, args, recompute_states=rc)
    if loss == "sum":
      y.sum().backward()
    else:
      y.backward(dy.to(DEV))
    return y.detach(), gd.grad, xd.grad

  y1, dg1, dx1 = run(True)
  y0, dg0, dx0 = run(False)
  assert torch.equal(y1, y0)
  h_st = _stored(oracle_fwd(g, x, lens), dtype)
  dx_ref, dg_ref = oracle_bwd(dy, g, h_st, lens)
  check_close(dx1, dx_ref, dtype, "dx")
  check_close(dg1, dg_ref, dtype, "dg")
  check_close(dx0, dx_ref, dtype, "dx (default mode)")


@pytest.mark.parametrize("compiled", [False, True], ids=["eager", "compiled"])
@pytest.mark.parametrize("use", ["both", "fwd-only"])
def test_bidirectional_recompute_mode(compiled, use):
  lens, C, dtype = [4096, 2 * 4096], 130, torch.float32
  fn = (ast.scan_bidirectional_branched_compiled if compiled
        else ast.scan_bidirectional_branched)
  gf, xf, dyf = make(lens, C, dtype, seed=1, glo=0.5, n=3)
  gb, xb, dyb = make(lens, C, dtype, seed=2, glo=0.5, n=3)
  args = grid_args(lens, C)
  ts = [t.to(DEV).requires_grad_(True) for t in (gf, xf, gb, xb)]
  yf, yb = fn(*ts, args, recompute_states=True)
  if use == "both":
    torch.autograd.backward([yf, yb], [dyf.to(DEV), dyb.to(DEV)])
  else:
    yf.backward(dyf.to(DEV))
    dyb = torch.zeros_like(dyb)
  hf = _stored(oracle_fwd(gf, xf, lens), dtype)
  hb = _stored(oracle_fwd(gb, xb, lens, reverse=True), dtype)
  dxf, dgf = oracle_bwd(dyf, gf, hf, lens, causal=True)
  dxb, dgb = oracle_bwd(dyb, gb, hb, lens, causal=False)
  check_close(ts[0].grad, dgf, dtype, "dg fwd")
  check_close(ts[1].grad, dxf, dtype, "dx fwd")
  check_close(ts[2].grad, dgb, dtype, "dg bwd")
  check_close(ts[3].grad, dxb, dtype, "dx bwd")


def test_recompute_misaligned_views_use_the_forward():
  """Tensors that are not 16-byte aligned: the backward recomputes the
  states with the forward scan into a temporary (same results)."""
  lens, C = [3000, 5001], 80
  T = sum(lens)
  g, x = make(lens, C, glo=0.5)
  big_g = torch.empty(C * T + 1, device=DEV)
  big_x = torch.empty(C * T + 1, device=DEV)
  gv = big_g[1:].view(C, T)
  xv = big_x[1:].view(C, T)
  gv.copy_(g.to(DEV))
  xv.copy_(x.to(DEV))
  cu = torch.tensor(cu_of(lens), device=DEV)
  assert not _ops.recompute_in_kernel(gv, xv, cu)
  gv.requires_grad_(True)
  xv.requires_grad_(True)
  y = ast.scan_causal(gv, xv, grid_args(lens, C), recompute_states=True)
  y.sum().backward()
  h_st = _stored(oracle_fwd(g, x, lens), torch.float32)
  dx_ref, dg_ref = oracle_bwd(torch.ones(C, T), g, h_st, lens)
  check_close(xv.grad, dx_ref, torch.float32, "dx")
  check_close(gv.grad, dg_ref, torch.float32, "dg")


def test_recompute_keeps_no_output_alive():
  """Between the forward and the backward the default mode keeps the
  [C, T] output for the backward; recompute mode keeps only the
  checkpoints (and the inputs, which the caller holds anyway)."""
  lens, C = [8 * 4096] * 4, 256
  T = sum(lens)
  g, x = make(lens, C, glo=0.5)
  args = grid_args(lens, C)
  gd = g.to(DEV).requires_grad_(True)
  xd = x.to(DEV).requires_grad_(True)
  nbytes = C * T * 4
  held = {}
  for rc in (False, True):
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    loss = ast.scan_causal(gd, xd, args, recompute_states=rc).sum()
    torch.cuda.synchronize()
    held[rc] = torch.cuda.memory_allocated() - base
    loss.backward()
    gd.grad = xd.grad = None
    del loss
  assert held[False] >= nbytes
  assert held[True] < nbytes // 100
