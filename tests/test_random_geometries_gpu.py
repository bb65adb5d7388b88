"""Seeded random geometries through every walk, against the fp64 oracle.

Each case draws a dtype, a row count, segment lengths from a mixture (single
elements, empty segments, short segments that take two items per wave,
lengths around the 16-byte vector and the sub-tile, multiples of the
chained walk's chunk with and without an element off the grid, long
segments), with and without the workspace, and runs the forward in both
directions, the backward of each, the two-branch calls and the row-constant
gradient; sampled rows are compared with the oracle.  In 30% of the cases
the single-branch tensors are views at independent element offsets 0-7
(their phases on the 16-byte grid differ, as with sliced inputs), and so
are the two-branch tensors.  The walk
a case takes follows from its geometry (tree, look-back, chained with its
one-wave partner, group, one-wave, workgroup), so the draws cover their
mixtures as well.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import DEV, check_close, cu_of, make, npf, oracle_bwd, oracle_fwd
from associative_scan_triton import _ops

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
NCASES = 96


def _chunk(dtype):
  return 4096 if dtype == torch.float32 else 8192


def _draw(seed):
  rng = np.random.default_rng(seed)
  dtype = DTYPES[rng.integers(3)]
  CH = _chunk(dtype)
  kind = rng.choice(["short", "mixed", "chunky", "long", "tiny", "tiny"])
  S = int(rng.integers(1, 24))
  lens = []
  for _ in range(S):
    r = rng.random()
    if kind == "tiny":
      n = int(rng.integers(0, 140)) if r < 0.9 else int(rng.integers(140, 600))
    elif kind == "short":
      n = int(rng.integers(0, 300)) if r < 0.9 else int(rng.integers(300, 2000))
    elif kind == "chunky":
      n = CH * int(rng.integers(1, 4)) + (int(rng.integers(-3, 4)) if r < 0.3 else 0)
    elif kind == "long":
      n = int(rng.integers(1, 60000))
    else:
      n = int(rng.choice([0, 1, 3, 4, 255, 256, 257, 511, 513, 1000, 4097,
                          CH, 2 * CH, int(rng.integers(1, 5000))]))
    lens.append(max(n, 0))
  if sum(lens) == 0:
    lens[0] = 1
  budget = 6_000_000 // sum(lens)
  C = int(max(1, min(budget, rng.choice([1, 3, 64, 129, 200]))))
  use_ws = bool(rng.random() < 0.7)
  return dtype, lens, C, use_ws


def _place(t, off):
  """t on the device; off >= 0: as a view that starts off elements into a
  fresh buffer (a pointer off the 16-byte grid for off not a multiple of the
  vector)."""
  if off < 0:
    return t.to(DEV)
  buf = torch.zeros(t.numel() + 16, dtype=t.dtype, device=DEV)
  v = buf[off:off + t.numel()].view(t.shape)
  v.copy_(t.to(DEV))
  return v


@pytest.mark.parametrize("seed", range(NCASES))
def test_random_geometry(seed):
  dtype, lens, C, use_ws = _draw(seed)
  T = sum(lens)
  g, x, dy = make(lens, C, dtype, seed=seed, glo=0.5, n=3)
  orng = np.random.default_rng(seed + 77)
  mis = bool(orng.random() < 0.3)
  offs = [int(v) for v in orng.integers(0, 8, 6)] if mis else [-1] * 6
  gd, xd, dyd = _place(g, offs[0]), _place(x, offs[1]), _place(dy, offs[2])
  cu = torch.tensor(cu_of(lens), device=DEV)
  rows = sorted({0, C // 2, C - 1})
  prev = _ops.USE_WORKSPACE
  _ops.USE_WORKSPACE = use_ws
  try:
    for rev in (False, True):
      h = _place(torch.zeros_like(x), offs[3])
      _ops.scan_fwd(gd, xd, h, cu, reverse=rev)
      dx, dg = _place(torch.zeros_like(x), offs[4]), _place(torch.zeros_like(x), offs[5])
      _ops.scan_bwd(dyd, gd, h, dx, dg, cu, causal=not rev)
      torch.cuda.synchronize()
      for r in rows:
        sl = slice(r, r + 1)
        what = f"seed {seed} {dtype} C={C} S={len(lens)} T={T} ws={use_ws} rev={rev} offs={offs} row {r}"
        check_close(h[sl], oracle_fwd(g[sl], x[sl], lens, reverse=rev), dtype,
                    "h " + what)
        dx_ref, dg_ref = oracle_bwd(dy[sl], g[sl], npf(h[sl]), lens,
                                    causal=not rev)
        check_close(dx[sl], dx_ref, dtype, "dx " + what)
        check_close(dg[sl], dg_ref, dtype, "dg " + what)
    bo = [int(v) for v in orng.integers(0, 8, 9)] if mis else [-1] * 9
    gd, xd, dyd = _place(g, bo[0]), _place(x, bo[1]), _place(dy, bo[2])
    # both branches in one call, and the gradient of out.sum() (one value
    # per row) against the same gradient materialised
    hf, hb = _place(torch.zeros_like(x), bo[3]), _place(torch.zeros_like(x), bo[4])
    _ops.scan_bidi_fwd(gd, xd, gd, dyd, hf, hb, cu)
    outs = [_place(torch.zeros_like(x), bo[5 + i]) for i in range(4)]
    _ops.scan_bidi_bwd(dyd, xd, gd, gd, hf, hb, *outs, cu)
    ones = torch.ones(C, dtype=dtype, device=DEV)
    dx1, dg1, dx2, dg2 = (torch.empty_like(xd) for _ in range(4))
    _ops.scan_bwd_rowgrad(ones, 1, gd, hf, dx1, dg1, cu, True)
    _ops.scan_bwd(torch.ones_like(xd), gd, hf, dx2, dg2, cu, causal=True)
    torch.cuda.synchronize()
    if mis:
      # tensors of different phases may take the look-back walk, whose last
      # bits can differ between two calls
      tol = 1e-5 if dtype == torch.float32 else 1e-2
      for a, b in ((dx1, dx2), (dg1, dg2)):
        sc = max(1.0, float(b.float().abs().mean()))
        torch.testing.assert_close(a.float(), b.float(), rtol=tol, atol=tol * sc)
    else:
      assert torch.equal(dx1, dx2) and torch.equal(dg1, dg2), f"seed {seed}"
    for r in rows:
      sl = slice(r, r + 1)
      what = f"seed {seed} two-branch row {r}"
      check_close(hf[sl], oracle_fwd(g[sl], x[sl], lens), dtype, "hf " + what)
      check_close(hb[sl], oracle_fwd(g[sl], dy[sl], lens, reverse=True), dtype,
                  "hb " + what)
      dxf, dgf = oracle_bwd(dy[sl], g[sl], npf(hf[sl]), lens, causal=True)
      dxb, dgb = oracle_bwd(x[sl], g[sl], npf(hb[sl]), lens, causal=False)
      check_close(outs[0][sl], dxf, dtype, "dxf " + what)
      check_close(outs[1][sl], dgf, dtype, "dgf " + what)
      check_close(outs[2][sl], dxb, dtype, "dxb " + what)
      check_close(outs[3][sl], dgb, dtype, "dgb " + what)
  finally:
    _ops.USE_WORKSPACE = prev


@pytest.mark.parametrize("seed", range(1000, 1032))
def test_random_recompute_geometry(seed):
  """The recompute backward (asc_scan_bwd_recompute, whichever walk it takes)
  on the same draws, one direction and a dense or row-constant gradient per
  seed, against the oracle; rows a whole number of 16-byte vectors (its
  contract), except every tenth seed, which must be refused."""
  from associative_scan_triton._lib import AscError
  from test_recompute_gpu import _chunk as _rc_chunk, _ckpt_expected, _stored
  dtype, lens, C, use_ws = _draw(seed)
  if seed % 10:
    lens[-1] += (-sum(lens)) % (4 if dtype == torch.float32 else 8)
  T = sum(lens)
  g, x, dy = make(lens, C, dtype, seed=seed, glo=0.5, n=3)
  gd, xd = g.to(DEV), x.to(DEV)
  cu = torch.tensor(cu_of(lens), device=DEV)
  rows = sorted({0, C // 2, C - 1})
  rng = np.random.default_rng(seed + 5)
  causal = bool(rng.random() < 0.5)
  rowgrad = bool(rng.random() < 0.3)
  if rowgrad:
    dy = torch.randn(C, 1, generator=torch.Generator().manual_seed(seed)).to(
      dtype).expand(C, T)
    dyd = dy[:, :1].to(DEV).expand(C, T)
  else:
    dyd = dy.to(DEV)
  h = torch.empty_like(xd)
  _ops.scan_fwd(gd, xd, h, cu, reverse=not causal)
  ck = _ops.scan_checkpoints(h, cu, reverse=not causal)
  dx, dg = torch.empty_like(xd), torch.empty_like(xd)
  prev = _ops.USE_WORKSPACE
  _ops.USE_WORKSPACE = use_ws
  try:
    if T % (4 if dtype == torch.float32 else 8):
      with pytest.raises(AscError, match="aligned"):
        _ops.scan_bwd_recompute_kernel(dyd, gd, xd, ck, dx, dg, cu, causal)
      return
    _ops.scan_bwd_recompute_kernel(dyd, gd, xd, ck, dx, dg, cu, causal)
    torch.cuda.synchronize()
  finally:
    _ops.USE_WORKSPACE = prev
  what = (f"seed {seed} {dtype} C={C} S={len(lens)} T={T} ws={use_ws} "
          f"causal={causal} rowgrad={rowgrad}")
  h_st = _stored(oracle_fwd(g[rows], x[rows], lens, reverse=not causal), dtype)
  dx_ref, dg_ref = oracle_bwd(dy[rows], g[rows], h_st, lens, causal=causal)
  check_close(dx[rows], dx_ref, dtype, "dx " + what)
  check_close(dg[rows], dg_ref, dtype, "dg " + what)
  exp = _ckpt_expected(npf(h[rows]), lens, not causal, _rc_chunk(dtype))
  assert np.array_equal(npf(ck[rows]), exp), "checkpoints " + what


@pytest.mark.parametrize("seed", range(2000, 2032))
def test_random_shift_pad_geometry(seed):
  """shift_pad on the same draws (empty segments made one element long),
  contiguous, at element offsets or transposed (strides (1, C)), either edge
  rule, int32 or int64 cu_seqlens, against the oracle bit for bit; nothing
  outside an offset output view is written."""
  from oracle import oracle
  dtype, lens, C, _ = _draw(seed)
  lens = [max(n, 1) for n in lens]
  L = sum(lens)
  C = min(C, max(1, 2_000_000 // L))
  rng = np.random.default_rng(seed + 11)
  backward, wrap = bool(rng.random() < 0.5), bool(rng.random() < 0.5)
  pad = float(rng.choice([0.0, 1.0, -2.5]))
  layout = rng.choice(["contig", "offset", "transposed"])
  data = torch.randn(C, L, generator=torch.Generator().manual_seed(seed)).to(dtype)
  cu_np = cu_of(lens)
  cu = torch.tensor(cu_np, device=DEV,
                    dtype=torch.int32 if rng.random() < 0.5 else torch.int64)
  oo = 0
  if layout == "offset":
    od, oo = int(rng.integers(0, 8)), int(rng.integers(0, 8))
    dbuf = torch.zeros(C * L + 8, dtype=dtype, device=DEV)
    obuf = torch.full((C * L + 8,), 7.0, dtype=dtype, device=DEV)
    dv = dbuf[od:od + C * L].view(C, L)
    dv.copy_(data.to(DEV))
    ov = obuf[oo:oo + C * L].view(C, L)
  elif layout == "transposed":
    dv = data.t().contiguous().to(DEV).t()
    ov = torch.empty(L, C, dtype=dtype, device=DEV).t()
  else:
    dv = data.to(DEV)
    ov = torch.empty_like(dv)
  _ops.shift_pad(dv, ov, cu, pad, backward=backward, wrap=wrap)
  ref = oracle.shift_pad(npf(data), cu_np, pad, backward, wrap=wrap)
  assert torch.equal(ov.cpu(), torch.from_numpy(ref).to(dtype)), (
    f"seed {seed} {dtype} C={C} L={L} {layout} backward={backward} wrap={wrap}")
  if layout == "offset":
    assert torch.all(obuf[:oo] == 7.0) and torch.all(obuf[oo + C * L:] == 7.0)


@pytest.mark.parametrize("seed", range(3000, 3024))
def test_random_public_api(seed):
  """The public autograd functions (eager and compiled, causal and
  bidirectional, with and without recompute_states) on the same draws, with
  a loss of out.sum(), row-weighted sums or a dense gradient, against the
  oracle on sampled rows."""
  import associative_scan_triton as ast
  from _helpers import grid_args
  dtype, lens, C, _ = _draw(seed)
  T = sum(lens)
  rng = np.random.default_rng(seed + 3)
  bidi = bool(rng.random() < 0.4)
  compiled = bool(rng.random() < 0.5)
  rec = bool(rng.random() < 0.3)
  loss = rng.choice(["sum", "rowweights", "dense"])
  g, x, x2 = make(lens, C, dtype, seed=seed, glo=0.5, n=3)
  g2 = g.clone()
  args = grid_args(lens, C, cu_dtype=torch.int64 if rng.random() < 0.5 else torch.int32)
  w = torch.rand(C, generator=torch.Generator().manual_seed(seed)).to(dtype)
  dense = torch.randn(C, T, generator=torch.Generator().manual_seed(seed + 1)).to(dtype)
  def grad_of(y):
    if loss == "sum":
      return torch.ones(C, T, dtype=dtype)
    if loss == "rowweights":
      return w[:, None].expand(C, T).contiguous()
    return dense
  def back(y):
    if loss == "sum":
      return y.sum()
    if loss == "rowweights":
      return (y.sum(-1) * w.to(DEV)).sum()
    return (y * dense.to(DEV)).sum()
  tens = [t.to(DEV).requires_grad_(True) for t in ((g, x, g2, x2) if bidi else (g, x))]
  rows = sorted({0, C // 2, C - 1})
  what = f"seed {seed} {dtype} C={C} S={len(lens)} T={T} bidi={bidi} compiled={compiled} rec={rec} loss={loss}"
  if bidi:
    fn = ast.scan_bidirectional_branched_compiled if compiled else ast.scan_bidirectional_branched
    yf, yb = fn(*tens, args, recompute_states=rec)
    (back(yf) + back(yb)).backward()
    dyf = grad_of(yf)
    for r in rows:
      sl = slice(r, r + 1)
      check_close(yf.detach()[sl], oracle_fwd(g[sl], x[sl], lens), dtype, "yf " + what)
      check_close(yb.detach()[sl], oracle_fwd(g2[sl], x2[sl], lens, reverse=True), dtype, "yb " + what)
      dxr, dgr = oracle_bwd(dyf[sl], g[sl], npf(yf.detach()[sl]), lens, causal=True)
      check_close(tens[1].grad[sl], dxr, dtype, "dxf " + what)
      check_close(tens[0].grad[sl], dgr, dtype, "dgf " + what)
      dxr, dgr = oracle_bwd(dyf[sl], g2[sl], npf(yb.detach()[sl]), lens, causal=False)
      check_close(tens[3].grad[sl], dxr, dtype, "dxb " + what)
      check_close(tens[2].grad[sl], dgr, dtype, "dgb " + what)
  else:
    fn = ast.scan_causal_compiled if compiled else ast.scan_causal
    y = fn(*tens, args, recompute_states=rec)
    back(y).backward()
    dy = grad_of(y)
    for r in rows:
      sl = slice(r, r + 1)
      check_close(y.detach()[sl], oracle_fwd(g[sl], x[sl], lens), dtype, "y " + what)
      dxr, dgr = oracle_bwd(dy[sl], g[sl], npf(y.detach()[sl]), lens, causal=True)
      check_close(tens[1].grad[sl], dxr, dtype, "dx " + what)
      check_close(tens[0].grad[sl], dgr, dtype, "dg " + what)
