"""GPU tests of the public API's own paths on the workspace walks.

* Gradients constant along time (``out.sum().backward()``), which autograd
  hands over as a stride-0 expanded tensor, on chunk-aligned geometries with
  more than 128 (segment, channel) items: the backward runs the chained
  walk's row-gradient kernels (one value per row, no materialised copy).
  They must match the dense-gradient chained kernels bit for bit (both
  compose carries in the same fixed order) and the fp64 oracle.
* In-place forward calls (``forward_scan_full(..., TESTING=False)`` with
  ``tokens_out=None``, kernel objects with ``INPLACE=True``) and an
  in-place backward (d_tokens over the gradient) on geometries whose
  out-of-place calls take the chained or look-back walk, with the
  bounded-wait fallback at its default and forced on every poll.
* Few-item problems (the tree walk) repeat bit for bit, by default and in
  deterministic mode; its bounded-wait fallback and the look-back walk (for
  tensors of different 16-byte phases) agree with the oracle.

Reference: scan_eager.py:50-64 (backward of grad_output.contiguous()),
tests/test_scan_causal.py:52-71 (out.sum() losses), _dispatcher.py:35-37
and _kernels.py:77-81 (in-place writes).
"""

import numpy as np
import pytest
import torch

import associative_scan_triton as ast
from _helpers import (DEV, check_close, cu_of, grid_args, make, npf,
                      oracle_bwd, oracle_fwd)
from associative_scan_triton import _lib, _ops

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
DT_IDS = ["f32", "f16", "bf16"]


def _chunk(dtype):
  """Elements per chained chunk: 4096 fp32, 8192 fp16/bf16."""
  return 4096 if dtype == torch.float32 else 8192


class _Counter:
  """Counts the calls of an _ops function while the test runs."""

  def __init__(self, monkeypatch, name):
    self.n = 0
    orig = getattr(_ops, name)

    def wrapped(*a, **k):
      self.n += 1
      return orig(*a, **k)

    monkeypatch.setattr(_ops, name, wrapped)


# segment lengths for a chunk of CH elements: one to three chunks per
# segment; a segment of 70 chunks (past the 64-chunk checkpoint) beside four
# one-chunk segments; two segments with an edge off the chunk grid (the
# one-wave walk takes them) beside a chunk-aligned one
GEOMS = {"short": lambda CH: [2 * CH, CH, 3 * CH],
         "checkpoint": lambda CH: [70 * CH, CH, CH, CH, CH],
         "mixed": lambda CH: [2 * CH + 5, CH - 5, 3 * CH]}


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("geom", sorted(GEOMS))
@pytest.mark.parametrize("compiled", [False, True], ids=["eager", "compiled"])
def test_time_constant_gradient_chained(dtype, geom, compiled, monkeypatch):
  C = 130
  lens = GEOMS[geom](_chunk(dtype))
  T = sum(lens)
  lib = _lib.load()
  assert lib.asc_scan_workspace_walk(len(lens), C, T, _lib.dtype_code(
    torch.empty((), dtype=dtype)), 1) == _lib.WALK_CHAINED
  fn = ast.scan_causal_compiled if compiled else ast.scan_causal
  g, x = make(lens, C, dtype, glo=0.5)
  args = grid_args(lens, C)
  w = torch.rand(C, generator=torch.Generator().manual_seed(3)).to(dtype).to(DEV)
  rowgrad = _Counter(monkeypatch, "scan_bwd_rowgrad")

  def grads(loss_of):
    gd = g.to(DEV).requires_grad_(True)
    xd = x.to(DEV).requires_grad_(True)
    y = fn(gd, xd, args)
    loss_of(y)
    return y.detach(), gd.grad, xd.grad

  rows = [0, 64, C - 1]
  for loss_of, dense in (
      (lambda y: y.sum().backward(), torch.ones(C, T, dtype=dtype, device=DEV)),
      (lambda y: (y.sum(-1) * w).sum().backward(),
       w[:, None].expand(C, T).contiguous())):
    n0 = rowgrad.n
    y1, dg1, dx1 = grads(loss_of)
    assert rowgrad.n == n0 + 1, "the time-constant gradient was materialised"
    y2, dg2, dx2 = grads(lambda y: y.backward(dense))
    assert rowgrad.n == n0 + 1
    assert torch.equal(y1, y2)
    assert torch.equal(dx1, dx2) and torch.equal(dg1, dg2)
    for r in rows:
      sl = slice(r, r + 1)
      check_close(y1[sl], oracle_fwd(g[sl], x[sl], lens), dtype, f"h row {r}")
      dx_ref, dg_ref = oracle_bwd(dense[sl].cpu(), g[sl], npf(y1[sl]), lens)
      check_close(dx1[sl], dx_ref, dtype, f"dx row {r}")
      check_close(dg1[sl], dg_ref, dtype, f"dg row {r}")
    # segment heads of the forward are exact
    heads = torch.tensor(cu_of(lens)[:-1], device=DEV)
    assert torch.equal(y1[:, heads].cpu(), x[:, heads.cpu()])


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("compiled", [False, True], ids=["eager", "compiled"])
@pytest.mark.parametrize("use", ["both", "fwd-only"])
def test_bidi_time_constant_gradient_chained(dtype, compiled, use, monkeypatch):
  """(out_f.sum() + out_b.sum()).backward() and out_f.sum().backward() (the
  reverse branch gets no gradient) on a chunk-aligned two-branch geometry:
  both branches take the chained row-gradient kernels; bit for bit equal to
  the dense gradients and within tolerance of the oracle."""
  C = 130
  CH = _chunk(dtype)
  lens = [CH, 2 * CH]
  T = sum(lens)
  lib = _lib.load()
  assert lib.asc_scan_workspace_walk(len(lens), C, T, _lib.dtype_code(
    torch.empty((), dtype=dtype)), 2) == _lib.WALK_CHAINED
  fn = (ast.scan_bidirectional_branched_compiled if compiled
        else ast.scan_bidirectional_branched)
  gf, xf = make(lens, C, dtype, seed=1, glo=0.5)
  gb, xb = make(lens, C, dtype, seed=2, glo=0.5)
  args = grid_args(lens, C)
  rowgrad = _Counter(monkeypatch, "scan_bidi_bwd_rowgrad")

  def run(loss_of):
    ts = [t.to(DEV).requires_grad_(True) for t in (gf, xf, gb, xb)]
    yf, yb = fn(*ts, args)
    loss_of(yf, yb)
    return (yf.detach(), yb.detach()), [t.grad for t in ts]

  ones = torch.ones(C, T, dtype=dtype, device=DEV)
  zeros = torch.zeros(C, T, dtype=dtype, device=DEV)
  if use == "both":
    loss_of, dyf, dyb = (lambda a, b: (a.sum() + b.sum()).backward()), ones, ones
  else:
    loss_of, dyf, dyb = (lambda a, b: a.sum().backward()), ones, zeros
  (yf, yb), got = run(loss_of)
  assert rowgrad.n == 1
  _, ref = run(lambda a, b: torch.autograd.backward([a, b], [dyf, dyb]))
  assert rowgrad.n == 1
  for a, b in zip(got, ref):
    assert torch.equal(a, b)
  for r in (0, 64, C - 1):
    sl = slice(r, r + 1)
    dxf, dgf = oracle_bwd(dyf[sl].cpu(), gf[sl], npf(yf[sl]), lens, causal=True)
    dxb, dgb = oracle_bwd(dyb[sl].cpu(), gb[sl], npf(yb[sl]), lens, causal=False)
    check_close(got[0][sl], dgf, dtype, "dg fwd")
    check_close(got[1][sl], dxf, dtype, "dx fwd")
    check_close(got[2][sl], dgb, dtype, "dg bwd")
    check_close(got[3][sl], dxb, dtype, "dx bwd")


# ---------------------------------------------------------------------------
# in-place calls on the workspace walks' geometries
# ---------------------------------------------------------------------------

# (dtype, C, lens): chained walk out of place (130 rows of chunk-aligned
# segments), look-back walk out of place (few items)
INPLACE_GEOMS = [
  (torch.float32, 130, [2 * 4096, 4096]),
  (torch.bfloat16, 130, [8192, 2 * 8192]),
  (torch.float32, 5, [5000, 3000]),
  (torch.bfloat16, 3, [70000, 1, 20000]),
]


@pytest.mark.parametrize("geom", INPLACE_GEOMS,
                         ids=["chained-f32", "chained-bf16", "lookback-f32",
                              "lookback-bf16"])
@pytest.mark.parametrize("spin", [None, 0], ids=["default-wait", "no-wait"])
@pytest.mark.parametrize("reverse", [False, True], ids=["causal", "reverse"])
def test_inplace_forward_on_workspace_geometries(geom, spin, reverse):
  dtype, C, lens = geom
  S, T = len(lens), sum(lens)
  lib = _lib.load()
  assert lib.asc_scan_workspace_walk(S, C, T, _lib.dtype_code(
    torch.empty((), dtype=dtype)), 1) in (_lib.WALK_CHAINED, _lib.WALK_LOOKBACK)
  g, x = make(lens, C, dtype, glo=0.5)
  h_ref = oracle_fwd(g, x, lens, reverse=reverse)
  args = grid_args(lens, C)
  cu = args["cu_seqlens"]
  prev = lib.asc_set_lookback_spin_limit(spin) if spin is not None else None
  try:
    # forward_scan_full: tokens_out=None writes h over the tokens
    gd, xd = g.to(DEV), x.to(DEV)
    ast.forward_scan_full(gd, xd, cu, args["grid"], REVERSE=reverse,
                          CHUNK_SIZE=128, TESTING=False)
    check_close(xd, h_ref, dtype, "forward_scan_full in place")
    assert torch.equal(gd.cpu(), g)
    # kernel object with INPLACE=True, TESTING=False
    gd, xd = g.to(DEV), x.to(DEV)
    ast.forward_scan_onepass_pipelined[(S, C)](
      gates_ptr=gd, tokens_ptr=xd, tokens_out_ptr=None, cu_seqlens_ptr=cu,
      REVERSE=reverse, CHUNK_SIZE=128, TESTING=False, INPLACE=True)
    check_close(xd, h_ref, dtype, "kernel object in place")
    # out of place on the same geometry (the workspace walk) agrees
    gd, xd = g.to(DEV), x.to(DEV)
    h = torch.empty_like(xd)
    ast.forward_scan_full(gd, xd, cu, args["grid"], REVERSE=reverse,
                          CHUNK_SIZE=128, TESTING=False, tokens_out=h)
    check_close(h, h_ref, dtype, "out of place")
    # backward with d_tokens over the gradient
    dy = make(lens, C, dtype, seed=11, n=2)[1]
    dx_ref, dg_ref = oracle_bwd(dy, g, npf(h), lens, causal=not reverse)
    dyd = dy.to(DEV)
    dg = torch.empty_like(dyd)
    ast.backward_scan_fused_full(dyd, gd, h, dyd, dg, cu, args["grid"],
                                 CHUNK_SIZE=128, CAUSAL=not reverse)
    check_close(dyd, dx_ref, dtype, "dx in place of dy")
    check_close(dg, dg_ref, dtype, "dg")
  finally:
    if prev is not None:
      lib.asc_set_lookback_spin_limit(prev)


def test_overlapping_outputs_are_refused():
  """An output over another input than its own is an argument error, raised
  before anything is launched."""
  lens, C = [300, 200], 4
  g, x = make(lens, C)
  gd, xd = g.to(DEV), x.to(DEV)
  cu = torch.tensor(cu_of(lens), device=DEV)
  with pytest.raises(_lib.AscError, match="invalid argument"):
    _ops.scan_fwd(gd, xd, gd, cu, reverse=False)
  dx = torch.empty_like(gd)
  with pytest.raises(_lib.AscError, match="invalid argument"):
    _ops.scan_bwd(xd, gd, xd, dx, dx, cu, causal=True)
  assert torch.equal(gd.cpu(), g) and torch.equal(xd.cpu(), x)


# ---------------------------------------------------------------------------
# deterministic mode
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("mode", ["default", "deterministic"])
def test_few_items_repeat_bitwise(dtype, mode):
  """A few-item geometry (the tree walk: carries composed in an order fixed
  by the data) gives identical bits on repeated forward + backward calls
  through the autograd API, by default and under
  torch.use_deterministic_algorithms(True), within tolerance of the
  oracle."""
  lens, C = [300001, 70000, 5], 2
  T = sum(lens)
  lib = _lib.load()
  code = _lib.dtype_code(torch.empty((), dtype=dtype))
  assert lib.asc_scan_workspace_walk(len(lens), C, T, code, 1) == _lib.WALK_LOOKBACK
  g, x, dy = make(lens, C, dtype, glo=0.5, n=3)
  args = grid_args(lens, C)
  prev = torch.are_deterministic_algorithms_enabled()
  torch.use_deterministic_algorithms(mode == "deterministic")
  try:
    runs = []
    for _ in range(3):
      gd = g.to(DEV).requires_grad_(True)
      xd = x.to(DEV).requires_grad_(True)
      y = ast.scan_causal(gd, xd, args)
      y.backward(dy.to(DEV))
      runs.append((y.detach(), gd.grad, xd.grad))
  finally:
    torch.use_deterministic_algorithms(prev)
  for other in runs[1:]:
    for a, b in zip(runs[0], other):
      assert torch.equal(a, b)
  y, dg, dx = runs[0]
  check_close(y, oracle_fwd(g, x, lens), dtype, "h")
  dx_ref, dg_ref = oracle_bwd(dy, g, npf(y), lens)
  check_close(dx, dx_ref, dtype, "dx")
  check_close(dg, dg_ref, dtype, "dg")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("rev", [False, True], ids=["causal", "reverse"])
def test_tree_walk_bits_survive_fallback(dtype, rev):
  """The tree walk and the workspace-free walk that recomputes a call whose
  bounded wait expired (forced with a spin limit of 0) agree with the oracle,
  and the tree walk's bits do not depend on the launch: two calls with the
  default spin limit are identical.  Tensors offset by one element from the
  others (a different 16-byte phase) take the look-back walk, which must
  agree with the oracle too."""
  lens, C = [200000, 3, 1, 77777], 3
  T = sum(lens)
  g, x, dy = make(lens, C, dtype, glo=0.5, n=3)
  gd, xd, dyd = g.to(DEV), x.to(DEV), dy.to(DEV)
  cu = torch.tensor(cu_of(lens), device=DEV)
  lib = _lib.load()

  def run(spin=None, offset=False):
    prev = lib.asc_set_lookback_spin_limit(spin) if spin is not None else None
    try:
      if offset:
        hb = torch.empty(C * T + 1, dtype=dtype, device=DEV)
        h = hb[1:].view(C, T)
      else:
        h = torch.empty_like(xd)
      _ops.scan_fwd(gd, xd, h, cu, rev)
      dx, dg = torch.empty_like(gd), torch.empty_like(gd)
      _ops.scan_bwd(dyd, gd, h.contiguous(), dx, dg, cu, causal=not rev)
      torch.cuda.synchronize()
      return h.clone(), dx, dg
    finally:
      if prev is not None:
        lib.asc_set_lookback_spin_limit(prev)

  a, b = run(), run()
  for u, w in zip(a, b):
    assert torch.equal(u, w)
  h_ref = oracle_fwd(g, x, lens, reverse=rev)
  for label, res in (("tree", a), ("fallback", run(spin=0)),
                     ("look-back", run(offset=True))):
    h, dx, dg = res
    check_close(h, h_ref, dtype, f"h ({label})")
    dx_ref, dg_ref = oracle_bwd(dy, g, npf(h), lens, causal=not rev)
    check_close(dx, dx_ref, dtype, f"dx ({label})")
    check_close(dg, dg_ref, dtype, f"dg ({label})")


# ---------------------------------------------------------------------------
# shift_pad on strided inputs (no copy; _shift_pad.py:140,156-157)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16],
                         ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("layout", ["transposed", "sliced", "row-broadcast"])
@pytest.mark.parametrize("backward", [True, False])
def test_shift_pad_strided_inputs(dtype, layout, backward):
  """Transposed, column-sliced and row-broadcast views are read through
  their strides: the compiled form writes torch.empty_like(data) (the
  transposed layout is kept), the eager form a contiguous tensor.  A shift
  only moves bits, so the oracle runs on the raw bit patterns (integers,
  exact in fp64, a NaN payload included) and both results must match them
  bit for bit."""
  from oracle import oracle
  C, L = 37, 1000
  lens = [1, 300, 7, 692]
  cu = torch.tensor(cu_of(lens), device=DEV, dtype=torch.int32)
  gen = torch.Generator().manual_seed(8)
  if layout == "transposed":
    base = torch.randn(L, C, generator=gen).to(dtype)
    base[17, 2] = float("nan")
    data = base.to(DEV).t()
  elif layout == "sliced":
    base = torch.randn(C, L + 13, generator=gen).to(dtype)
    base[2, 5 + 17] = float("nan")
    data = base.to(DEV)[:, 5:5 + L]
  else:
    base = torch.randn(1, L, generator=gen).to(dtype)
    data = base.to(DEV).expand(C, L)
  iv = torch.int32 if dtype == torch.float32 else torch.int16
  if dtype != torch.float32 and layout != "row-broadcast":
    # a NaN with a payload (quiet bit plus low bits)
    nan_bits = torch.tensor([0x7FC5 if dtype == torch.bfloat16 else 0x7E05],
                            dtype=torch.int16).view(dtype)
    data[2, 17] = nan_bits.to(DEV)[0]
  src = data.cpu().contiguous().view(iv).to(torch.int64).numpy().astype(float)
  pad = float(torch.tensor([0.5], dtype=dtype).view(iv).item())
  cu_np = cu_of(lens)
  for compiled, out in ((True, ast.shift_pad_compiled(data, cu, 0.5, backward)),
                        (False, ast.shift_pad(data, cu, 0.5, backward))):
    exp = oracle.shift_pad(src, cu_np, pad, backward=backward,
                           wrap=not compiled)
    got = out.cpu().contiguous().view(iv).to(torch.int64).numpy()
    assert out.shape == (C, L)
    assert (got == exp.astype(np.int64)).all(), (compiled, layout)
    if compiled and layout == "transposed":
      assert out.stride() == data.stride()
    if not compiled:
      assert out.is_contiguous()
