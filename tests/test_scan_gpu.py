"""GPU parity tests: the gfx950 kernels (through the C ABI, via the public
API) against the fp64 oracle and the reference's known-answer vectors.

Inputs are generated on the CPU with seeded torch generators, so the oracle
and the kernels see identical values.  Tolerances (elementwise
|got - ref| <= atol + rtol*|ref|) are in tests/_helpers.py: fp32 rtol 1e-5.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import associative_scan_triton as ast
from _helpers import (DEV, TOL, check_close, cu_of, grid_args, make, npf,
                      oracle_bwd, oracle_fwd)
from oracle import oracle

pytestmark = pytest.mark.gpu

GOLD = json.loads(
  (Path(__file__).parent / "golden" / "known_answers.json").read_text())

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
DT_IDS = ["f32", "f16", "bf16"]

# Segment-length sets: single elements, lengths around the 16-byte vector
# and the 64-vector sub-tile (256 fp32 / 512 half elements), odd lengths,
# and a few thousand.
LENS = [
  [1],
  [3],
  [4],
  [1, 1, 1, 1, 1],
  [255],
  [256],
  [257],
  [511, 512, 513],
  [1000, 3, 4097],
  [17, 1, 2, 3, 1024, 1025, 250],
  [2 * 4096 + 3, 7],
  # long segments: without a workspace, fp32 walks them with the
  # workgroup-cooperative kernels (8 waves from a mean of 8192 elements, 16
  # from 16384 / 32768); short segments mixed in
  [20000],
  [16384 * 2 + 5],
  [70000, 1, 2, 5000, 100000],
]


# ---------------------------------------------------------------------------
# known-answer vectors (reference tests)
# ---------------------------------------------------------------------------

def _gold_tensors(case):
  g = torch.tensor(case["g"], dtype=torch.float32, device=DEV)
  x = torch.tensor(case["x"], dtype=torch.float32, device=DEV)
  cu = torch.tensor(case["cu"], device=DEV)
  return g, x, cu


@pytest.mark.parametrize("case", GOLD["forward"], ids=lambda c: c["name"])
def test_golden_forward_scan_full(case):
  """forward_scan_full in place with TESTING=True (gates <- A)."""
  for chunk in case["chunk_sizes"]:
    g, x, cu = _gold_tensors(case)
    cu_np = np.array(case["cu"])
    grid = ast.get_grid(len(cu_np), int(np.diff(cu_np).max()), chunk,
                        case["channels"])
    ast.forward_scan_full(g, x, cu, grid, REVERSE=case["reverse"],
                          CHUNK_SIZE=chunk, TESTING=True)
    exp_h = torch.tensor(case["h"], device=DEV).reshape(x.shape)
    assert torch.allclose(x, exp_h, rtol=case["rtol"], atol=case["atol"]), x
    if "A" in case:
      exp_a = torch.tensor(case["A"], device=DEV).reshape(g.shape)
      assert torch.allclose(g, exp_a, rtol=case["rtol"], atol=case["atol"]), g


@pytest.mark.parametrize("case", GOLD["forward"], ids=lambda c: c["name"])
def test_golden_kernel_objects(case):
  """kernel[grid](...) call convention (test_scan_kernels.py:160-168)."""
  g, x, cu = _gold_tensors(case)
  chunk = case["chunk_sizes"][0]
  cu_np = np.array(case["cu"])
  grid = ast.get_grid(len(cu_np), int(np.diff(cu_np).max()), chunk,
                      case["channels"])
  out = torch.empty_like(x)
  ast.forward_scan_chunked[grid](
    gates_ptr=g, tokens_ptr=x, tokens_out_ptr=out, cu_seqlens_ptr=cu,
    REVERSE=case["reverse"], CHUNK_SIZE=chunk, TESTING=False, INPLACE=False)
  exp_h = torch.tensor(case["h"], device=DEV).reshape(x.shape)
  assert torch.allclose(out, exp_h, rtol=case["rtol"], atol=case["atol"])
  out2 = torch.empty_like(x)
  ast.forward_scan_onepass_pipelined[(grid[0], grid[2])](
    gates_ptr=g, tokens_ptr=x, tokens_out_ptr=out2, cu_seqlens_ptr=cu,
    REVERSE=case["reverse"], CHUNK_SIZE=chunk, NUM_CHUNKS=grid[1],
    TESTING=False, NUM_STAGES=3, INPLACE=False)
  assert torch.equal(out, out2)
  # inputs untouched when TESTING=False and INPLACE=False
  g0, x0, _ = _gold_tensors(case)
  assert torch.equal(g, g0) and torch.equal(x, x0)


@pytest.mark.parametrize("case", GOLD["causal_grad"], ids=lambda c: c["name"])
@pytest.mark.parametrize("compiled", [False, True])
def test_golden_causal_grad(case, compiled):
  """test_scan_causal.py:19-71, eager and compiled."""
  fn = ast.scan_causal_compiled if compiled else ast.scan_causal
  for chunk in case["chunk_sizes"]:
    g = torch.tensor([case["g"]], device=DEV, requires_grad=True)
    x = torch.tensor([case["x"]], device=DEV, requires_grad=True)
    cu = torch.tensor(case["cu"], device=DEV)
    grid = ast.get_grid(len(case["cu"]), 4, chunk, 1)
    y = fn(g, x, {"cu_seqlens": cu, "chunk_size": chunk, "grid": grid})
    tol = dict(rtol=case["rtol"], atol=case["atol"])
    assert torch.allclose(y, torch.tensor([case["h"]], device=DEV), **tol)
    y.sum().backward()
    assert torch.allclose(g.grad, torch.tensor([case["dg"]], device=DEV), **tol)
    assert torch.allclose(x.grad, torch.tensor([case["dx"]], device=DEV), **tol)


# ---------------------------------------------------------------------------
# random parity against the fp64 oracle
# ---------------------------------------------------------------------------

@pytest.fixture(params=["lookback", "direct"])
def walk(request):
  """Runs a test with the workspace (decoupled look-back walk) and without
  it (one wave or one workgroup per segment)."""
  from associative_scan_triton import _ops
  prev = _ops.USE_WORKSPACE
  _ops.USE_WORKSPACE = request.param == "lookback"
  yield request.param
  _ops.USE_WORKSPACE = prev


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("reverse", [False, True], ids=["causal", "reverse"])
@pytest.mark.parametrize("lens", LENS, ids=lambda l: "x".join(map(str, l))[:40])
def test_forward_parity(dtype, reverse, lens, walk):
  C = 3
  g, x = make(lens, C, dtype)
  gd, xd = g.to(DEV), x.to(DEV)
  h = torch.empty_like(xd)
  a = torch.empty_like(gd)
  cu = torch.tensor(cu_of(lens), device=DEV, dtype=torch.int32)
  from associative_scan_triton import _ops
  ref, a_ref = oracle.scan_fwd(npf(g), npf(x), cu_of(lens), reverse,
                               gate_prod=True)
  # without the gate product (long segments take the workgroup walk) ...
  _ops.scan_fwd(gd, xd, h, cu, reverse=reverse)
  check_close(h, ref, dtype, "h")
  # ... and with it (always the one-wave-per-segment walk)
  h2 = torch.empty_like(xd)
  _ops.scan_fwd(gd, xd, h2, cu, reverse=reverse, gate_prod_out=a)
  check_close(h2, ref, dtype, "h (with gate product)")
  check_close(a, a_ref, dtype, "gate product")
  assert torch.equal(gd, g.to(DEV)) and torch.equal(xd, x.to(DEV))


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "anticausal"])
@pytest.mark.parametrize("lens", LENS, ids=lambda l: "x".join(map(str, l))[:40])
def test_backward_parity(dtype, causal, lens, walk):
  C = 3
  g, h, dy = make(lens, C, dtype, n=3)
  dx = torch.empty(C, sum(lens), dtype=dtype, device=DEV)
  dg = torch.empty_like(dx)
  cu = torch.tensor(cu_of(lens), device=DEV, dtype=torch.int64)
  from associative_scan_triton import _ops
  _ops.scan_bwd(dy.to(DEV), g.to(DEV), h.to(DEV), dx, dg, cu, causal=causal)
  dx_ref, dg_ref = oracle.scan_bwd(npf(dy), npf(g), npf(h), cu_of(lens), causal)
  check_close(dx, dx_ref, dtype, "dx")
  check_close(dg, dg_ref, dtype, "dg")


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("lens", [[37], [1, 600, 2], [4096, 4096]],
                         ids=lambda l: "x".join(map(str, l)))
def test_scan_causal_autograd_parity(dtype, lens):
  C = 4
  g, x, dy = make(lens, C, dtype, n=3)
  args = grid_args(lens, C)
  gd = g.to(DEV).requires_grad_(True)
  xd = x.to(DEV).requires_grad_(True)
  y = ast.scan_causal(gd, xd, args)
  y.backward(dy.to(DEV))
  h_ref = oracle_fwd(g, x, lens)
  check_close(y, h_ref, dtype, "h")
  dx_ref, dg_ref = oracle_bwd(dy, g, npf(y), lens)
  check_close(xd.grad, dx_ref, dtype, "dx")
  check_close(gd.grad, dg_ref, dtype, "dg")


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("compiled", [False, True], ids=["eager", "compiled"])
@pytest.mark.parametrize("lens", [[5], [64, 1, 300], [2048, 33]],
                         ids=lambda l: "x".join(map(str, l)))
def test_bidirectional_parity(dtype, compiled, lens, walk):
  C = 3
  gf, xf, dyf = make(lens, C, dtype, seed=1, glo=0.9, n=3)
  gb, xb, dyb = make(lens, C, dtype, seed=2, glo=0.9, n=3)
  args = grid_args(lens, C)
  fn = (ast.scan_bidirectional_branched_compiled if compiled
        else ast.scan_bidirectional_branched)
  ts = [t.to(DEV).requires_grad_(True) for t in (gf, xf, gb, xb)]
  yf, yb = fn(*ts, args)
  torch.autograd.backward([yf, yb], [dyf.to(DEV), dyb.to(DEV)])
  hf = oracle_fwd(gf, xf, lens)
  hb = oracle_fwd(gb, xb, lens, reverse=True)
  check_close(yf, hf, dtype, "h fwd branch")
  check_close(yb, hb, dtype, "h bwd branch")
  dxf, dgf = oracle_bwd(dyf, gf, npf(yf), lens, causal=True)
  dxb, dgb = oracle_bwd(dyb, gb, npf(yb), lens, causal=False)
  check_close(ts[0].grad, dgf, dtype, "dg fwd")
  check_close(ts[1].grad, dxf, dtype, "dx fwd")
  check_close(ts[2].grad, dgb, dtype, "dg bwd")
  check_close(ts[3].grad, dxb, dtype, "dx bwd")


def test_bidirectional_compiled_matches_eager():
  """test_compiled.py:49-89 (B in {1,4}, T in {64,256}, C=64, chunk 128)."""
  for B in (1, 4):
    for T in (64, 256):
      lens = [T] * B
      gen = torch.Generator().manual_seed(1155)
      C = 64
      gf, gb = torch.rand(C, T * B, generator=gen), torch.rand(C, T * B, generator=gen)
      xf, xb = torch.randn(C, T * B, generator=gen), torch.randn(C, T * B, generator=gen)
      args = grid_args(lens, C)
      d = [t.to(DEV) for t in (gf, xf, gb, xb)]
      ref = ast.scan_bidirectional_branched(*[t.clone() for t in d], args)
      got = ast.scan_bidirectional_branched_compiled(*[t.clone() for t in d], args)
      torch.testing.assert_close(ref[0], got[0], rtol=1e-5, atol=1e-5)
      torch.testing.assert_close(ref[1], got[1], rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------
# segment boundaries: exact, and no leakage across documents
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_segment_boundaries_bit_exact(dtype, walk):
  lens = [1, 2, 3, 257, 64, 1, 513, 9]
  C = 5
  g, x, dy = make(lens, C, dtype, n=3, glo=-2.0, ghi=2.0)
  # signed zeros and a zero at segment heads
  x[:, 0] = -0.0
  x[1, 3] = -0.0
  dy[:, -1] = -0.0
  cu = cu_of(lens)
  heads, tails = cu[:-1], cu[1:] - 1
  cud = torch.tensor(cu, device=DEV)
  from associative_scan_triton import _ops
  gd, xd, dyd = g.to(DEV), x.to(DEV), dy.to(DEV)
  for rev in (False, True):
    h = torch.empty_like(xd)
    _ops.scan_fwd(gd, xd, h, cud, reverse=rev)
    first = tails if rev else heads
    got = h[:, first].cpu()
    assert torch.equal(got.view(torch.int16 if dtype != torch.float32 else torch.int32),
                       x[:, first].view(torch.int16 if dtype != torch.float32 else torch.int32))
    dx = torch.empty_like(xd)
    dg = torch.empty_like(xd)
    _ops.scan_bwd(dyd, gd, h, dx, dg, cud, causal=not rev)
    start = heads if rev else tails        # first element of the adjoint scan
    last = tails if rev else heads         # where the shifted state is padded
    iv = torch.int16 if dtype != torch.float32 else torch.int32
    assert torch.equal(dx[:, start].cpu().view(iv), dy[:, start].view(iv))
    exp = (torch.zeros((), dtype=torch.float32) * dx[:, last].float()).to(dtype)
    assert torch.equal(dg[:, last].cpu().view(iv), exp.cpu().view(iv))


def test_nonfinite_values_stay_in_their_segment(walk):
  lens = [300, 5, 700, 1]
  C = 2
  g, x, dy = make(lens, C, n=3)
  cu = cu_of(lens)
  g[:, cu[1] + 2] = float("inf")
  x[:, cu[1] + 1] = float("nan")
  dy[:, cu[1] + 3] = float("nan")
  gd, xd = g.to(DEV), x.to(DEV)
  from associative_scan_triton import _ops
  cud = torch.tensor(cu, device=DEV)
  for rev in (False, True):
    h = torch.empty_like(xd)
    _ops.scan_fwd(gd, xd, h, cud, reverse=rev)
    dx = torch.empty_like(xd)
    dg = torch.empty_like(xd)
    _ops.scan_bwd(dy.to(DEV), gd, h, dx, dg, cud, causal=not rev)
    ref = oracle.scan_fwd(npf(g), npf(x), cu, rev)
    ok = np.r_[0:cu[1], cu[2]:cu[4]]
    check_close(h[:, ok], ref[:, ok], torch.float32, "h outside the bad segment")
    dxr, dgr = oracle.scan_bwd(npf(dy), npf(g), npf(h), cu, not rev)
    check_close(dx[:, ok], dxr[:, ok], torch.float32, "dx outside")
    check_close(dg[:, ok], dgr[:, ok], torch.float32, "dg outside")


# ---------------------------------------------------------------------------
# layouts: flat 1-D tensors, misaligned views, int32/int64 cu_seqlens
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("offsets", [(1, 1, 1), (2, 2, 2), (3, 1, 2), (0, 1, 0)],
                         ids=["phase1", "phase2", "mixed", "mixed2"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("lens", [[100, 1, 33, 150], [700, 1, 33, 1500],
                                  [40000, 3, 90001]],
                         ids=["tiny", "short", "long"])
def test_misaligned_views(offsets, dtype, lens, walk):
  C = 3
  T = sum(lens)
  g, x, dy = make(lens, C, dtype, n=3)

  def view_at(src, off):
    buf = torch.zeros(C * T + 16, dtype=dtype, device=DEV)
    v = buf[off:off + C * T].view(C, T)
    v.copy_(src.to(DEV))
    return v

  gd, xd = view_at(g, offsets[0]), view_at(x, offsets[1])
  h = view_at(torch.zeros_like(x), offsets[2])
  cu = torch.tensor(cu_of(lens), device=DEV)
  from associative_scan_triton import _ops
  _ops.scan_fwd(gd, xd, h, cu, reverse=False)
  check_close(h, oracle_fwd(g, x, lens), dtype, "h (misaligned)")
  dx = view_at(torch.zeros_like(x), offsets[0])
  dg = view_at(torch.zeros_like(x), offsets[2])
  _ops.scan_bwd(view_at(dy, offsets[1]), gd, h, dx, dg, cu, causal=True)
  dxr, dgr = oracle.scan_bwd(npf(dy), npf(g), npf(h), cu_of(lens), True)
  check_close(dx, dxr, dtype, "dx (misaligned)")
  check_close(dg, dgr, dtype, "dg (misaligned)")


def test_flat_layout_and_cu_dtypes():
  """1-D [C*T] tensors addressed with the grid's channel count, as the
  reference's test data (test_utils.py:89-100)."""
  lens = [3, 5, 8]
  C = 2
  g, x = make(lens, C)
  ref = oracle_fwd(g, x, lens)
  for cu_dtype in (torch.int32, torch.int64):
    cu = torch.tensor(cu_of(lens), device=DEV, dtype=cu_dtype)
    grid = ast.get_grid(len(cu), 8, 4, C)
    gd, xd = g.flatten().to(DEV), x.flatten().to(DEV)
    ast.forward_scan_full(gd, xd, cu, grid, REVERSE=False, CHUNK_SIZE=4,
                          TESTING=False)
    check_close(xd.view(C, -1), ref, torch.float32, f"flat h {cu_dtype}")


# ---------------------------------------------------------------------------
# reference dtype tests (test_scan_dtypes.py)
# ---------------------------------------------------------------------------

REF_TOL = {  # test_scan_dtypes.py:42-46
  torch.float32: {"atol": 1e-5, "rtol": 1e-4},
  torch.float16: {"atol": 5e-3, "rtol": 5e-2},
  torch.bfloat16: {"atol": 3e-2, "rtol": 1e-1},
}


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("seqlen", [32, 128, 512, 1024])
@pytest.mark.parametrize("num_channels", [1, 4])
def test_reference_forward_vs_gold(dtype, seqlen, num_channels):
  """test_scan_dtypes.py:62-90 with inputs drawn on the CPU."""
  gen = torch.Generator().manual_seed(1155)
  g = torch.rand(num_channels, seqlen, generator=gen).to(dtype)
  x = torch.randn(num_channels, seqlen, generator=gen).to(dtype)
  chunk = min(seqlen, 512)
  args = grid_args([seqlen], num_channels, chunk)
  y = ast.scan_causal(g.to(DEV), x.to(DEV), args)
  gold = torch.from_numpy(oracle_fwd(g, x, [seqlen]))
  torch.testing.assert_close(y.cpu().double(), gold, **REF_TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_reference_multi_chunk_rmse(dtype):
  """test_scan_dtypes.py:115-142: fp16 RMSE < 1e-3, bf16 < 5e-3."""
  gen = torch.Generator().manual_seed(1155)
  g = torch.rand(4, 1024, generator=gen).to(dtype)
  x = torch.randn(4, 1024, generator=gen).to(dtype)
  y = ast.scan_causal(g.to(DEV), x.to(DEV), grid_args([1024], 4, 512))
  rmse = float(np.sqrt(np.mean((npf(y) - oracle_fwd(g, x, [1024])) ** 2)))
  assert rmse < (1e-3 if dtype == torch.float16 else 5e-3), rmse


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_reference_varlen_packed(dtype):
  """test_scan_dtypes.py:221-256."""
  seqlens = [32, 64, 128]
  gen = torch.Generator().manual_seed(1155)
  g = torch.rand(2, 224, generator=gen).to(dtype)
  x = torch.randn(2, 224, generator=gen).to(dtype)
  y = ast.scan_causal(g.to(DEV), x.to(DEV), grid_args(seqlens, 2, 128))
  ref = oracle_fwd(g, x, seqlens)
  torch.testing.assert_close(y.cpu().double(), torch.from_numpy(ref),
                             **REF_TOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("seqlen", [64, 256, 1024])
def test_reference_bidi_vs_gold(dtype, seqlen):
  """test_scan_dtypes.py:148-189 (reverse gold = flip o scan o flip)."""
  gen = torch.Generator().manual_seed(1155)
  ts = [torch.rand(4, seqlen, generator=gen).to(dtype) if i % 2 == 0
        else torch.randn(4, seqlen, generator=gen).to(dtype) for i in range(4)]
  yf, yb = ast.scan_bidirectional_branched(
    *[t.to(DEV) for t in ts], grid_args([seqlen], 4, min(seqlen, 512)))
  gold_f = oracle_fwd(ts[0], ts[1], [seqlen])
  gold_b = oracle.scan_fwd(npf(ts[2])[:, ::-1], npf(ts[3])[:, ::-1],
                           [0, seqlen])[:, ::-1]
  torch.testing.assert_close(yf.cpu().double(), torch.from_numpy(gold_f),
                             **REF_TOL[dtype])
  torch.testing.assert_close(yb.cpu().double(),
                             torch.from_numpy(np.ascontiguousarray(gold_b)),
                             **REF_TOL[dtype])


# The reference's causal sweep (test_scan_causal.py:75-130): one sequence,
# chunk sizes 2..256, 1/2/32 channels, gates ~ U(0,1), tokens ~ N(0,1),
# scan_causal then out.sum().backward().  The reference compares with JAX
# (not installed here, rtol = atol = 1e-4); the oracle states the same
# recurrences in fp64.
CAUSAL_SWEEP = [(cs, nc, sl) for cs in [2 ** i for i in range(1, 9)]
                for nc in (1, 2, 32) for sl in (1, 5, 32, 128)]


@pytest.mark.parametrize("chunk_size,num_channels,seqlen", CAUSAL_SWEEP)
def test_reference_causal_sweep(chunk_size, num_channels, seqlen):
  gen = torch.Generator().manual_seed(1155)
  g = torch.rand(num_channels, seqlen, generator=gen)
  x = torch.randn(num_channels, seqlen, generator=gen)
  gd, xd = g.to(DEV).requires_grad_(True), x.to(DEV).requires_grad_(True)
  out = ast.scan_causal(gd, xd, grid_args([seqlen], num_channels, chunk_size))
  out.sum().backward()
  cu = cu_of([seqlen])
  h = oracle.scan_fwd(npf(g), npf(x), cu, False)
  dx, dg = oracle.scan_bwd(np.ones((num_channels, seqlen)), npf(g), h, cu, True)
  for name, got, ref in (("forward", out, h), ("gate grad", gd.grad, dg),
                         ("token grad", xd.grad, dx)):
    check_close(got, ref, torch.float32, name)
    assert torch.allclose(got.detach().cpu().double(), torch.from_numpy(ref),
                          rtol=1e-4, atol=1e-4), name


# test_scan_kernels.py:287-467: forward_scan_full with a grid of several
# chunks per sequence against one chunk per sequence (10 sequences of
# `seqlen`, in place with the gate product, both directions).  The reference
# computes torch.allclose without asserting it; here every launch scans whole
# segments, so the two must agree bit for bit, and they are also checked
# against the oracle.
@pytest.mark.parametrize("reverse", [False, True], ids=["causal", "reverse"])
@pytest.mark.parametrize("seqlen,chunk_size,no_channels",
                         [(4, 2, 2), (8, 4, 1), (8, 4, 2), (8, 4, 3), (8, 2, 1),
                          (8, 2, 2), (8, 2, 3), (16, 8, 2), (16, 4, 2),
                          (16, 2, 2)])
def test_reference_one_vs_multiple_chunks(seqlen, chunk_size, no_channels,
                                          reverse):
  lens = [seqlen] * 10
  gen = torch.Generator().manual_seed(1155)
  g = torch.rand(no_channels, seqlen * 10, generator=gen)
  x = torch.rand(no_channels, seqlen * 10, generator=gen)
  cu = torch.tensor(cu_of(lens), device=DEV)
  outs = []
  for cs in (chunk_size, seqlen):
    gd, xd = g.to(DEV), x.to(DEV)
    grid = ast.get_grid(len(cu), seqlen, cs, no_channels)
    ast.forward_scan_full(gates=gd, tokens=xd, cu_seqlens=cu, CHUNK_SIZE=cs,
                          grid=grid, REVERSE=reverse)
    outs.append((gd, xd))
  assert torch.equal(outs[0][0], outs[1][0]), "gate products"
  assert torch.equal(outs[0][1], outs[1][1]), "states"
  h, a = oracle.scan_fwd(npf(g), npf(x), cu_of(lens), reverse, gate_prod=True)
  check_close(outs[0][1], h, torch.float32, "states")
  check_close(outs[0][0], a, torch.float32, "gate products")


# The reference's bidirectional sweep (test_scan_bidi.py:21-128, and
# :129-200 with testing=False where the chunk covers the sequence): one
# sequence, chunk sizes 2..256 (below the sequence length too), 1/2/32
# channels, loss = out_fwd.sum() + out_bwd.sum().  The reference compares with
# JAX's lax.associative_scan (jax is not installed here); the oracle states
# the same recurrences in fp64, and both the reference's own tolerance and
# the fp32 bound of these tests are checked.
BIDI_SWEEP = [(t, cs, nc, sl) for t in (True, False)
              for cs in [2 ** i for i in range(1, 9)]
              for nc in (1, 2, 32) for sl in (1, 5, 32, 128)
              if t or cs >= sl]


@pytest.mark.parametrize("testing,chunk_size,num_channels,seqlen", BIDI_SWEEP)
def test_reference_bidi_sweep(testing, chunk_size, num_channels, seqlen):
  gen = torch.Generator().manual_seed(1155)
  ts = [torch.rand(num_channels, seqlen, generator=gen) for _ in range(4)]
  leaves = [t.to(DEV).requires_grad_(True) for t in ts]
  args = grid_args([seqlen], num_channels, chunk_size)
  yf, yb = ast.scan_bidirectional_branched(*leaves, args, testing=testing)
  (yf.sum() + yb.sum()).backward()
  cu = cu_of([seqlen])
  ones = np.ones((num_channels, seqlen))
  hf = oracle.scan_fwd(npf(ts[0]), npf(ts[1]), cu, False)
  hb = oracle.scan_fwd(npf(ts[2]), npf(ts[3]), cu, True)
  dxf, dgf = oracle.scan_bwd(ones, npf(ts[0]), hf, cu, True)
  dxb, dgb = oracle.scan_bwd(ones, npf(ts[2]), hb, cu, False)
  for name, got, ref in (("states fwd", yf, hf), ("states bwd", yb, hb),
                         ("gates grad fwd", leaves[0].grad, dgf),
                         ("tokens grad fwd", leaves[1].grad, dxf),
                         ("gates grad bwd", leaves[2].grad, dgb),
                         ("tokens grad bwd", leaves[3].grad, dxb)):
    check_close(got, ref, torch.float32, name)
    assert torch.allclose(got.detach().cpu().double(), torch.from_numpy(ref),
                          rtol=1e-4, atol=1e-7), name


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("seqlen", [64, 512, 1024])
def test_reference_bidi_backward_finite(dtype, seqlen):
  """test_scan_dtypes.py:191-215."""
  ts = [(torch.rand if i % 2 == 0 else torch.randn)(4, seqlen, dtype=dtype,
                                                     device=DEV).requires_grad_(True)
        for i in range(4)]
  yf, yb = ast.scan_bidirectional_branched(*ts, grid_args([seqlen], 4, 512))
  (yf.sum() + yb.sum()).backward()
  for t in ts:
    assert t.grad is not None and torch.isfinite(t.grad).all()


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_accuracy_no_worse_than_reference(dtype):
  """RMSE against the fp64 gold at C=4, T in {128, 512, 2048, 8192}
  (bench_accuracy.py:31-37) must not exceed the reference's published RMSE
  (README.md:266-281) by more than sampling noise (inputs differ: the
  reference drew them with the CUDA generator).  Averaged over 4 seeds."""
  acc = GOLD["accuracy_rmse"]
  key = {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16"}[dtype]
  for T, pub in zip(acc["seqlens"], acc[key]):
    rmses = []
    for seed in range(4):
      gen = torch.Generator().manual_seed(42 + seed)
      g = torch.rand(4, T, generator=gen).to(dtype)
      x = torch.randn(4, T, generator=gen).to(dtype)
      y = ast.scan_causal(g.to(DEV), x.to(DEV), grid_args([T], 4, min(T, 512)))
      rmses.append(np.sqrt(np.mean((npf(y) - oracle_fwd(g, x, [T])) ** 2)))
    assert np.mean(rmses) <= 1.25 * pub, (key, T, np.mean(rmses), pub)


# ---------------------------------------------------------------------------
# shift_pad
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", GOLD["shift_pad"]["cases"], ids=lambda c: c["name"])
@pytest.mark.parametrize("backward", [True, False])
def test_shift_pad_golden(case, backward):
  pad = GOLD["shift_pad"]["pad"]
  data = torch.tensor(case["data"], device=DEV)
  cu = torch.tensor(case["cu"], device=DEV)
  exp = torch.tensor(case["backward" if backward else "forward"], device=DEV)
  assert torch.equal(ast.shift_pad(data, cu, pad, backward), exp)
  assert torch.equal(ast.shift_pad_compiled(data, cu, pad, backward), exp)


def test_shift_pad_zero_length_raises():
  z = GOLD["shift_pad"]["zero_length"]
  with pytest.raises(AssertionError, match=z["message"]):
    ast.shift_pad(torch.tensor(z["data"], device=DEV),
                  torch.tensor(z["cu"], device=DEV), -1, True)


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("backward", [True, False])
@pytest.mark.parametrize("pad_value", [0.0, 1.0, -1.5])
def test_shift_pad_parity(dtype, backward, pad_value):
  """Random data vs the oracle; compiled == eager bit for bit
  (test_compiled.py:91-104)."""
  gen = torch.Generator().manual_seed(9)
  lens = [64, 1, 700, 3, 1300]
  C, L = 7, sum(lens)
  data = torch.randn(C, L, generator=gen).to(dtype)
  cu = torch.tensor(cu_of(lens), device=DEV, dtype=torch.int32)
  dd = data.to(DEV)
  eager = ast.shift_pad(dd, cu, pad_value, backward)
  comp = ast.shift_pad_compiled(dd, cu, pad_value, backward)
  assert torch.equal(eager, comp)
  ref = oracle.shift_pad(npf(data), cu_of(lens), pad_value, backward, wrap=True)
  ref_t = torch.from_numpy(ref).to(dtype)
  assert torch.equal(eager.cpu(), ref_t)


# ---------------------------------------------------------------------------
# torch.compile / custom-op checks
# ---------------------------------------------------------------------------

def test_custom_ops_opcheck():
  lens = [40, 9]
  C = 3
  g, x, dy = make(lens, C, n=3)
  cu = torch.tensor(cu_of(lens), device=DEV, dtype=torch.int32)
  gd = g.to(DEV).requires_grad_(True)
  xd = x.to(DEV).requires_grad_(True)
  torch.library.opcheck(torch.ops.associative_scan_triton.scan_causal_fwd,
                        (gd, xd, cu, 1, C, 64))
  torch.library.opcheck(torch.ops.associative_scan_triton.scan_bidi_fwd,
                        (gd, xd, gd, xd, cu, 1, C, 64))
  torch.library.opcheck(torch.ops.associative_scan_triton.shift_pad,
                        (xd.detach(), cu, 0.0, True))


def test_custom_ops_opcheck_backward():
  """The backward ops too, with a dense and a time-constant (stride-0)
  incoming gradient."""
  lens = [40, 9]
  C = 3
  g, h, dy = make(lens, C, n=3)
  cu = torch.tensor(cu_of(lens), device=DEV, dtype=torch.int32)
  gd, hd, dyd = g.to(DEV), h.to(DEV), dy.to(DEV)
  ones = torch.ones((), device=DEV).expand(C, sum(lens))
  for grad in (dyd, ones):
    torch.library.opcheck(torch.ops.associative_scan_triton.scan_causal_bwd,
                          (grad, gd, hd, cu, 1, C, 64))
  torch.library.opcheck(torch.ops.associative_scan_triton.scan_bidi_bwd,
                        (dyd, dyd, hd, hd, gd, gd, cu, 1, C, 64))


def test_torch_compile_dynamic_num_seq():
  """With the grid from get_static_grid the compiled graph does not depend on
  the number of packed sequences: after one dynamic-shape compile, other
  counts of sequences (and total lengths) run without recompiling
  (the reference's reason for get_static_grid, _grid.py:57-70)."""
  import torch._dynamo
  C = 6
  static = ast.get_static_grid(512, 128, C)

  def f(g, x, cu):
    args = {"cu_seqlens": cu, "chunk_size": 128, "grid": (cu.shape[0] - 1,) + static}
    return ast.scan_causal_compiled(g, x, args).square().sum()

  torch._dynamo.reset()
  cf = torch.compile(f, backend="aot_eager", fullgraph=True, dynamic=True)
  for i, lens in enumerate(([100, 28, 7], [5, 300, 17, 1, 64], [512] * 4 + [3] * 5)):
    g, x = make(lens, C, seed=40 + i)
    cu = torch.tensor(cu_of(lens), device=DEV, dtype=torch.int32)
    gd = g.to(DEV).requires_grad_(True)
    xd = x.to(DEV).requires_grad_(True)
    if i == 0:
      loss = cf(gd, xd, cu)
    else:
      with torch._dynamo.config.patch(error_on_recompile=True):
        loss = cf(gd, xd, cu)
    loss.backward()
    g2 = g.to(DEV).requires_grad_(True)
    x2 = x.to(DEV).requires_grad_(True)
    loss2 = f(g2, x2, cu)
    loss2.backward()
    torch.testing.assert_close(loss, loss2)
    torch.testing.assert_close(gd.grad, g2.grad)
    torch.testing.assert_close(xd.grad, x2.grad)


def test_torch_compile_fullgraph():
  lens = [100, 28]
  C = 4
  g, x = make(lens, C)
  args = grid_args(lens, C)

  def f(g, x):
    return ast.scan_causal_compiled(g, x, args).square().sum()

  cf = torch.compile(f, backend="aot_eager", fullgraph=True)
  gd = g.to(DEV).requires_grad_(True)
  xd = x.to(DEV).requires_grad_(True)
  loss = cf(gd, xd)
  loss.backward()
  g2 = g.to(DEV).requires_grad_(True)
  x2 = x.to(DEV).requires_grad_(True)
  loss2 = f(g2, x2)
  loss2.backward()
  torch.testing.assert_close(loss, loss2)
  torch.testing.assert_close(gd.grad, g2.grad)
  torch.testing.assert_close(xd.grad, x2.grad)


def test_backward_kernel_objects():
  """backward_scan_fused[grid](...) as bench_kernels.py:119-135 calls it."""
  lens = [1024, 1024]
  C = 2
  g, h, dy = make(lens, C, n=3)
  cu = torch.tensor(cu_of(lens), device=DEV, dtype=torch.int32)
  grid = ast.get_grid(3, 1024, 128, C)
  outs = []
  for kern, gr in ((ast.backward_scan_fused, (grid[0], grid[2])),
                   (ast.backward_scan_fused_single_chunk, (grid[0], 1, grid[2]))):
    dx = torch.empty(C, 2048, device=DEV)
    dg = torch.empty_like(dx)
    kw = dict(grad_ptr=dy.to(DEV), gates_ptr=g.to(DEV), states_ptr=h.to(DEV),
              d_tokens_ptr=dx, d_gates_ptr=dg, cu_seqlens_ptr=cu,
              CHUNK_SIZE=128, CAUSAL=True)
    if kern is ast.backward_scan_fused:
      kw.update(NUM_CHUNKS=grid[1], NUM_STAGES=3)
    kern[gr](**kw)
    outs.append((dx, dg))
  dxr, dgr = oracle.scan_bwd(npf(dy), npf(g), npf(h), cu_of(lens), True)
  for dx, dg in outs:
    check_close(dx, dxr, torch.float32, "dx")
    check_close(dg, dgr, torch.float32, "dg")
  dxb = torch.empty(C, 2048, device=DEV)
  dgb = torch.empty_like(dxb)
  ast.backward_scan_fused_full(dy.to(DEV), g.to(DEV), h.to(DEV), dxb, dgb, cu,
                               grid, CHUNK_SIZE=128, CAUSAL=True)
  assert torch.equal(dxb, outs[0][0]) and torch.equal(dgb, outs[0][1])


def test_stream_semantics():
  """Launches go to the caller's current stream."""
  lens = [5000]
  g, x = make(lens, 8)
  gd, xd = g.to(DEV), x.to(DEV)
  s = torch.cuda.Stream()
  with torch.cuda.stream(s):
    h = torch.empty_like(xd)
    from associative_scan_triton import _ops
    _ops.scan_fwd(gd, xd, h, torch.tensor(cu_of(lens), device=DEV), False)
  s.synchronize()
  check_close(h, oracle_fwd(g, x, lens), torch.float32, "h on side stream")


@pytest.mark.parametrize("lens", [[5000], [20000, 3, 1, 7000], [1, 2, 3, 4, 5, 900]],
                         ids=["one", "mixed", "short"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_lookback_fallback_path(lens, dtype):
  """With a spin limit of 0 every look-back that finds a predecessor not yet
  published computes that tile's map from its inputs (the bounded-wait
  path that guarantees progress).  Results must not change."""
  from associative_scan_triton import _lib, _ops
  lib = _lib.load()
  prev_ws = _ops.USE_WORKSPACE
  _ops.USE_WORKSPACE = True
  prev = lib.asc_set_lookback_spin_limit(0)
  try:
    C = 5
    g, x, dy = make(lens, C, dtype, n=3, glo=0.5)
    gd, xd, dyd = g.to(DEV), x.to(DEV), dy.to(DEV)
    cu = torch.tensor(cu_of(lens), device=DEV)
    for rev in (False, True):
      h = torch.empty_like(xd)
      _ops.scan_fwd(gd, xd, h, cu, reverse=rev)
      check_close(h, oracle_fwd(g, x, lens, rev), dtype, "h (fallback)")
      dx, dg = torch.empty_like(xd), torch.empty_like(xd)
      _ops.scan_bwd(dyd, gd, h, dx, dg, cu, causal=not rev)
      dxr, dgr = oracle.scan_bwd(npf(dy), npf(g), npf(h), cu_of(lens), not rev)
      check_close(dx, dxr, dtype, "dx (fallback)")
      check_close(dg, dgr, dtype, "dg (fallback)")
  finally:
    lib.asc_set_lookback_spin_limit(prev)
    _ops.USE_WORKSPACE = prev_ws


# ---------------------------------------------------------------------------
# gradients constant along time (out.sum().backward())
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("lens,C", [([3000, 17, 5000], 80), ([70000, 40000], 40),
                                    ([100, 200], 2)],
                         ids=["short", "long", "few-items"])
@pytest.mark.parametrize("compiled", [False, True], ids=["eager", "compiled"])
def test_time_constant_gradient(dtype, lens, C, compiled):
  """out.sum() and (out.sum(-1) * w).sum() hand the backward an expanded
  gradient (time stride 0); reading one value per row must give the same
  bits as the materialised gradient, and match the oracle."""
  fn = ast.scan_causal_compiled if compiled else ast.scan_causal
  g, x = make(lens, C, dtype, glo=0.5)
  args = grid_args(lens, C)
  w = torch.rand(C, generator=torch.Generator().manual_seed(3)).to(dtype).to(DEV)

  def grads(loss_of):
    gd = g.to(DEV).requires_grad_(True)
    xd = x.to(DEV).requires_grad_(True)
    y = fn(gd, xd, args)
    loss_of(y)
    return y.detach(), gd.grad, xd.grad

  T = sum(lens)
  # every walk (few items: the tree walk) reads the per-row value where the
  # dense walk reads the element, so the bits must agree
  for loss_of, dense in (
      (lambda y: y.sum().backward(), torch.ones(C, T, dtype=dtype, device=DEV)),
      (lambda y: (y.sum(-1) * w).sum().backward(),
       w[:, None].expand(C, T).contiguous())):
    y1, dg1, dx1 = grads(loss_of)
    y2, dg2, dx2 = grads(lambda y: y.backward(dense))
    assert torch.equal(dx1, dx2) and torch.equal(dg1, dg2)
    dx_ref, dg_ref = oracle_bwd(dense.cpu(), g, npf(y1), lens)
    check_close(dx1, dx_ref, dtype, "dx")
    check_close(dg1, dg_ref, dtype, "dg")


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "anticausal"])
def test_rowgrad_entry_point(dtype, causal):
  """asc_scan_bwd_rowgrad directly: one value per row, rows 3 elements
  apart, every walk (workgroup for long fp32 segments, one wave per item)."""
  from associative_scan_triton import _ops
  for lens, C in (([70000, 5, 33000], 70), ([900, 1, 2, 4096], 100)):
    g, h = make(lens, C, dtype, n=2, glo=0.5)
    rows = torch.randn(C, 3, generator=torch.Generator().manual_seed(5)).to(dtype)
    T = sum(lens)
    dx = torch.empty(C, T, dtype=dtype, device=DEV)
    dg = torch.empty_like(dx)
    cu = torch.tensor(cu_of(lens), device=DEV)
    rd = rows.to(DEV)
    _ops.scan_bwd_rowgrad(rd[:, 1], 3, g.to(DEV), h.to(DEV), dx, dg, cu, causal)
    dy = rows[:, 1:2].expand(C, T)
    dx_ref, dg_ref = oracle.scan_bwd(npf(dy), npf(g), npf(h), cu_of(lens), causal)
    check_close(dx, dx_ref, dtype, "dx")
    check_close(dg, dg_ref, dtype, "dg")


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "anticausal"])
@pytest.mark.parametrize("lens,C", [([1000], 100), ([3], 120), ([5, 2], 60),
                                    ([4099, 1], 20), ([70001], 3),
                                    ([20000, 7, 13000], 2)],
                         ids=["rows1000", "rows3", "rows7", "rows4100",
                              "long", "ragged"])
@pytest.mark.parametrize("spin", [None, 0], ids=["tree", "fallback"])
def test_tree_rowgrad_rows_in_chunk(dtype, causal, lens, C, spin):
  """Few items with a gradient constant along time (one value per row, rows
  3 elements apart): the tree walk's chunks hold many short rows (rows of
  3-7 elements share a vector) or lie in one row; the per-row read must
  give the bits of the dense gradient and match the oracle.  With a spin
  limit of 0 the tree walk gives up at its first wait and the
  workspace-free walk recomputes both calls, which must agree too."""
  from associative_scan_triton import _lib, _ops
  T = sum(lens)
  lib = _lib.load()
  prev = lib.asc_set_lookback_spin_limit(spin) if spin is not None else None
  try:
    _tree_rowgrad_case(lib, dtype, causal, lens, C, T)
  finally:
    if prev is not None:
      lib.asc_set_lookback_spin_limit(prev)


def _tree_rowgrad_case(lib, dtype, causal, lens, C, T):
  from associative_scan_triton import _lib, _ops
  assert lib.asc_scan_workspace_walk(len(lens), C, T, _lib.dtype_code(
    torch.empty((), dtype=dtype)), 1) == _lib.WALK_LOOKBACK
  g, h = make(lens, C, dtype, n=2, glo=0.5)
  rows = torch.randn(C, 3, generator=torch.Generator().manual_seed(5)).to(dtype)
  cu = torch.tensor(cu_of(lens), device=DEV)
  gd, hd, rd = g.to(DEV), h.to(DEV), rows.to(DEV)
  dx = torch.empty(C, T, dtype=dtype, device=DEV)
  dg = torch.empty_like(dx)
  _ops.scan_bwd_rowgrad(rd[:, 1], 3, gd, hd, dx, dg, cu, causal)
  dy = rows[:, 1:2].expand(C, T)
  dxd, dgd = torch.empty_like(dx), torch.empty_like(dx)
  _ops.scan_bwd(dy.contiguous().to(DEV), gd, hd, dxd, dgd, cu, causal)
  assert torch.equal(dx, dxd) and torch.equal(dg, dgd)
  dx_ref, dg_ref = oracle.scan_bwd(npf(dy), npf(g), npf(h), cu_of(lens), causal)
  check_close(dx, dx_ref, dtype, "dx")
  check_close(dg, dg_ref, dtype, "dg")


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_bidi_rowgrad_entry_point(dtype):
  """asc_scan_bidi_bwd_rowgrad directly: per-row values with different
  strides per branch (3 and 0), every walk; matches the dense entry point
  bit for bit (both run the workspace-free walks) and the oracle."""
  from associative_scan_triton import _ops
  prev = _ops.USE_WORKSPACE
  _ops.USE_WORKSPACE = False
  try:
    for lens, C in (([70000, 5, 33000], 70), ([900, 1, 2, 4096], 100)):
      gf, hf = make(lens, C, dtype, seed=1, n=2, glo=0.5)
      gb, hb = make(lens, C, dtype, seed=2, n=2, glo=0.5)
      rows = torch.randn(C, 3, generator=torch.Generator().manual_seed(5)).to(dtype)
      one = torch.randn(1, generator=torch.Generator().manual_seed(6)).to(dtype)
      T = sum(lens)
      cu = torch.tensor(cu_of(lens), device=DEV)
      d = [t.to(DEV) for t in (gf, gb, hf, hb)]
      outs = [torch.empty(C, T, dtype=dtype, device=DEV) for _ in range(4)]
      rd, od = rows.to(DEV), one.to(DEV)
      _ops.scan_bidi_bwd_rowgrad(rd[:, 1], 3, od, 0, *d, *outs, cu)
      dyf = rows[:, 1:2].expand(C, T)
      dyb = one.reshape(1, 1).expand(C, T)
      dense = [torch.empty_like(o) for o in outs]
      _ops.scan_bidi_bwd(dyf.contiguous().to(DEV), dyb.contiguous().to(DEV),
                         *d, *dense, cu)
      for a, b in zip(outs, dense):
        assert torch.equal(a, b)
      dxf, dgf = oracle.scan_bwd(npf(dyf), npf(gf), npf(hf), cu_of(lens), True)
      dxb, dgb = oracle.scan_bwd(npf(dyb), npf(gb), npf(hb), cu_of(lens), False)
      check_close(outs[0], dxf, dtype, "dx fwd")
      check_close(outs[1], dgf, dtype, "dg fwd")
      check_close(outs[2], dxb, dtype, "dx bwd")
      check_close(outs[3], dgb, dtype, "dg bwd")
  finally:
    _ops.USE_WORKSPACE = prev


@pytest.mark.parametrize("compiled", [False, True], ids=["eager", "compiled"])
@pytest.mark.parametrize("use", ["both", "fwd-only", "bwd-only", "mixed"])
def test_bidi_time_constant_gradients(compiled, use):
  """Bidirectional API with gradients that are constant along time
  (out.sum()), with one branch unused (its gradient is None), and with one
  dense gradient: every combination matches the materialised gradients bit
  for bit and the oracle."""
  lens, C, dtype = [3000, 17, 5000], 80, torch.float32
  fn = (ast.scan_bidirectional_branched_compiled if compiled
        else ast.scan_bidirectional_branched)
  gf, xf = make(lens, C, dtype, seed=1, n=2, glo=0.5)
  gb, xb = make(lens, C, dtype, seed=2, n=2, glo=0.5)
  T = sum(lens)
  args = grid_args(lens, C)
  dense_b = torch.rand(C, T, generator=torch.Generator().manual_seed(9)).to(DEV)

  def run(loss_of):
    ts = [t.to(DEV).requires_grad_(True) for t in (gf, xf, gb, xb)]
    yf, yb = fn(*ts, args)
    loss_of(yf, yb)
    return (yf.detach(), yb.detach()), [t.grad for t in ts]

  ones = torch.ones(C, T, device=DEV)
  zeros = torch.zeros(C, T, device=DEV)
  losses = {
    "both": (lambda yf, yb: (yf.sum() + yb.sum()).backward(), ones, ones),
    "fwd-only": (lambda yf, yb: yf.sum().backward(), ones, zeros),
    "bwd-only": (lambda yf, yb: yb.sum().backward(), zeros, ones),
    "mixed": (lambda yf, yb: (yf.sum() + (yb * dense_b).sum()).backward(),
              ones, dense_b),
  }
  loss_of, dyf, dyb = losses[use]
  (yf, yb), got = run(loss_of)
  _, ref = run(lambda a, b: torch.autograd.backward([a, b], [dyf, dyb]))
  from associative_scan_triton import _lib
  lookback = _lib.load().asc_scan_workspace_bytes(
    len(lens), C, T, _lib.dtype_code(gf), 2) > 0
  assert not lookback
  for a, b in zip(got, ref):
    assert torch.equal(a, b)
  dxf, dgf = oracle_bwd(dyf.cpu(), gf, npf(yf), lens, causal=True)
  dxb, dgb = oracle_bwd(dyb.cpu(), gb, npf(yb), lens, causal=False)
  check_close(got[0], dgf, dtype, "dg fwd")
  check_close(got[1], dxf, dtype, "dx fwd")
  check_close(got[2], dgb, dtype, "dg bwd")
  check_close(got[3], dxb, dtype, "dx bwd")


# ---------------------------------------------------------------------------
# chained-chunk walk (segments aligned to 4096 fp32 / 8192 fp16-bf16
# elements, more than 128 items)
# ---------------------------------------------------------------------------

def _chunk(dtype):
  return 4096 if dtype == torch.float32 else 8192


def _chain_case(dtype, lens, C, rows, spin=None):
  """Forward (both directions) and backward (both) through the library with
  a workspace; checks rows `rows` against the oracle and returns the device
  results."""
  from associative_scan_triton import _lib, _ops
  lib = _lib.load()
  T = sum(lens)
  g, x, dy = make(lens, C, dtype, glo=0.5, n=3)
  cu = torch.tensor(cu_of(lens), device=DEV)
  gd, xd, dyd = g.to(DEV), x.to(DEV), dy.to(DEV)
  assert lib.asc_scan_workspace_walk(len(lens), C, T, _lib.dtype_code(gd),
                                    1) == _lib.WALK_CHAINED
  prev = lib.asc_set_lookback_spin_limit(spin) if spin is not None else None
  try:
    out = {}
    for rev in (False, True):
      h = torch.empty_like(gd)
      _ops.scan_fwd(gd, xd, h, cu, rev)
      dx, dg = torch.empty_like(gd), torch.empty_like(gd)
      _ops.scan_bwd(dyd, gd, h, dx, dg, cu, causal=not rev)
      out[rev] = (h, dx, dg)
      for r in rows:
        h_ref = oracle_fwd(g[r:r + 1], x[r:r + 1], lens, reverse=rev)
        check_close(h[r:r + 1], h_ref, dtype, f"h row {r} rev={rev}")
        dx_ref, dg_ref = oracle_bwd(dy[r:r + 1], g[r:r + 1], npf(h[r:r + 1]),
                                    lens, causal=not rev)
        check_close(dx[r:r + 1], dx_ref, dtype, f"dx row {r} rev={rev}")
        check_close(dg[r:r + 1], dg_ref, dtype, f"dg row {r} rev={rev}")
    return out
  finally:
    if prev is not None:
      lib.asc_set_lookback_spin_limit(prev)


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_chain_walk_parity_and_reproducible(dtype):
  """Aligned segments of 1-3 chunks over 130 rows: every row matches the
  oracle, and a second run gives the same bits (the carries are composed in
  a fixed order)."""
  CH = _chunk(dtype)
  lens = [2 * CH, CH, 3 * CH]
  a = _chain_case(dtype, lens, 130, rows=range(130))
  b = _chain_case(dtype, lens, 130, rows=[])
  for rev in (False, True):
    for u, v in zip(a[rev], b[rev]):
      assert torch.equal(u, v)


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
def test_chain_walk_mixed_segments(dtype):
  """Same row width, some segment edges off the chunk grid: the per-item
  walk (launched first) takes the segments with an edge off the grid, the
  chained walk the others, in one call; both must match the oracle."""
  CH = _chunk(dtype)
  _chain_case(dtype, [2 * CH + 5, CH - 5, 3 * CH], 130, rows=[0, 77, 129])
  _chain_case(dtype, [2 * CH, CH, 3 * CH - 1, 1], 130, rows=[0, 129])
  _chain_case(dtype, [2 * CH + 5, CH - 5, 3 * CH + 1, CH - 1], 130,
              rows=[0, 129])   # no segment aligned: the chained grid idles


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16],
                         ids=["f32", "bf16"])
def test_chain_walk_mixed_with_checkpoint(dtype):
  """A chunk-aligned segment of 70 chunks (past the 64-chunk checkpoint)
  between short unaligned ones: the chained walk carries across its
  checkpoint while the per-item walk takes its neighbours."""
  CH = _chunk(dtype)
  _chain_case(dtype, [CH - 3, 3, 70 * CH, CH + 5, CH - 5], 130,
              rows=[0, 64, 129])


@pytest.mark.parametrize("case", ["300-aligned", "300-mixed", "5000-aligned"])
def test_chain_walk_many_segments(case):
  """More segments than one wave surveys at once: 300 chunk-aligned ones
  (the per-item walk's first wave surveys them in two batches: the chained
  walk reads each chunk before looking it up), 300 with two edges off the
  grid (per-chunk lookups), 5000 (past what is surveyed: per-chunk lookups
  and per-item tests)."""
  CH = 4096
  if case == "300-aligned":
    lens, C = [CH * (1 + i % 3) for i in range(300)], 2
  elif case == "300-mixed":
    lens, C = [CH * (1 + i % 3) for i in range(300)], 2
    lens[100] += 9
    lens[101] -= 9
  else:
    lens, C = [CH] * 5000, 1
  _chain_case(torch.float32, lens, C, rows=range(C))


def test_chain_walk_dirty_workspace():
  """A workspace whose every slot reads as published (as a previous call or
  unrelated data may leave it): the per-item walk launched first clears the
  slots, so the chained walk's carries are still right, forward and
  backward, and the results equal a clean workspace's bit for bit."""
  from associative_scan_triton import _lib
  lib = _lib.load()
  CH = 4096
  lens, C = [3 * CH, 66 * CH, CH], 130
  S, T = len(lens), sum(lens)
  g, x, dy = make(lens, C, torch.float32, glo=0.5, n=3)
  gd, xd, dyd = g.to(DEV), x.to(DEV), dy.to(DEV)
  cu = torch.tensor(cu_of(lens), device=DEV)
  code = _lib.dtype_code(gd)
  assert lib.asc_scan_workspace_walk(S, C, T, code, 1) == _lib.WALK_CHAINED
  nb = lib.asc_scan_workspace_bytes(S, C, T, code, 1)
  stream = torch.cuda.current_stream().cuda_stream
  outs = []
  for dirty in (False, True):
    ws = torch.zeros(nb // 8, dtype=torch.int64, device=DEV)
    if dirty:
      ws.fill_((2 << 32) | 0x3F800000)   # status "inclusive", value 1.0
    h, dx, dg = (torch.empty_like(gd) for _ in range(3))
    assert lib.asc_scan_fwd(gd.data_ptr(), xd.data_ptr(), h.data_ptr(), None,
                            cu.data_ptr(), 1, S, C, T, code, 0, ws.data_ptr(),
                            nb, stream) == 0
    if dirty:
      ws.fill_((2 << 32) | 0x3F800000)
    assert lib.asc_scan_bwd(dyd.data_ptr(), gd.data_ptr(), h.data_ptr(),
                            dx.data_ptr(), dg.data_ptr(), cu.data_ptr(), 1, S,
                            C, T, code, 1, ws.data_ptr(), nb, stream) == 0
    torch.cuda.synchronize()
    outs.append((h, dx, dg))
  for a, b in zip(*outs):
    assert torch.equal(a, b)
  h, dx, dg = outs[1]
  for r in (0, 129):
    sl = slice(r, r + 1)
    check_close(h[sl], oracle_fwd(g[sl], x[sl], lens), torch.float32, "h")
    dx_ref, dg_ref = oracle_bwd(dy[sl], g[sl], npf(h[sl]), lens, causal=True)
    check_close(dx[sl], dx_ref, torch.float32, "dx")
    check_close(dg[sl], dg_ref, torch.float32, "dg")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16],
                         ids=["f32", "bf16"])
def test_chain_walk_checkpoints(dtype):
  """A segment of 70 chunks crosses the 64-chunk checkpoint (chunks past it
  take their carry from the checkpoint's inclusive value); an empty segment
  is skipped."""
  CH = _chunk(dtype)
  _chain_case(dtype, [70 * CH, 0, CH], 130, rows=[0, 65, 129])
  _chain_case(dtype, [3 * CH, 60 * CH, 7 * CH], 129, rows=[3, 128])


def test_chain_walk_bounded_wait_fallback():
  """Spin limit 0: every chunk that finds a predecessor's slot empty scans
  its segment's prefix itself; results still match the oracle."""
  CH = 4096
  _chain_case(torch.float32, [3 * CH, 66 * CH, CH], 130, rows=[0, 64, 129],
              spin=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16],
                         ids=["f32", "bf16"])
@pytest.mark.parametrize("mixed", [False, True], ids=["aligned", "mixed"])
def test_chain_walk_bidirectional(dtype, mixed):
  """Both branches with long segments over 130 rows (one chained launch per
  branch), all chunk-aligned or some with an edge off the chunk grid (those
  run the per-item walk, both branches in one grid)."""
  from associative_scan_triton import _lib, _ops
  CH = _chunk(dtype)
  lens = [CH + 3, 2 * CH - 3, 2 * CH] if mixed else [CH, 2 * CH]
  C = 130
  gf, xf, dyf = make(lens, C, dtype, seed=1, glo=0.5, n=3)
  gb, xb, dyb = make(lens, C, dtype, seed=2, glo=0.5, n=3)
  T = sum(lens)
  assert _lib.load().asc_scan_workspace_walk(len(lens), C, T,
                                             _lib.dtype_code(gf), 2) == _lib.WALK_CHAINED
  cu = torch.tensor(cu_of(lens), device=DEV)
  d = [t.to(DEV) for t in (gf, xf, gb, xb, dyf, dyb)]
  hf, hb = torch.empty_like(d[0]), torch.empty_like(d[0])
  _ops.scan_bidi_fwd(d[0], d[1], d[2], d[3], hf, hb, cu)
  outs = [torch.empty_like(d[0]) for _ in range(4)]
  _ops.scan_bidi_bwd(d[4], d[5], d[0], d[2], hf, hb, *outs, cu)
  for r in (0, 64, 129):
    sl = slice(r, r + 1)
    check_close(hf[sl], oracle_fwd(gf[sl], xf[sl], lens), dtype, "hf")
    check_close(hb[sl], oracle_fwd(gb[sl], xb[sl], lens, reverse=True), dtype, "hb")
    dxf, dgf = oracle_bwd(dyf[sl], gf[sl], npf(hf[sl]), lens, causal=True)
    dxb, dgb = oracle_bwd(dyb[sl], gb[sl], npf(hb[sl]), lens, causal=False)
    check_close(outs[0][sl], dxf, dtype, "dxf")
    check_close(outs[1][sl], dgf, dtype, "dgf")
    check_close(outs[2][sl], dxb, dtype, "dxb")
    check_close(outs[3][sl], dgb, dtype, "dgb")


# ---------------------------------------------------------------------------
# two items per wave, one per 32-lane half (a mean segment of at most 128
# fp32 / 256 fp16-bf16 elements, 16-byte aligned tensors, no workspace)
# ---------------------------------------------------------------------------

# (means of up to one step of a half, and a few geometries just past it,
# which run one wave per item)
GROUP_LENS = {
  "uniform": [128] * 8,
  # items of several steps of a half beside one-element and empty ones
  "ragged": [1, 300, 7, 0, 129, 64, 2, 33, 97],
  "odd": [5, 9, 100],
  "uniform2": [256] * 6,
  "ragged2": [1, 700, 150, 0, 255, 257, 3, 400, 33],
  "uniform2-half": [512] * 5,
  # means within a quarter's step (16 lanes x 1 vector: 64 fp32 / 128
  # fp16-bf16 elements): four items per wave, some of them absent or empty
  "quad": [64] * 8,
  "quad-ragged": [1, 40, 64, 0, 17, 63, 2, 130, 9],
}


def _group_geometry(lens, dtype):
  per_half = 128 if dtype == torch.float32 else 256
  assert sum(lens) <= len(lens) * 4 * per_half


@pytest.fixture
def no_workspace():
  from associative_scan_triton import _ops
  prev = _ops.USE_WORKSPACE
  _ops.USE_WORKSPACE = False
  yield
  _ops.USE_WORKSPACE = prev


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("name", sorted(GROUP_LENS))
@pytest.mark.parametrize("C", [7, 130])
def test_group_walk_parity(dtype, name, C, no_workspace):
  """The group walk (two or four short items per wave): forward (both
  directions) and dense backward (both) against the oracle; an item count
  that is not a multiple of the group count leaves the last wave short."""
  from associative_scan_triton import _ops
  lens = GROUP_LENS[name]
  _group_geometry(lens, dtype)
  g, x, dy = make(lens, C, dtype, glo=0.5, n=3)
  gd, xd, dyd = g.to(DEV), x.to(DEV), dy.to(DEV)
  cu = torch.tensor(cu_of(lens), device=DEV)
  for rev in (False, True):
    h = torch.empty_like(xd)
    _ops.scan_fwd(gd, xd, h, cu, reverse=rev)
    check_close(h, oracle_fwd(g, x, lens, reverse=rev), dtype, f"h rev={rev}")
    dx, dg = torch.empty_like(xd), torch.empty_like(xd)
    _ops.scan_bwd(dyd, gd, h, dx, dg, cu, causal=not rev)
    dx_ref, dg_ref = oracle_bwd(dy, g, npf(h), lens, causal=not rev)
    check_close(dx, dx_ref, dtype, f"dx rev={rev}")
    check_close(dg, dg_ref, dtype, f"dg rev={rev}")


@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("name", ["ragged", "odd", "ragged2", "quad-ragged"])
def test_group_walk_bidirectional_and_row_gradient(dtype, name, no_workspace):
  """Both branches in one launch (each wave's items from one branch),
  and a gradient constant along time (each half reads its row's value):
  bits equal to the dense gradient's, values against the oracle."""
  from associative_scan_triton import _ops
  lens, C = GROUP_LENS[name], 9
  _group_geometry(lens, dtype)
  gf, xf, dyf = make(lens, C, dtype, seed=1, glo=0.5, n=3)
  gb, xb, dyb = make(lens, C, dtype, seed=2, glo=0.5, n=3)
  cu = torch.tensor(cu_of(lens), device=DEV)
  d = [t.to(DEV) for t in (gf, xf, gb, xb, dyf, dyb)]
  hf, hb = torch.empty_like(d[0]), torch.empty_like(d[0])
  _ops.scan_bidi_fwd(d[0], d[1], d[2], d[3], hf, hb, cu)
  check_close(hf, oracle_fwd(gf, xf, lens), dtype, "hf")
  check_close(hb, oracle_fwd(gb, xb, lens, reverse=True), dtype, "hb")
  outs = [torch.empty_like(d[0]) for _ in range(4)]
  _ops.scan_bidi_bwd(d[4], d[5], d[0], d[2], hf, hb, *outs, cu)
  dxf, dgf = oracle_bwd(dyf, gf, npf(hf), lens, causal=True)
  dxb, dgb = oracle_bwd(dyb, gb, npf(hb), lens, causal=False)
  check_close(outs[0], dxf, dtype, "dxf")
  check_close(outs[1], dgf, dtype, "dgf")
  check_close(outs[2], dxb, dtype, "dxb")
  check_close(outs[3], dgb, dtype, "dgb")
  # one value per row, three elements apart, against the same value dense
  rows = torch.randn(C, 3, generator=torch.Generator().manual_seed(5)).to(dtype)
  T = sum(lens)
  dense = rows[:, 1:2].expand(C, T).contiguous()
  dx1, dg1, dx2, dg2 = (torch.empty_like(d[0]) for _ in range(4))
  _ops.scan_bwd_rowgrad(rows.to(DEV)[:, 1], 3, d[0], hf, dx1, dg1, cu, True)
  _ops.scan_bwd(dense.to(DEV), d[0], hf, dx2, dg2, cu, causal=True)
  assert torch.equal(dx1, dx2) and torch.equal(dg1, dg2)
  dx_ref, dg_ref = oracle_bwd(dense, gf, npf(hf), lens, causal=True)
  check_close(dx1, dx_ref, dtype, "dx (row gradient)")
  check_close(dg1, dg_ref, dtype, "dg (row gradient)")


# ---------------------------------------------------------------------------
# HIP graph capture
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("C,lens", [(2, [5000, 3000]), (80, [700, 300]),
                                    (130, [8192, 4096])],
                         ids=["lookback", "per-item", "chained"])
def test_graph_capture_replay(C, lens):
  """Forward + backward captured in one graph (the look-back and chained
  walks clear their workspace with a kernel, not a memset) and replayed
  with fresh inputs and eager launches in between; every replay matches the
  oracle, and the reproducible walks (per-item, chained) match the eager
  launch bit for bit."""
  from associative_scan_triton import _ops
  T = sum(lens)
  cu = torch.tensor(cu_of(lens), device=DEV)
  g = torch.empty(C, T, device=DEV)
  x, dy = torch.empty_like(g), torch.empty_like(g)
  h, dx, dg = torch.empty_like(g), torch.empty_like(g), torch.empty_like(g)

  def step():
    _ops.scan_fwd(g, x, h, cu, reverse=False)
    _ops.scan_bwd(dy, g, h, dx, dg, cu, causal=True)

  gen = torch.Generator(device=DEV).manual_seed(9)

  def fresh():
    g.copy_(torch.rand(C, T, device=DEV, generator=gen).mul_(0.5).add_(0.5))
    x.copy_(torch.randn(C, T, device=DEV, generator=gen))
    dy.copy_(torch.rand(C, T, device=DEV, generator=gen))

  fresh()
  side = torch.cuda.Stream()
  side.wait_stream(torch.cuda.current_stream())
  with torch.cuda.stream(side):
    step()
  torch.cuda.current_stream().wait_stream(side)
  graph = torch.cuda.CUDAGraph()
  with torch.cuda.graph(graph):
    step()
  from associative_scan_triton import _lib
  walk = _lib.load().asc_scan_workspace_walk(len(lens), C, T, 0, 1)
  assert walk == {2: _lib.WALK_LOOKBACK, 80: 0, 130: _lib.WALK_CHAINED}[C]
  lookback = walk == _lib.WALK_LOOKBACK
  for _ in range(4):
    fresh()
    graph.replay()
    torch.cuda.synchronize()
    got = [t.clone() for t in (h, dx, dg)]
    gs, xs, dys = g.cpu(), x.cpu(), dy.cpu()
    check_close(got[0], oracle_fwd(gs, xs, lens), torch.float32, "h (replay)")
    dx_ref, dg_ref = oracle.scan_bwd(npf(dys), npf(gs), npf(got[0]), cu_of(lens), True)
    check_close(got[1], dx_ref, torch.float32, "dx (replay)")
    check_close(got[2], dg_ref, torch.float32, "dg (replay)")
    step()
    torch.cuda.synchronize()
    if not lookback:
      assert all(torch.equal(a, b) for a, b in zip(got, (h, dx, dg)))


# ---------------------------------------------------------------------------
# shift_pad: the vectorised kernel (data and out of one phase) and the
# element kernel (different phases), rows that straddle vectors, several
# chunks per row, both edge rules
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("backward", [True, False])
@pytest.mark.parametrize("wrap", [True, False])
@pytest.mark.parametrize("offsets", [(0, 0), (1, 1), (3, 3), (1, 0)],
                         ids=["aligned", "phase1", "phase3", "mixed"])
def test_shift_pad_layouts(dtype, backward, wrap, offsets):
  from associative_scan_triton import _ops
  lens = [1, 700, 3, 5001, 2, 1300]          # rows of 7007: not a multiple of 4 or 8
  C, L = 9, sum(lens)
  gen = torch.Generator().manual_seed(17)
  data = torch.randn(C, L, generator=gen).to(dtype)
  cu_np = cu_of(lens)
  cu = torch.tensor(cu_np, device=DEV, dtype=torch.int32)
  od, oo = offsets
  dbuf = torch.zeros(C * L + 8, dtype=dtype, device=DEV)
  obuf = torch.full((C * L + 8,), 7.0, dtype=dtype, device=DEV)
  dv = dbuf[od:od + C * L].view(C, L)
  ov = obuf[oo:oo + C * L].view(C, L)
  dv.copy_(data.to(DEV))
  _ops.shift_pad(dv, ov, cu, -2.5, backward=backward, wrap=wrap)
  ref = oracle.shift_pad(npf(data), cu_np, -2.5, backward, wrap=wrap)
  assert torch.equal(ov.cpu(), torch.from_numpy(ref).to(dtype))
  # nothing outside the output view is written
  assert torch.all(obuf[:oo] == 7.0) and torch.all(obuf[oo + C * L:] == 7.0)


def test_shift_pad_negative_boundary_and_raw_bits():
  """A zero-length first segment puts the forward pad at position -1, which
  counts from the row end (torch indexing in the reference); values move
  as raw bits, NaN payloads included."""
  from associative_scan_triton import _ops
  C, L = 3, 2051
  raw = torch.randint(-2**31, 2**31 - 1, (C, L), generator=torch.Generator().manual_seed(2),
                      dtype=torch.int32)
  raw[0, 5] = 0x7f800001          # a signalling NaN
  raw[1, 9] = -0x00400001         # a negative NaN with a payload (0xffbfffff)
  data = raw.view(torch.float32)
  cu_np = np.array([0, 0, 700, L])
  cu = torch.tensor(cu_np, device=DEV)
  for backward in (True, False):
    out = torch.empty(C, L, device=DEV)
    _ops.shift_pad(data.to(DEV), out, cu, 0.0, backward=backward, wrap=False)
    idx = torch.arange(L)
    src = (idx - 1).clamp(min=0) if backward else (idx + 1).clamp(max=L - 1)
    exp = raw[:, src].clone()
    pads = cu_np[:-1] if backward else cu_np[1:] - 1
    for q in pads:
      exp[:, int(q) % L] = 0      # pad 0.0 has all-zero bits
    assert torch.equal(out.cpu().view(torch.int32), exp)
