"""Pins the CPU oracle (oracle/) before any GPU result is judged against it.

Every oracle function is checked by something other than a retyped copy of
its own formula:

* scan_fwd (+ gate product): the reference's known-answer vectors
  (tests/golden/known_answers.json, from test_scan_kernels.py and
  test_scan_causal.py); bit equality with the reference's gold-label method
  run in torch fp64 (test_scan_dtypes.py:26-38); closed forms (geometric
  series, cumsum, cumprod); reverse = flip o forward o flip
  (test_scan_dtypes.py:175-177); segment independence.
* scan_bwd: the reference's known gradients (test_scan_causal.py:59-64);
  torch autograd through an fp64 Python loop (the brute force of
  test_scan_kernels.py:900-918) for causal and reverse scans and varlen
  packing; the reference's hand derivation on its two 3-vectors.
* shift_pad: the reference's vectors (test_shift_pad.py) and torch.roll +
  mask (_shift_pad.py:41-53) on random data.
* planted mistakes (a dropped term, a wrong neighbour index, a missing
  segment reset) in copies of the oracle must fail these checks.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle

GOLD = json.loads(
  (Path(__file__).parent / "golden" / "known_answers.json").read_text())


def _allclose(got, exp, rtol, atol):
  return np.allclose(np.asarray(got, float), np.asarray(exp, float),
                     rtol=rtol, atol=atol)


# ---------------------------------------------------------------------------
# known-answer vectors
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", GOLD["forward"], ids=lambda c: c["name"])
@pytest.mark.parametrize("impl", ["c", "numpy"])
def test_forward_golden(case, impl):
  g = np.array(case["g"], float)
  x = np.array(case["x"], float)
  cu = case["cu"]
  C = case["channels"]
  if impl == "c":
    h, a = oracle.scan_fwd(g, x, cu, case["reverse"], C, gate_prod=True)
    if "A" in case:
      assert _allclose(a, case["A"], case["rtol"], case["atol"])
  else:
    h = oracle.np_scan_fwd(g, x, cu, case["reverse"], C)
  assert _allclose(h, case["h"], case["rtol"], case["atol"])


@pytest.mark.parametrize("case", GOLD["causal_grad"], ids=lambda c: c["name"])
def test_causal_grad_golden(case):
  g = np.array(case["g"], float)
  x = np.array(case["x"], float)
  h = oracle.scan_fwd(g, x, case["cu"])
  assert _allclose(h, case["h"], case["rtol"], case["atol"])
  dy = np.ones_like(x)  # d(out.sum())/d(out)
  for dx, dg in (oracle.scan_bwd(dy, g, h, case["cu"]),
                 oracle.np_scan_bwd(dy, g, h, case["cu"])):
    assert _allclose(dx, case["dx"], case["rtol"], case["atol"])
    assert _allclose(dg, case["dg"], case["rtol"], case["atol"])


def _loop_grads(g, x, dy, reverse=False):
  """torch.func-style brute force: autograd through a python loop in fp64
  (test_scan_kernels.py:900-918, extended to a reverse loop)."""
  g = torch.tensor(g, dtype=torch.float64, requires_grad=True)
  x = torch.tensor(x, dtype=torch.float64, requires_grad=True)
  n = len(x)
  hs = [None] * n
  h = torch.zeros((), dtype=torch.float64)
  order = range(n - 1, -1, -1) if reverse else range(n)
  for i in order:
    h = g[i] * h + x[i]
    hs[i] = h
  y = torch.stack(hs)
  (y * torch.tensor(dy, dtype=torch.float64)).sum().backward()
  return y.detach().numpy(), x.grad.numpy(), g.grad.numpy()


@pytest.mark.parametrize("case", GOLD["manual_grad"], ids=lambda c: c["name"])
def test_manual_grad_vectors(case):
  g, x = np.array(case["g"]), np.array(case["x"])
  y, dx_ref, dg_ref = _loop_grads(g, x, np.ones(3))
  h = oracle.scan_fwd(g, x, [0, 3])
  dx, dg = oracle.scan_bwd(np.ones(3), g, h, [0, 3])
  np.testing.assert_allclose(h, y, rtol=1e-15)
  np.testing.assert_allclose(dx, dx_ref, rtol=1e-14)
  np.testing.assert_allclose(dg, dg_ref, rtol=1e-14, atol=1e-15)
  # the reference's hand derivation (test_scan_kernels.py:873-897)
  assert dg[0] == 0.0
  assert dx[2] == 1.0
  assert np.isclose(dx[1], 1 + g[2])
  assert np.isclose(dx[0], 1 + g[1] * (1 + g[2]))


# ---------------------------------------------------------------------------
# brute force autograd on random packed inputs
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("lens", [[1], [5], [3, 1, 7], [16, 2, 9, 1]])
def test_backward_brute_force(reverse, lens):
  rng = np.random.default_rng(7 + len(lens) + 3 * reverse)
  C = 3
  T = sum(lens)
  cu = np.concatenate([[0], np.cumsum(lens)])
  g = rng.uniform(0.2, 1.3, (C, T))
  x = rng.normal(size=(C, T))
  dy = rng.normal(size=(C, T))
  h = oracle.scan_fwd(g, x, cu, reverse)
  dx, dg = oracle.scan_bwd(dy, g, h, cu, causal=not reverse)
  for c in range(C):
    for s in range(len(lens)):
      b, e = cu[s], cu[s + 1]
      y, dx_ref, dg_ref = _loop_grads(g[c, b:e], x[c, b:e], dy[c, b:e], reverse)
      np.testing.assert_allclose(h[c, b:e], y, rtol=1e-13, atol=1e-14)
      np.testing.assert_allclose(dx[c, b:e], dx_ref, rtol=1e-12, atol=1e-13)
      np.testing.assert_allclose(dg[c, b:e], dg_ref, rtol=1e-12, atol=1e-13)


# ---------------------------------------------------------------------------
# the reference's gold-label method, bit for bit
# ---------------------------------------------------------------------------

def _torch_gold(gates, tokens):
  """test_scan_dtypes.py:26-38, run in torch fp64."""
  g = gates.to(torch.float64)
  x = tokens.to(torch.float64)
  _, T = g.shape
  out = torch.empty_like(x)
  out[:, 0] = x[:, 0]
  for t in range(1, T):
    out[:, t] = g[:, t] * out[:, t - 1] + x[:, t]
  return out


@pytest.mark.parametrize("T", [1, 33, 700])
def test_forward_matches_torch_gold_bitwise(T):
  gen = torch.Generator().manual_seed(1155)
  g = torch.rand(4, T, generator=gen)
  x = torch.randn(4, T, generator=gen)
  gold = _torch_gold(g, x).numpy()
  h = oracle.scan_fwd(g.numpy(), x.numpy(), [0, T])
  assert np.array_equal(h, gold)
  assert np.array_equal(oracle.np_scan_fwd(g.numpy(), x.numpy(), [0, T]), gold)
  # reverse via flip (test_scan_dtypes.py:175-177)
  gold_r = _torch_gold(g.flip(-1), x.flip(-1)).flip(-1).numpy()
  assert np.array_equal(oracle.scan_fwd(g.numpy(), x.numpy(), [0, T], True),
                        gold_r)


def test_c_and_numpy_oracles_agree_bitwise():
  rng = np.random.default_rng(3)
  lens = [1, 2, 17, 64, 5]
  cu = np.concatenate([[0], np.cumsum(lens)])
  C, T = 4, sum(lens)
  g, x, dy = (rng.uniform(0, 1.1, (C, T)), rng.normal(size=(C, T)),
              rng.normal(size=(C, T)))
  for rev in (False, True):
    h = oracle.scan_fwd(g, x, cu, rev)
    assert np.array_equal(h, oracle.np_scan_fwd(g, x, cu, rev))
    dx, dg = oracle.scan_bwd(dy, g, h, cu, causal=not rev)
    dx2, dg2 = oracle.np_scan_bwd(dy, g, h, cu, causal=not rev)
    assert np.array_equal(dx, dx2) and np.array_equal(dg, dg2)


# ---------------------------------------------------------------------------
# closed forms and invariants
# ---------------------------------------------------------------------------

def test_geometric_series_closed_form():
  c, n = 0.75, 50
  h = oracle.scan_fwd(np.full(n, c), np.ones(n), [0, n])
  t = np.arange(n)
  np.testing.assert_allclose(h, (1 - c ** (t + 1)) / (1 - c), rtol=1e-14)


def test_unit_gates_give_segmented_cumsum_and_cumprod():
  rng = np.random.default_rng(1)
  lens = [4, 1, 9]
  cu = np.concatenate([[0], np.cumsum(lens)])
  x = rng.normal(size=(2, sum(lens)))
  g = rng.uniform(0.5, 1.5, (2, sum(lens)))
  h = oracle.scan_fwd(np.ones_like(x), x, cu)
  _, a = oracle.scan_fwd(g, x, cu, gate_prod=True)
  _, ar = oracle.scan_fwd(g, x, cu, reverse=True, gate_prod=True)
  for s in range(3):
    b, e = cu[s], cu[s + 1]
    np.testing.assert_allclose(h[:, b:e], np.cumsum(x[:, b:e], axis=1), rtol=1e-13)
    np.testing.assert_allclose(a[:, b:e], np.cumprod(g[:, b:e], axis=1), rtol=1e-14)
    np.testing.assert_allclose(
      ar[:, b:e], np.cumprod(g[:, b:e][:, ::-1], axis=1)[:, ::-1], rtol=1e-14)
  assert np.all(oracle.scan_fwd(g, np.zeros_like(x), cu) == 0)


def test_segments_are_independent():
  rng = np.random.default_rng(2)
  lens = [3, 8, 1, 5]
  cu = np.concatenate([[0], np.cumsum(lens)])
  g, x = rng.uniform(0, 1, (2, sum(lens))), rng.normal(size=(2, sum(lens)))
  h = oracle.scan_fwd(g, x, cu)
  perm = [2, 0, 3, 1]
  pieces = lambda a: [a[:, cu[s]:cu[s + 1]] for s in range(len(lens))]  # noqa: E731
  g2 = np.concatenate([pieces(g)[p] for p in perm], axis=1)
  x2 = np.concatenate([pieces(x)[p] for p in perm], axis=1)
  cu2 = np.concatenate([[0], np.cumsum([lens[p] for p in perm])])
  h2 = oracle.scan_fwd(g2, x2, cu2)
  assert np.array_equal(np.concatenate([pieces(h)[p] for p in perm], axis=1), h2)


def test_op_is_associative():
  """test_scan_kernels.py:23-43 with the package's combine op."""
  from associative_scan_triton import op
  for a, b, c in [((0.5, 0.3), (0.6, 0.9), (0.7, 0.8)),
                  ((0.6, 0.9), (0.5, 0.3), (0.7, 0.8)),
                  ((0.6, 0.9), (0.7, 0.8), (0.5, 0.3))]:
    ab = op(a[0], a[1], b[0], b[1])
    abc1 = op(ab[0], ab[1], c[0], c[1])
    bc = op(b[0], b[1], c[0], c[1])
    abc2 = op(a[0], a[1], bc[0], bc[1])
    assert np.allclose(abc1, abc2)


# ---------------------------------------------------------------------------
# shift_pad
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", GOLD["shift_pad"]["cases"], ids=lambda c: c["name"])
@pytest.mark.parametrize("backward", [True, False])
@pytest.mark.parametrize("wrap", [True, False])
def test_shift_pad_golden(case, backward, wrap):
  pad = GOLD["shift_pad"]["pad"]
  exp = case["backward"] if backward else case["forward"]
  out = oracle.shift_pad(case["data"], case["cu"], pad, backward, wrap)
  assert np.array_equal(out, np.array(exp))
  assert np.array_equal(
    oracle.np_shift_pad(case["data"], case["cu"], pad, backward, wrap), out)


@pytest.mark.parametrize("backward", [True, False])
def test_shift_pad_matches_roll_and_mask(backward):
  """_shift_pad.py:41-53 in torch on random data."""
  gen = torch.Generator().manual_seed(5)
  data = torch.randn(6, 40, generator=gen, dtype=torch.float64)
  cu = torch.tensor([0, 3, 4, 19, 40])
  ref = torch.roll(data, shifts=1 if backward else -1, dims=-1)
  mask = torch.zeros(40, dtype=torch.bool)
  if backward:
    mask[cu[:-1]] = True
  else:
    mask[cu[1:] - 1] = True
  ref[:, mask] = 2.5
  out = oracle.shift_pad(data.numpy(), cu.numpy(), 2.5, backward, wrap=True)
  assert np.array_equal(out, ref.numpy())


# ---------------------------------------------------------------------------
# planted mistakes: each must be caught by the checks above
# ---------------------------------------------------------------------------

def _bwd_wrong_gate_index(dy, g, h, cu):
  """Bug: uses g[t] instead of g[t+1] (unshifted gates)."""
  dx = np.zeros_like(dy)
  dg = np.zeros_like(dy)
  for s in range(len(cu) - 1):
    b, e = cu[s], cu[s + 1]
    for t in range(e - 1, b - 1, -1):
      dx[t] = dy[t] if t == e - 1 else dy[t] + dx[t + 1] * g[t]
      dg[t] = (0.0 if t == b else h[t - 1]) * dx[t]
  return dx, dg


def _fwd_no_reset(g, x, cu):
  """Bug: carries h across segment boundaries."""
  h = np.zeros_like(x)
  prev = 0.0
  for t in range(len(x)):
    prev = g[t] * prev + x[t]
    h[t] = prev
  return h


def _fwd_dropped_gate(g, x, cu):
  """Bug: drops the gate term (plain cumsum)."""
  h = np.zeros_like(x)
  for s in range(len(cu) - 1):
    b, e = cu[s], cu[s + 1]
    h[b:e] = np.cumsum(x[b:e])
  return h


def test_planted_mistakes_are_caught():
  case = GOLD["causal_grad"][0]
  g = np.array(case["g"])
  x = np.array(case["x"])
  cu = case["cu"]
  h = oracle.scan_fwd(g, x, cu)
  dx, dg = _bwd_wrong_gate_index(np.ones(8), g, h, cu)
  assert not _allclose(dx, case["dx"], case["rtol"], case["atol"])
  assert not _allclose(_fwd_no_reset(g, x, cu), case["h"], 1e-4, 1e-4)
  assert not _allclose(_fwd_dropped_gate(g, x, cu), case["h"], 1e-4, 1e-4)
  # the brute force also catches the wrong gate index on random data
  rng = np.random.default_rng(0)
  g2, x2, dy2 = rng.uniform(0.2, 1, 6), rng.normal(size=6), rng.normal(size=6)
  _, dx_ref, _ = _loop_grads(g2, x2, dy2)
  h2 = oracle.scan_fwd(g2, x2, [0, 6])
  assert not np.allclose(_bwd_wrong_gate_index(dy2, g2, h2, [0, 6])[0], dx_ref)


# ---------------------------------------------------------------------------
# the CPU baseline's function (fp32 storage, fp64 accumulation)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("threads", [1, 4])
def test_fwd_bwd_f32io_is_the_oracle_rounded(threads):
  """fwd_bwd_f32io accumulates in fp64 from the fp32-stored inputs and
  rounds each output once, so h and dx are the fp64 oracle's values rounded
  to fp32, bit for bit, and dg is the oracle's dg of the stored fp32 states
  rounded; checked against both restatements (C and numpy) on varlen
  packing with an empty segment, for any thread count."""
  rng = np.random.default_rng(7)
  lens = [1, 37, 0, 300, 2, 1029]
  cu = np.concatenate([[0], np.cumsum(lens)])
  C, T = 6, int(cu[-1])
  g = rng.uniform(0.5, 1.0, (C, T)).astype(np.float32)
  x = rng.standard_normal((C, T)).astype(np.float32)
  dy = rng.standard_normal((C, T)).astype(np.float32)
  h, dx, dg = oracle.fwd_bwd_f32io(g, x, dy, cu, C, threads)
  for fwd, bwd in ((oracle.scan_fwd, oracle.scan_bwd),
                   (oracle.np_scan_fwd, oracle.np_scan_bwd)):
    h64 = fwd(g, x, cu)
    assert np.array_equal(h, h64.astype(np.float32))
    dx64, dg64 = bwd(dy, g, h.astype(np.float64), cu)
    assert np.array_equal(dx, dx64.astype(np.float32))
    assert np.array_equal(dg, dg64.astype(np.float32))
  # a dropped gate term in the backward would not go unnoticed
  assert not np.array_equal(dx, dy)


def test_torch_method_is_the_oracle_bitwise():
  """torch_fwd_bwd_f64 (the reference's CPU method, timed by bench.py as a
  baseline) gives the C oracle's fp64 results bit for bit: both round each
  multiply and add separately."""
  rng = np.random.default_rng(11)
  lens = [1, 40, 0, 300, 2]
  cu = np.concatenate([[0], np.cumsum(lens)])
  C, T = 5, int(cu[-1])
  g = rng.uniform(0.5, 1.0, (C, T))
  x = rng.standard_normal((C, T))
  dy = rng.standard_normal((C, T))
  h, dx, dg = (t.numpy() for t in oracle.torch_fwd_bwd_f64(g, x, dy, cu))
  h_ref = oracle.scan_fwd(g, x, cu)
  dx_ref, dg_ref = oracle.scan_bwd(dy, g, h_ref, cu)
  assert np.array_equal(h, h_ref)
  assert np.array_equal(dx, dx_ref)
  assert np.array_equal(dg, dg_ref)
