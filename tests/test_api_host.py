"""Host-side behaviour of the public API (CPU only, no kernel launches).

Mirrors the reference's argument errors (AssertionError with the same
messages) and checks that there is no CPU fallback: CPU tensors are refused.
"""

import pytest
import torch

import associative_scan_triton as ast

REFERENCE_EXPORTS = [
  "op", "forward_scan_chunked", "forward_scan_onepass_pipelined",
  "forward_scan_full", "backward_scan_fused",
  "backward_scan_fused_single_chunk", "backward_scan_fused_full",
  "shift_pad", "shift_pad_compiled", "next_power_of_2", "get_grid",
  "get_static_grid", "scan_causal", "scan_causal_compiled",
  "scan_bidirectional_branched", "scan_bidirectional_branched_compiled",
]


def test_exports_match_reference():
  """Reference __init__.py:15-36 plus get_num_stages and __version__."""
  assert ast.__all__ == REFERENCE_EXPORTS
  for name in REFERENCE_EXPORTS + ["get_num_stages"]:
    assert hasattr(ast, name)
  assert ast.__version__ == "1.0.0"


def _args(C=2, T=8):
  cu = torch.tensor([0, T], dtype=torch.int32)
  return {"cu_seqlens": cu, "chunk_size": 4, "grid": ast.get_grid(2, T, 4, C)}


def test_cpu_tensors_are_refused():
  g, x = torch.rand(2, 8), torch.rand(2, 8)
  with pytest.raises(ValueError, match="HIP devices only"):
    ast.scan_causal(g, x, _args())
  with pytest.raises(ValueError, match="HIP devices only"):
    ast.scan_bidirectional_branched(g, x, g, x, _args())
  with pytest.raises(ValueError, match="HIP devices only"):
    ast.forward_scan_full(g, x, _args()["cu_seqlens"], _args()["grid"],
                          REVERSE=False, CHUNK_SIZE=4)
  with pytest.raises(ValueError, match="HIP devices only"):
    ast.shift_pad(g, torch.tensor([0, 8]))


def test_reference_assertions():
  g, x = torch.rand(2, 8), torch.rand(2, 8)
  with pytest.raises(AssertionError):
    ast.scan_causal(g, torch.rand(2, 7), _args())          # shape mismatch
  with pytest.raises(AssertionError):
    ast.scan_causal(g.t().contiguous().t(), x, _args(8, 2))  # non-contiguous
  bad = dict(_args())
  bad["grid"] = (3, 2, 2)
  with pytest.raises(AssertionError, match="cu_seqlens do not match grid"):
    ast.scan_causal(g, x, bad)
  with pytest.raises(AssertionError, match="cu_seqlens do not match grid"):
    ast.forward_scan_full(g, x, bad["cu_seqlens"], bad["grid"],
                          REVERSE=False, CHUNK_SIZE=4)
  with pytest.raises(AssertionError):
    ast.scan_bidirectional_branched(g, x, g, torch.rand(2, 7), _args())


def test_shift_pad_zero_length_message():
  """test_shift_pad.py:129-132: the check runs before any device work."""
  with pytest.raises(AssertionError, match="can't shift_pad zero-length seqments"):
    ast.shift_pad(torch.tensor([[1.0, 2.0, 3.0]]),
                  torch.tensor([0, 0, 1, 1, 3]), -1, True)


def test_custom_ops_registered():
  ns = torch.ops.associative_scan_triton
  for name in ("scan_causal_fwd", "scan_causal_bwd", "scan_bidi_fwd",
               "scan_bidi_bwd", "shift_pad"):
    assert hasattr(ns, name)


def test_fake_tensor_shapes():
  """register_fake implementations propagate shapes without a device."""
  from torch._subclasses.fake_tensor import FakeTensorMode
  with FakeTensorMode():
    g = torch.empty(4, 16)
    x = torch.empty(4, 16)
    cu = torch.empty(3, dtype=torch.int32)
    out = torch.ops.associative_scan_triton.scan_causal_fwd(g, x, cu, 1, 4, 16)
    assert out.shape == (4, 16)
    dg, dx = torch.ops.associative_scan_triton.scan_causal_bwd(
      out, g, out, cu, 1, 4, 16)
    assert dg.shape == dx.shape == (4, 16)
    of, ob = torch.ops.associative_scan_triton.scan_bidi_fwd(
      g, x, g, x, cu, 1, 4, 16)
    assert of.shape == ob.shape == (4, 16)
    r = torch.ops.associative_scan_triton.scan_bidi_bwd(
      of, ob, of, ob, g, g, cu, 1, 4, 16)
    assert len(r) == 4 and all(t.shape == (4, 16) for t in r)
    sp = torch.ops.associative_scan_triton.shift_pad(g, cu, 0.0, True)
    assert sp.shape == (4, 16)


def test_op_on_tensors():
  fl, xl = torch.tensor([0.5, 2.0]), torch.tensor([1.0, -1.0])
  fr, xr = torch.tensor([0.25, 3.0]), torch.tensor([2.0, 0.5])
  f, x = ast.op(fl, xl, fr, xr)
  assert torch.equal(f, fr * fl)
  assert torch.equal(x, fr * xl + xr)


def test_row_constant_stride_detection():
  """Which incoming gradient layouts take the one-value-per-row backward."""
  from associative_scan_triton._ops import row_constant_stride
  like = torch.empty(6, 50)
  assert row_constant_stride(torch.ones(()).expand(6, 50), like) == 0
  assert row_constant_stride(torch.ones(6, 1).expand(6, 50), like) == 1
  w = torch.ones(6, 3)[:, 1:2].expand(6, 50)       # rows 3 elements apart
  assert row_constant_stride(w, like) == 3
  assert row_constant_stride(w, like, num_channels=6) == 3
  assert row_constant_stride(w, like, num_channels=3) is None  # flat addressing
  assert row_constant_stride(torch.ones(6, 50), like) is None   # dense
  assert row_constant_stride(torch.ones(50).expand(6, 50), like) is None
  assert row_constant_stride(torch.ones(()).expand(6, 50).double(), like) is None
  flat = torch.empty(300)
  assert row_constant_stride(torch.ones(()).expand(300), flat) == 0
  assert row_constant_stride(torch.ones(300), flat) is None


def test_deterministic_mode_avoids_lookback():
  """Under torch.use_deterministic_algorithms(True) the few-item walk is
  kept only when every tensor of the call has the same address modulo 16
  bytes (the library then runs the tree walk, which composes carries in a
  fixed order; otherwise the look-back walk, whose last bits can vary from
  run to run); the chained walk, whose carries are composed in a fixed
  order, is always kept."""
  from associative_scan_triton import _lib, _ops
  lib = _lib.load()
  base = torch.empty(64)
  same = (base[0:8], base[4:12], torch.empty(8))   # 0, 16, 0 mod 16 bytes
  mixed = (base[0:8], base[1:9])                   # 0 and 4 mod 16 bytes
  assert _ops._walk(lib, 2, 4, 1_000_000, 0, 1) == _lib.WALK_LOOKBACK
  assert _ops._walk(lib, 2, 4, 1_000_000, 0, 1, mixed) == _lib.WALK_LOOKBACK
  prev = torch.are_deterministic_algorithms_enabled()
  torch.use_deterministic_algorithms(True)
  try:
    assert _ops._walk(lib, 2, 4, 1_000_000, 0, 1) == 0
    assert _ops._walk(lib, 2, 4, 1_000_000, 0, 1, mixed) == 0
    assert _ops._walk(lib, 2, 4, 1_000_000, 0, 1, same) == _lib.WALK_LOOKBACK
    assert _ops._walk(lib, 8, 1536, 524288, 0, 1) == _lib.WALK_CHAINED
  finally:
    torch.use_deterministic_algorithms(prev)
  assert _ops._walk(lib, 2, 4, 1_000_000, 0, 1) == _lib.WALK_LOOKBACK
