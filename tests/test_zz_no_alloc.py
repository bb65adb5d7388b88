"""The allocation-free forward entry point (asc_scan_fwd_noalloc) against
asc_scan_fwd given a torch-allocated workspace, through the C ABI.

Two calls in a row on each walk that uses a workspace, the second with a
smaller input (the static buffer keeps the first call's slots, which the
second must clear): the chained walk and the few-item tree walk (both
reproducible: bit for bit), the look-back walk (few items, an output at
another 16-byte phase than the inputs; its last bits can vary from run to
run: the fp64 oracle's tolerance, and against each other to twice it), and
a geometry that needs no workspace.  Every result is also checked against the oracle.  (A
geometry too large for the static buffer is rejected on the host before any
launch; tests/test_abi.py checks that on the CPU.)
"""

import ctypes

import pytest
import torch

from _helpers import DEV, check_close, cu_of, make, oracle_fwd
from associative_scan_triton import _lib, _ops

pytestmark = pytest.mark.gpu

# (name, dtype, C, lens, walk, out_offset): each pair of rows runs a
# geometry, then a smaller one on the same walk; out_offset (elements) puts
# the output at another 16-byte phase than the inputs
CASES = [
  ("chained", torch.float32, 130, [70 * 4096] + [4096] * 4, _lib.WALK_CHAINED, 0),
  ("chained", torch.float32, 129, [4096, 2 * 4096], _lib.WALK_CHAINED, 0),
  ("chained-bf16", torch.bfloat16, 300, [8192, 8192], _lib.WALK_CHAINED, 0),
  ("chained-bf16", torch.bfloat16, 200, [8192], _lib.WALK_CHAINED, 0),
  # edges off the chunk grid: the one-wave walk takes those segments
  ("chained-mixed", torch.float32, 130, [2 * 4096 + 5, 4096 - 5, 3 * 4096],
   _lib.WALK_CHAINED, 0),
  ("chained-mixed", torch.float32, 129, [4096 + 3, 4096 - 3], _lib.WALK_CHAINED, 0),
  ("tree", torch.float32, 5, [300000, 7, 50000], _lib.WALK_LOOKBACK, 0),
  ("tree", torch.float32, 2, [20000, 3], _lib.WALK_LOOKBACK, 0),
  ("tree-bf16", torch.bfloat16, 3, [400000, 9], _lib.WALK_LOOKBACK, 0),
  ("tree-bf16", torch.bfloat16, 1, [70001], _lib.WALK_LOOKBACK, 0),
  ("lookback", torch.float32, 5, [300000, 7, 50000], _lib.WALK_LOOKBACK, 1),
  ("lookback", torch.float32, 2, [20000, 3], _lib.WALK_LOOKBACK, 1),
  ("per-item", torch.float32, 80, [700, 1, 300], 0, 0),
  ("per-item", torch.float32, 200, [30], 0, 0),
]


def _noalloc(lib, g, x, h, cu, S, C, T, reverse):
  st = lib.asc_scan_fwd_noalloc(
    g.data_ptr(), x.data_ptr(), h.data_ptr(), None, cu.data_ptr(),
    _lib.cu_code(cu), S, C, T, _lib.dtype_code(x), int(reverse),
    torch.cuda.current_stream().cuda_stream)
  _lib.check(st)


@pytest.mark.parametrize("reverse", [False, True], ids=["causal", "reverse"])
def test_noalloc_forward_matches_workspace_entry_point(reverse):
  lib = _lib.load()
  for i, (name, dtype, C, lens, walk, off) in enumerate(CASES):
    S, T = len(lens), sum(lens)
    code = _lib.dtype_code(torch.empty((), dtype=dtype))
    assert lib.asc_scan_workspace_walk(S, C, T, code, 1) == walk, name
    g, x = make(lens, C, dtype, seed=100 + i, glo=0.5)
    gd, xd = g.to(DEV), x.to(DEV)
    cu = torch.tensor(cu_of(lens), device=DEV)
    def out_buffer():
      buf = torch.full((C * T + off,), float("nan"), dtype=dtype, device=DEV)
      return buf[off:].view(C, T)
    ref = out_buffer()
    _ops.scan_fwd(gd, xd, ref, cu, reverse)        # torch workspace
    h = out_buffer()
    _noalloc(lib, gd, xd, h, cu, S, C, T, reverse)  # static scratch
    torch.cuda.synchronize()
    print(f"[no-alloc] case {i} {name} C={C} T={T} rev={reverse}", flush=True)
    if off:  # the look-back walk
      rtol, atol = (1e-5, 1e-5) if dtype == torch.float32 else (1e-2, 1e-2)
      torch.testing.assert_close(h, ref, rtol=2 * rtol, atol=2 * atol)
    else:
      assert torch.equal(h, ref), f"{name}: not bit-identical"
    rows = sorted({0, C // 2, C - 1})
    check_close(h[rows], oracle_fwd(g[rows], x[rows], lens, reverse), dtype,
                f"{name} h")

