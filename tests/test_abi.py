"""C ABI surface of the built library (CPU only: no kernel is launched).

The library must load, report its ABI version, and export every entry point
that include/assocscan.h declares.  Argument validation happens on the host
before any HIP call, so invalid calls can be exercised without a GPU.
"""

import ctypes
import re
from pathlib import Path

import pytest

from associative_scan_triton import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "assocscan.h"


def _declared():
  text = HEADER.read_text()
  text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
  return sorted(set(re.findall(r"\b(asc_[a-z0-9_]+)\s*\(", text)))


def test_library_is_built():
  assert _lib.LIB_PATH.exists(), "run __graft_entry__.build() first"


def test_exports_every_declared_symbol():
  lib = ctypes.CDLL(str(_lib.LIB_PATH))
  names = _declared()
  assert names, "no declarations parsed"
  missing = [n for n in names if not hasattr(lib, n)]
  assert not missing, f"declared but not exported: {missing}"
  # and the ctypes binding covers exactly the declared set
  assert sorted(_lib.SIGNATURES) == names


def test_abi_version_and_strerror():
  lib = _lib.load()
  assert lib.asc_abi_version() == 6
  assert lib.asc_strerror(0) == b"success"
  for code in (-1, -2, -3, -4, -5, -6):
    assert lib.asc_strerror(code) and lib.asc_strerror(code) != b"unknown error"
  assert lib.asc_strerror(-99) == b"unknown error"


def _fwd(lib, **kw):
  a = dict(gates=8, tokens=8, h_out=8, gate_prod_out=None, cu=8, cu_dtype=0,
           S=1, C=1, T=4, dtype=0, reverse=0, ws=None, ws_bytes=0, stream=None)
  a.update(kw)
  return lib.asc_scan_fwd(*a.values())


def test_host_validation_codes():
  lib = _lib.load()
  assert _fwd(lib, gates=None) == -1
  assert _fwd(lib, cu=None) == -1
  assert _fwd(lib, dtype=7) == -2
  assert _fwd(lib, cu_dtype=3) == -2
  assert _fwd(lib, S=-1) == -3
  assert _fwd(lib, C=-2) == -3
  assert _fwd(lib, tokens=6) == -4          # fp32 pointer not 4-byte aligned
  assert _fwd(lib, cu=10, cu_dtype=1) == -4  # int64 cu not 8-byte aligned
  # empty problems are a successful no-op (nothing is launched)
  assert _fwd(lib, S=0) == 0
  assert _fwd(lib, C=0) == 0
  assert lib.asc_scan_bwd(8, 8, 8, 8, None, 8, 0, 1, 1, 4, 0, 1, None, 0,
                          None) == -1
  assert lib.asc_shift_pad(8, 8, 8, 0, 1, 1, 4, 5, 0.0, 1, 1, None) == -2


def test_workspace_bytes():
  lib = _lib.load()
  # few (segment, channel) items: the larger of the tree walk's need (a
  # 256-byte flag block, then per branch one 16-byte slot per chunk of
  # 8192 fp32 / 16384 fp16-bf16 elements and one per group of 64 slots of
  # the level below, up to a level of at most 64) and the look-back walk's
  # (one slot per tile of 16384 elements); both for the worst-case phase
  def tree(n, chunk, nbranch):
    cnt, slots = -(-n // chunk), 0
    while True:
      slots += cnt
      if cnt <= 64:
        break
      cnt = -(-cnt // 64)
    return 256 + 16 * slots * nbranch

  n = 4 * 1_000_000
  b1 = lib.asc_scan_workspace_bytes(2, 4, 1_000_000, 0, 1)
  b2 = lib.asc_scan_workspace_bytes(2, 4, 1_000_000, 0, 2)
  assert b1 == max(tree(n + 3, 8192, 1), 16 * -(-(n + 3) // 16384))
  assert b2 == max(tree(n + 3, 8192, 2), 2 * 16 * -(-(n + 3) // 16384))
  assert lib.asc_scan_workspace_bytes(2, 4, 1_000_000, 2, 1) == max(
    tree(n + 7, 16384, 1), 16 * -(-(n + 7) // 16384))
  # one row of 2^27 elements: 16385 chunks, 257 groups, 5 groups of groups
  assert lib.asc_scan_workspace_bytes(1, 1, 1 << 27, 0, 1) == tree((1 << 27) + 3, 8192, 1)
  # many items (more than 128 (segment, channel, branch) items): rows that
  # are a whole number of chunks (4096 fp32 / 8192 fp16-bf16 elements) with
  # segments of at least one chunk on average take the chained walk, a
  # 256-byte flag plus one 16-byte slot per chunk and branch; other
  # geometries run the workspace-free walks and need none
  assert lib.asc_scan_workspace_bytes(8, 1536, 524288, 0, 1) == 256 + 16 * 1536 * 128
  assert lib.asc_scan_workspace_bytes(8, 1536, 131072, 0, 2) == 256 + 16 * 2 * 1536 * 32
  assert lib.asc_scan_workspace_bytes(1, 1536, 524288, 0, 1) == 0     # 128 chunks
  assert lib.asc_scan_workspace_bytes(8, 1536, 524288, 2, 1) == 256 + 16 * 1536 * 64
  assert lib.asc_scan_workspace_bytes(8, 1536, 524289, 0, 1) == 0     # ragged rows
  assert lib.asc_scan_workspace_bytes(256, 1536, 524288, 0, 1) == 0   # mean 2048
  assert lib.asc_scan_workspace_bytes(1, 128, 4000, 0, 1) > 0
  assert lib.asc_scan_workspace_bytes(1, 129, 4000, 0, 1) == 0
  assert lib.asc_scan_workspace_bytes(1, 64, 4000, 0, 2) > 0
  assert lib.asc_scan_workspace_bytes(1, 65, 4000, 0, 2) == 0
  assert lib.asc_scan_workspace_bytes(2, 64, 4096, 2, 1) > 0
  assert lib.asc_scan_workspace_bytes(2, 65, 4096, 1, 1) == 0
  # empty problems need nothing; invalid arguments are errors
  assert lib.asc_scan_workspace_bytes(0, 4, 128, 0, 1) == 0
  assert lib.asc_scan_workspace_bytes(1, 4, 128, 9, 1) < 0
  assert lib.asc_scan_workspace_bytes(1, 4, 128, 0, 3) < 0
  assert lib.asc_scan_workspace_bytes(-1, 4, 128, 0, 1) < 0
  walk = lib.asc_scan_workspace_walk
  assert walk(8, 1536, 524288, 0, 1) == _lib.WALK_CHAINED
  assert walk(2, 4, 1_000_000, 0, 1) == _lib.WALK_LOOKBACK
  assert walk(8, 1536, 524289, 0, 1) == 0
  assert walk(8, 1536, 524288, 9, 1) < 0
  prev = lib.asc_set_lookback_spin_limit(7)
  assert lib.asc_set_lookback_spin_limit(prev) == 7


def test_error_is_raised_with_message():
  with pytest.raises(_lib.AscError, match="NULL"):
    _lib.check(-1)


def test_rowgrad_validation_codes():
  lib = _lib.load()
  args = dict(grad=8, rs=0, gates=64, states=128, dx=192, dg=256, cu=8,
              cu_dtype=0, S=1, C=1, T=4, dtype=0, causal=1, ws=None,
              ws_bytes=0, stream=None)

  def call(**kw):
    a = dict(args)
    a.update(kw)
    return lib.asc_scan_bwd_rowgrad(*a.values())

  assert call(grad=None) == -1
  assert call(dg=None) == -1
  assert call(rs=-1) == -5
  assert call(dtype=5) == -2
  assert call(grad=6) == -4       # fp32 gradient not 4-byte aligned
  assert call(S=0) == 0           # empty: nothing launched


def test_bidi_rowgrad_validation_codes():
  lib = _lib.load()
  # row gradients, then gates, states and the four outputs 64 bytes apart
  # (fp32, C=1, T=4: 16 bytes per tensor), then cu_seqlens
  base = ([8, 0, 8, 0] + [64 * (i + 1) for i in range(8)] + [8]
          + [0, 1, 1, 4, 0, None, 0, None])

  def call(i=None, v=None):
    a = list(base)
    if i is not None:
      a[i] = v
    return lib.asc_scan_bidi_bwd_rowgrad(*a)

  assert call(0, None) == -1      # forward-branch gradient
  assert call(2, None) == -1      # reverse-branch gradient
  assert call(12, None) == -1     # cu_seqlens
  assert call(1, -1) == -5        # negative row stride
  assert call(3, -2) == -5
  assert call(17, 9) == -2        # dtype
  assert call(2, 6) == -4         # fp32 gradient not 4-byte aligned
  assert call(14, 0) == 0         # num_seq = 0: nothing launched


def test_aliasing_rule_codes():
  """An output may replace only its own input (h the tokens, the gate
  product the gates, d_tokens the dense gradient); any other overlap is
  ASC_E_ARG.  fp32, C=1, T=4: 16 bytes per tensor; S=0, so an accepted
  call launches nothing."""
  lib = _lib.load()
  ok = dict(S=0, gates=64, tokens=128, h_out=192)
  assert _fwd(lib, **ok) == 0
  assert _fwd(lib, **{**ok, "h_out": 128}) == 0          # h replaces tokens
  assert _fwd(lib, **{**ok, "h_out": 64}) == -5          # h over the gates
  assert _fwd(lib, **{**ok, "h_out": 136}) == -5         # partial overlap
  assert _fwd(lib, **{**ok, "gate_prod_out": 64}) == 0   # TESTING in place
  assert _fwd(lib, **{**ok, "h_out": 128, "gate_prod_out": 64}) == 0
  assert _fwd(lib, **{**ok, "gate_prod_out": 192}) == -5  # both outputs
  assert _fwd(lib, **{**ok, "gate_prod_out": 128}) == -5  # A over tokens
  assert _fwd(lib, **{**ok, "h_out": 60}) == -5          # ends inside gates
  assert _fwd(lib, **{**ok, "h_out": 48}) == 0           # ends where gates begin

  def bwd(grad=64, gates=128, states=192, dx=256, dg=320):
    return lib.asc_scan_bwd(grad, gates, states, dx, dg, 8, 0, 0, 1, 4, 0, 1,
                            None, 0, None)

  assert bwd() == 0
  assert bwd(dx=64) == 0          # d_tokens replaces the gradient
  assert bwd(dg=64) == -5         # d_gates over the gradient
  assert bwd(dx=128) == -5        # over the gates
  assert bwd(dg=192) == -5        # over the states
  assert bwd(dx=320) == -5        # the two outputs
  assert bwd(dx=200) == -5        # partial overlap with the states
  # bidirectional: an output of one branch over an input of the other
  base = [64 * (i + 1) for i in range(6)] + [8, 0, 0, 1, 4, 0, None, 0, None]
  assert lib.asc_scan_bidi_fwd(*base) == 0
  bad = list(base)
  bad[4] = bad[3]                 # h_fwd over tokens_bwd
  assert lib.asc_scan_bidi_fwd(*bad) == -5
  inplace = list(base)
  inplace[4], inplace[5] = inplace[1], inplace[3]   # each branch in place
  assert lib.asc_scan_bidi_fwd(*inplace) == 0


def test_noalloc_forward_limits():
  """asc_scan_fwd_noalloc validates on the host before any HIP call: a
  geometry whose workspace would exceed its 8 MiB static buffer is
  ASC_E_SCRATCH, an empty problem is a successful no-op."""
  lib = _lib.load()
  # 4096 rows of 256 chunk-aligned 4096-element chunks: 16 MiB of slots
  assert lib.asc_scan_workspace_bytes(8, 4096, 1 << 20, 0, 1) > 8 << 20
  assert lib.asc_scan_fwd_noalloc(64, 128, 192, None, 8, 0, 8, 4096, 1 << 20,
                                  0, 0, None) == -6
  assert b"8 MiB" in lib.asc_strerror(-6)
  assert lib.asc_scan_fwd_noalloc(64, 128, 192, None, 8, 0, 0, 1, 4, 0, 0,
                                  None) == 0
  assert lib.asc_scan_fwd_noalloc(64, 128, 64, None, 8, 0, 0, 1, 4, 0, 0,
                                  None) == -5


def test_recompute_entry_points_validation():
  """Checkpoint counts and the recompute backward's host-side checks: whole
  16-byte vectors (aligned tensors, rows a multiple of the vector width),
  the aliasing rule (the checkpoints are an input); S = 0 launches nothing."""
  lib = _lib.load()
  ce = lib.asc_scan_checkpoint_elems
  assert ce(1536, 524288, 0) == 1536 * 128          # 4096 fp32 per chunk
  assert ce(1536, 524288, 2) == 1536 * 64           # 8192 bf16 per chunk
  assert ce(3, 4097, 0) == 3 * 2 and ce(3, 4096, 0) == 3 and ce(3, 0, 0) == 0
  assert ce(3, 10, 9) < 0 and ce(-1, 10, 0) < 0

  def rc(grad=64, rs=-1, gates=128, tokens=192, ckpt=256, dx=320, dg=384,
         S=0, C=1, T=4, dtype=0):
    return lib.asc_scan_bwd_recompute(grad, rs, gates, tokens, ckpt, dx, dg,
                                      8, 0, S, C, T, dtype, 1, None, 0, None)

  assert rc() == 0
  assert rc(dx=64) == 0               # d_tokens over the dense gradient
  assert rc(dx=256) == -5             # over the checkpoints
  assert rc(dg=192) == -5             # over the tokens
  assert rc(rs=0, grad=68, dx=64) == -5   # the row gradient is not replaced
  assert rc(tokens=200) == -4         # not 16-byte aligned
  assert rc(grad=72) == -4            # a dense gradient must be aligned too
  assert rc(grad=72, rs=0) == 0       # one value per row need not be
  assert rc(T=6) == -4                # rows not a whole number of vectors
  assert rc(T=8, dtype=2) == 0 and rc(T=12, dtype=2) == -4
  assert rc(ckpt=258) == -4
  assert rc(gates=None) == -1 and rc(ckpt=None) == -1
  # C = 0: no checkpoints, nothing launched (with rows, S = 0 still writes
  # zero checkpoints)
  assert lib.asc_scan_checkpoints(64, 128, 8, 0, 0, 0, 4, 0, 0, None) == 0
  assert lib.asc_scan_checkpoints(64, 66, 8, 0, 0, 1, 4, 0, 0, None) == -4
  assert lib.asc_scan_checkpoints(64, 72, 8, 0, 0, 1, 4, 0, 0, None) == -5
  assert lib.asc_scan_checkpoints(None, 128, 8, 0, 0, 1, 4, 0, 0, None) == -1


def test_shift_pad_strided_validation():
  """Strides are >= 0; out must not overlap itself or data (host checks,
  before any launch); C = 0 launches nothing."""
  lib = _lib.load()

  def sp(data=64, ds0=4, ds1=1, out=256, os0=4, os1=1, C=0, L=4):
    return lib.asc_shift_pad_strided(data, ds0, ds1, out, os0, os1, 8, 0, 1,
                                     C, L, 0, 0.0, 1, 1, None)

  assert sp() == 0
  assert sp(C=2, ds0=-1) == -5
  assert sp(C=2, os0=2) == -5            # rows of out overlap
  assert sp(C=2, os0=0) == -5
  assert sp(C=2, out=64) == -5           # in place
  assert sp(C=2, out=72) == -5           # overlapping data
  assert sp(C=2, data=None) == -1
