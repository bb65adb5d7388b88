"""Shared helpers for the GPU parity tests (inputs, oracle comparison)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import oracle

DEV = torch.device("cuda:0")

# |got - ref| <= atol * s + rtol * |ref| against the fp64 oracle run on the
# same (storage-rounded) inputs, where s = max(1, RMS(ref)) is the value scale
# of the compared block.  fp32: the north-star bar rtol 1e-5; fp16/bf16: one
# rounding of the output dominates (2^-11 and 2^-8 relative).  The atol is
# tied to the value scale because near a zero crossing of h the absolute
# error of any fp32 evaluation, sequential included, is set by the size of h
# around it, not by h itself (see test_long_memory_error_vs_sequential_fp32).
TOL = {
  torch.float32: (1e-5, 1e-5),
  torch.float16: (2e-3, 2e-3),
  torch.bfloat16: (1e-2, 1e-2),
}


def cu_of(lens) -> np.ndarray:
  return np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)


def make(lens, C, dtype=torch.float32, seed=1155, glo=0.0, ghi=1.0, n=2):
  """n seeded [C, T] tensors on the CPU: gates ~ U(glo, ghi), then N(0,1)."""
  gen = torch.Generator().manual_seed(seed)
  T = int(sum(lens))
  out = [(glo + (ghi - glo) * torch.rand(C, T, generator=gen)).to(dtype)]
  for _ in range(n - 1):
    out.append(torch.randn(C, T, generator=gen).to(dtype))
  return out


def npf(t: torch.Tensor) -> np.ndarray:
  return t.detach().cpu().to(torch.float64).numpy()


def value_scale(ref: np.ndarray) -> float:
  return max(1.0, float(np.sqrt(np.mean(np.square(ref))))) if ref.size else 1.0


def check_close(got: torch.Tensor, ref: np.ndarray, dtype, what: str,
                scale: float | None = None) -> float:
  """Asserts elementwise closeness; returns the max error / bound."""
  rtol, atol = TOL[dtype]
  g = npf(got)
  assert g.shape == ref.shape, (what, g.shape, ref.shape)
  if scale is None:
    scale = value_scale(ref)
  err = np.abs(g - ref)
  bound = atol * scale + rtol * np.abs(ref)
  bad = ~(err <= bound)
  if bad.any():
    i = np.unravel_index(np.argmax(np.where(bad, err / bound, 0)), err.shape)
    raise AssertionError(
      f"{what}: {bad.sum()} of {err.size} elements out of tolerance "
      f"(rtol={rtol}, atol={atol * scale}); worst at {i}: got {g[i]!r}, "
      f"ref {ref[i]!r}")
  return float((err / bound).max()) if err.size else 0.0


def grid_args(lens, C, chunk=128, cu_dtype=torch.int32):
  import associative_scan_triton as ast
  cu = torch.tensor(cu_of(lens), dtype=cu_dtype, device=DEV)
  grid = ast.get_grid(len(lens) + 1, max(max(lens), 1), chunk, C)
  return {"cu_seqlens": cu, "chunk_size": chunk, "grid": grid}


def oracle_fwd(g, x, lens, reverse=False):
  return oracle.scan_fwd(npf(g), npf(x), cu_of(lens), reverse)


def oracle_bwd(dy, g, h_ref, lens, causal=True):
  """Backward from the oracle's own fp64 states."""
  return oracle.scan_bwd(npf(dy), npf(g), h_ref, cu_of(lens), causal)
