"""Grid helpers: same integers as the reference (_grid.py:4-70)."""

import pytest

from associative_scan_triton import (
  get_grid,
  get_num_stages,
  get_static_grid,
  next_power_of_2,
)


@pytest.mark.parametrize(("n", "exp"), [
  (0, 0), (1, 1), (2, 2), (3, 4), (4, 4), (5, 8), (127, 128), (128, 128),
  (129, 256), (512, 512), (2**31 - 1, 2**31), (2**40 + 1, 2**41),
])
def test_next_power_of_2(n, exp):
  assert next_power_of_2(n) == exp


def test_get_grid_matches_reference_formula():
  # get_grid(len(cu), max_seqlen, chunk, C) = (len(cu)-1, pow2(ceil), C)
  assert get_grid(2, 128, 128, 4) == (1, 1, 4)
  assert get_grid(9, 4096, 128, 1536) == (8, 32, 1536)
  assert get_grid(9, 65536, 128, 1536) == (8, 512, 1536)
  assert get_grid(65, 8192, 128, 1024) == (64, 64, 1024)
  assert get_grid(3, 5, 4, 2) == (2, 2, 2)
  assert get_grid(2, 5, 2, 1) == (1, 4, 1)  # ceil(5/2)=3 -> 4
  assert get_grid(2, 1, 2, 1) == (1, 1, 1)


def test_get_grid_rejects_odd_chunk():
  with pytest.raises(AssertionError, match="chunk size must be divisible by 2"):
    get_grid(2, 16, 3, 1)


def test_get_num_stages_table():
  assert get_num_stages(1) == 1
  assert get_num_stages(1, "bwd") == 1
  assert [get_num_stages(n) for n in (2, 4, 5, 512)] == [1, 1, 3, 3]
  assert [get_num_stages(n, "bwd") for n in (2, 4, 5, 512)] == [2, 2, 3, 3]


def test_get_static_grid():
  assert get_static_grid(65536, 128, 1536) == (512, 1536)
  assert get_static_grid(100, 64, 3) == (2, 3)
