"""Build recipe for libassocscan.so (gfx950), kept beside the package.

The shared library is built in-tree (next to this file) so it travels with
the source tree; nothing is installed into site-packages.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC_DIR = PKG_DIR.parent / "csrc"
REPO_ROOT = PKG_DIR.parent.parent
INCLUDE_DIR = REPO_ROOT / "include"
LIB_NAME = "libassocscan.so"
LIB_PATH = PKG_DIR / LIB_NAME

ARCH = os.environ.get("ASC_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
# Symbols are hidden unless marked: only the extern "C" entry points (between
# visibility pragmas in the sources) are exported.
HIPCC_FLAGS = [
  "-O3",
  "-std=c++17",
  "-fPIC",
  "-fvisibility=hidden",
  f"--offload-arch={ARCH}",
  "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
  "-Wall",
]


def hipcc() -> str:
  path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
  if not Path(path).exists():
    raise RuntimeError("hipcc not found; cannot build libassocscan")
  return path


def _run(cmd: list[str], verbose: bool) -> None:
  if verbose:
    print(" ".join(cmd), flush=True)
  res = subprocess.run(cmd, capture_output=True, text=True)
  if res.returncode != 0:
    raise RuntimeError(
      f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
  if verbose and (res.stdout or res.stderr):
    print(res.stdout, res.stderr, flush=True)


def build(verbose: bool = False, extra_flags: list[str] | None = None,
          out: Path | None = None, jobs: int | None = None) -> Path:
  """Compiles each csrc/*.hip to an object (in parallel), links them into one
  shared library and returns its path."""
  out = Path(out) if out is not None else LIB_PATH
  sources = sorted(CSRC_DIR.glob("*.hip"))
  if not sources:
    raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
  flags = [*HIPCC_FLAGS, *(extra_flags or []), f"-I{INCLUDE_DIR}",
           f"-I{CSRC_DIR}"]
  jobs = jobs or min(len(sources), int(os.environ.get("MAX_JOBS", "0"))
                     or os.cpu_count() or 1)
  with tempfile.TemporaryDirectory(prefix="asc_build_") as tmpdir:
    objs = [Path(tmpdir) / (s.stem + ".o") for s in sources]
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
      futs = [pool.submit(_run, [hipcc(), *flags, "-c", str(s), "-o", str(o)],
                          verbose) for s, o in zip(sources, objs)]
      for f in futs:
        f.result()
    tmp = out.with_name(out.name + f".tmp{os.getpid()}")
    _run([hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}",
          *[str(o) for o in objs], "-o", str(tmp)], verbose)
  os.replace(tmp, out)
  return out


if __name__ == "__main__":
  print(build(verbose=True))
