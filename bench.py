"""Kernel-level benchmark of the chunked linear-recurrence scan on one MI355X.

Default workload (the BASELINE metric's configuration, cfg5): causal scan,
fp32, B=8 sequences of T=65536 packed along time, C=1536 channels
(805,306,368 elements per tensor), chunk_size 128,
g = 0.99 + 0.01*U(0,1), x ~ N(0,1), dy ~ U(0,1) (dense, as the reference's
kernel bench uses rand_like, bench_kernels.py:296).  One "step" is one
forward launch plus one fused backward launch over the whole batch, with all
tensors resident in HBM (the reference's bench_kernels fwd+bwd subject,
bench_kernels.py:279-312).

Reported: whole-job algorithmic HBM throughput (GB/s) and ms per step;
per-kernel average durations from HIP events recorded on the launch stream;
the roofline of the dominant kernel (the backward, 20 B/element); the CPU
baseline (the fp64-accumulating sequential oracle on the host cores, on a
row sample of the same inputs); and a parity check of sampled rows against
the oracle, outside the timed region.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg5]

--config sweep runs the reference's kernel benchmark sweep over T instead
(see sweep()); --config accuracy its accuracy benchmark (see accuracy()).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "associative-scan-triton_amd"))
sys.path.insert(0, str(ROOT))

METRIC = ("fwd+bwd scan ms + achieved HBM GB/s (% peak), "
          "B=8 C=1536 T=64K fp32")
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E

# name -> (description, B, C, T, dtype, kind, gate range)
CONFIGS = {
  "cfg5": ("causal fwd+bwd, B=8 C=1536 T=65536, fp32, chunk 128, "
           "g~0.99+0.01U(0,1)", 8, 1536, 65536, "float32", "causal", (0.99, 1.0)),
  "cfg4": ("bidirectional fwd+bwd (both branches, one launch each way), "
           "B=8 C=1536 T=16384, fp32, g~U(0.9,1)", 8, 1536, 16384, "float32",
           "bidi", (0.9, 1.0)),
  "cfg2": ("causal forward only, B=8 C=1536 T=4096, fp32, g=sigmoid(N(0,1))",
           8, 1536, 4096, "float32", "fwd", None),
  "cfg3": ("varlen causal fwd+bwd, 64 seqs U[16,8192], C=1024, bf16 storage, "
           "fp32 accumulate, g~U(0.5,1)", 64, 1024, None, "bfloat16", "causal",
           (0.5, 1.0)),
  # not a BASELINE config: cfg5's shape with bf16 storage (fp32 accumulation)
  "bf16": ("causal fwd+bwd, B=8 C=1536 T=65536, bf16 storage, fp32 "
           "accumulate, g~0.99+0.01U(0,1)", 8, 1536, 65536, "bfloat16", "causal",
           (0.99, 1.0)),
  # not BASELINE configs: one long sequence in one channel (one item: the
  # few-item tree walk), cfg5's per-tensor size / 6
  "row": ("causal fwd+bwd, one sequence T=2^27 in one channel (few-item "
          "walk), fp32, g~0.99+0.01U(0,1)", 1, 1, 1 << 27, "float32",
          "causal", (0.99, 1.0)),
  "row_bf16": ("causal fwd+bwd, one sequence T=2^27 in one channel (few-item "
               "walk), bf16 storage, fp32 accumulate, g~0.99+0.01U(0,1)", 1, 1,
               1 << 27, "bfloat16", "causal", (0.99, 1.0)),
  # not a BASELINE config: the segment-aware shift of _shift_pad.py at cfg5's
  # tensor size (compiled semantics, pad at segment starts)
  "shift": ("shift_pad backward=True (compiled form), B=8 C=1536 T=65536, "
            "fp32", 8, 1536, 65536, "float32", "shift", None),
}


def log(*a):
  print(*a, file=sys.stderr, flush=True)


def parse():
  p = argparse.ArgumentParser()
  p.add_argument("--gpus", type=int, default=1)
  p.add_argument("--steps", type=int, default=20)
  p.add_argument("--warmup", type=int, default=5)
  p.add_argument("--config", default="cfg5",
                 choices=sorted(CONFIGS) + ["sweep", "accuracy"])
  p.add_argument("--no-cpu-baseline", action="store_true")
  p.add_argument("--no-check", action="store_true")
  p.add_argument("--no-api", action="store_true",
                 help="skip the API-level (autograd, out.sum()) timing")
  p.add_argument("--no-recompute", action="store_true",
                 help="skip the recompute-mode legs (kernel and API level)")
  p.add_argument("--profile-copy", action="store_true",
                 help="also launch one plain device copy of one tensor "
                      "(rocprof byte-counter calibration)")
  return p.parse_args()


def main():
  a = parse()
  if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
    print(json.dumps({"error": "this build measures one GPU only; the scan "
                      "shards over channels/sequences with no communication, "
                      "so one GPU's share at its real shape is the measured "
                      "unit; run with --gpus 1"}))
    sys.exit(2)
  if a.config == "sweep":
    return sweep(a)
  if a.config == "accuracy":
    return accuracy(a)

  import numpy as np
  import torch

  from associative_scan_triton import _ops

  dev = torch.device("cuda:0")
  desc, B, C, T, dts, kind, grange = CONFIGS[a.config]
  dtype = getattr(torch, dts)
  esize = torch.tensor([], dtype=dtype).element_size()

  # ---- inputs (seeded, on the device) ----
  gen = torch.Generator(device=dev).manual_seed(1155)
  if T is None:  # varlen
    lens = torch.randint(16, 8192 + 1, (B,),
                         generator=torch.Generator().manual_seed(1155))
    cu = torch.cat([torch.zeros(1, dtype=torch.int64), lens.cumsum(0)])
    Tt = int(cu[-1])
  else:
    cu = torch.arange(B + 1, dtype=torch.int64) * T
    Tt = B * T
  cu = cu.to(torch.int32).to(dev)
  N = C * Tt

  def gates():
    if grange is None:
      return torch.randn(C, Tt, device=dev, generator=gen).sigmoid_().to(dtype)
    lo, hi = grange
    return torch.rand(C, Tt, device=dev, generator=gen).mul_(hi - lo).add_(lo).to(dtype)

  def normal():
    return torch.randn(C, Tt, device=dev, generator=gen).to(dtype)

  nbr = 2 if kind == "bidi" else 1
  g = [gates() for _ in range(nbr)]
  x = [normal() for _ in range(nbr)]
  h = [torch.empty_like(x[0]) for _ in range(nbr)]
  with_bwd = kind not in ("fwd", "shift")
  if with_bwd:
    dy = [torch.rand(C, Tt, device=dev, generator=gen).to(dtype) for _ in range(nbr)]
    dx = [torch.empty_like(x[0]) for _ in range(nbr)]
    dg = [torch.empty_like(x[0]) for _ in range(nbr)]
  torch.cuda.synchronize()
  log(f"[bench] {a.config}: {desc}; N={N} elements/tensor, "
      f"{torch.cuda.get_device_name(0)}")

  def fwd():
    if kind == "shift":
      _ops.shift_pad(x[0], h[0], cu, 0.0, backward=True, wrap=False)
    elif kind == "bidi":
      _ops.scan_bidi_fwd(g[0], x[0], g[1], x[1], h[0], h[1], cu)
    else:
      _ops.scan_fwd(g[0], x[0], h[0], cu, reverse=False)

  def bwd():
    if kind == "bidi":
      _ops.scan_bidi_bwd(dy[0], dy[1], g[0], g[1], h[0], h[1], dx[0], dg[0],
                         dx[1], dg[1], cu)
    else:
      _ops.scan_bwd(dy[0], g[0], h[0], dx[0], dg[0], cu, causal=True)

  if a.profile_copy:
    tmp = torch.empty_like(x[0])
    tmp.copy_(x[0])
    torch.cuda.synchronize()
    del tmp

  for _ in range(a.warmup):
    fwd()
    if with_bwd:
      bwd()
  torch.cuda.synchronize()

  # ---- timed region: K steps back to back, one event pair around them on
  # the launch stream (an event between steps is a marker packet of a few
  # microseconds, 9% of a cfg2 step) ----
  stream = torch.cuda.current_stream(dev)
  e_start = torch.cuda.Event(enable_timing=True)
  e_end = torch.cuda.Event(enable_timing=True)
  torch.cuda.synchronize()
  t0 = time.perf_counter()
  e_start.record(stream)
  for _ in range(a.steps):
    fwd()
    if with_bwd:
      bwd()
  e_end.record(stream)
  torch.cuda.synchronize()
  wall = time.perf_counter() - t0
  step_ms = e_start.elapsed_time(e_end) / a.steps

  # ---- the same K steps again with events around each call: the per-call
  # durations of the forward and the backward (the roofline's kernel
  # time) ----
  ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)]
        for _ in range(a.steps)]
  torch.cuda.synchronize()
  for k in range(a.steps):
    ev[k][0].record(stream)
    fwd()
    ev[k][1].record(stream)
    if with_bwd:
      bwd()
    ev[k][2].record(stream)
  torch.cuda.synchronize()
  fwd_ms = [e[0].elapsed_time(e[1]) for e in ev]
  bwd_ms = [e[1].elapsed_time(e[2]) for e in ev] if with_bwd else [0.0]

  # ---- and once more, each step alone after a 1 GiB write that flushes
  # the caches (four times the 256 MB MALL), as the reference's do_bench
  # does; the median of these is reported beside the back-to-back mean ----
  flush = torch.empty(1 << 28, dtype=torch.int32, device=dev)
  fl = []
  for _ in range(a.steps):
    flush.fill_(0)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    fwd()
    if with_bwd:
      bwd()
    e1.record(stream)
    e1.synchronize()
    fl.append(e0.elapsed_time(e1))
  del flush
  flushed_ms = float(np.median(fl))
  log(f"[bench] timed {a.steps} steps in {wall:.3f} s wall, "
      f"{step_ms:.4f} ms per step; per call: fwd {np.mean(fwd_ms):.4f} ms, "
      f"bwd {np.mean(bwd_ms):.4f} ms")

  fwd_bytes = (2 if kind == "shift" else 3) * esize * N * nbr
  bwd_bytes = 5 * esize * N * nbr if with_bwd else 0
  step_bytes = fwd_bytes + bwd_bytes
  gbs = step_bytes / (step_ms * 1e-3) / 1e9
  f_ms, b_ms = float(np.mean(fwd_ms)), float(np.mean(bwd_ms))
  if with_bwd:
    dom, dom_ms, dom_bytes = "bwd", b_ms, bwd_bytes
  else:
    dom = "shift_pad" if kind == "shift" else "fwd"
    dom_ms, dom_bytes = f_ms, fwd_bytes
  achieved = dom_bytes / (dom_ms * 1e-3) / 1e9

  # ---- parity of sampled rows (outside the timed region) ----
  # |got - ref| <= tol * (|ref| + s) against the fp64 oracle on the same
  # inputs, s = RMS of the reference rows (the value scale; tol = 1e-5 for
  # fp32, 1e-2 for bf16); reported as the largest ratio of error to bound,
  # so <= 1 passes.
  check = None
  if not a.no_check:
    from oracle import oracle
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    rows = sorted({0, C // 2, C - 1})
    cu_np = cu.cpu().numpy().astype(np.int64)
    ratios = {}

    def ratio(got, ref):
      s = max(1.0, float(np.sqrt(np.mean(ref * ref))))
      return float(np.max(np.abs(got - ref) / (tol * s + tol * np.abs(ref))))

    for b in range(nbr):
      if kind == "shift":  # a copy: bit-exact against the oracle
        xs = x[0][rows].double().cpu().numpy()
        ref = oracle.shift_pad(xs, cu_np, 0.0, backward=True, wrap=False)
        ratios["out"] = 0.0 if np.array_equal(h[0][rows].double().cpu().numpy(), ref) else float("inf")
        break
      rev = b == 1
      gs = g[b][rows].double().cpu().numpy()
      xs = x[b][rows].double().cpu().numpy()
      href = oracle.scan_fwd(gs, xs, cu_np, rev)
      hg = h[b][rows].double().cpu().numpy()
      ratios[f"h{b}"] = ratio(hg, href)
      if with_bwd:
        dxr, dgr = oracle.scan_bwd(dy[b][rows].double().cpu().numpy(), gs, hg,
                                   cu_np, causal=not rev)
        ratios[f"dx{b}"] = ratio(dx[b][rows].double().cpu().numpy(), dxr)
        ratios[f"dg{b}"] = ratio(dg[b][rows].double().cpu().numpy(), dgr)
    check = {"rows": rows, "rtol": tol, "atol": f"{tol} x RMS(ref)",
             "max_err_over_bound": ratios,
             "pass": all(v <= 1.0 for v in ratios.values())}
    log(f"[bench] parity on rows {rows}: {check}")

  # ---- CPU baseline on a row sample of the same inputs ----
  cpu = cpu_ref = None
  if not a.no_cpu_baseline and with_bwd and kind == "causal" and dtype == torch.float32:
    from oracle import oracle
    threads = max(1, min(16, os.cpu_count() or 1))
    rows = max(1, C // 4)
    gs = g[0][:rows].cpu().numpy()
    xs = x[0][:rows].cpu().numpy()
    dys = dy[0][:rows].cpu().numpy()
    outs = tuple(np.empty_like(xs) for _ in range(3))
    cu_np = cu.cpu().numpy().astype(np.int64)
    oracle.fwd_bwd_f32io(gs, xs, dys, cu_np, rows, threads, out=outs)  # page-in
    # repeat the sample for about 10 s of CPU work
    reps, t1 = 0, time.perf_counter()
    while True:
      oracle.fwd_bwd_f32io(gs, xs, dys, cu_np, rows, threads, out=outs)
      reps += 1
      cpu_total = time.perf_counter() - t1
      if cpu_total >= 10.0 or reps >= 2000:
        break
    cpu_s = cpu_total / reps
    n_s = rows * Tt
    cpu = {"value": round(32 * n_s / cpu_s / 1e9, 3), "unit": "GB/s",
           "cores": threads, "threads": threads,
           "host_cpus": os.cpu_count(), "kind": "port",
           "sample": f"first {rows} of {C} channels, all {B} sequences "
                     f"({n_s} elements, fwd+bwd, fp32 storage, fp64 "
                     f"accumulation, OpenMP over (sequence, channel) rows), "
                     f"repeated {reps} times in {cpu_total:.1f} s; "
                     f"{cpu_s * 1e3:.1f} ms per repetition",
           "ms_per_step_equiv": round(cpu_s * 1e3 * N / n_s, 1)}
    log(f"[bench] cpu baseline: {cpu}")
    # the reference's own CPU method: its fp64 gold-label loop over time in
    # torch, vectorised over the channels, and the hand-derived reverse
    # recurrence for the backward (torch's intra-op threads)
    L = min(4096, int(cu[1]) - int(cu[0]))
    gs_t = g[0][:, :L].cpu()
    xs_t = x[0][:, :L].cpu()
    dys_t = dy[0][:, :L].cpu()
    oracle.torch_fwd_bwd_f64(gs_t, xs_t, dys_t, [0, L])  # warm-up
    reps, t1 = 0, time.perf_counter()
    while True:
      oracle.torch_fwd_bwd_f64(gs_t, xs_t, dys_t, [0, L])
      reps += 1
      tt = time.perf_counter() - t1
      if tt >= 10.0 or reps >= 1000:
        break
    ts = tt / reps
    n_t = C * L
    cpu_ref = {"value": round(32 * n_t / ts / 1e9, 3), "unit": "GB/s",
               "cores": torch.get_num_threads(),
               "threads": torch.get_num_threads(),
               "host_cpus": os.cpu_count(), "kind": "port",
               "method": "the reference's CPU scan (torch fp64 loop over time, "
                         "tests/test_scan_dtypes.py:26-38) and its reverse-"
                         "recurrence backward (test_scan_kernels.py:873-897)",
               "sample": f"all {C} channels x the first {L} steps of the "
                         f"first sequence ({n_t} elements, fwd+bwd), repeated "
                         f"{reps} times in {tt:.1f} s; {ts * 1e3:.1f} ms per "
                         "repetition",
               "ms_per_step_equiv": round(ts * 1e3 * N / n_t, 1)}
    log(f"[bench] cpu baseline (reference method): {cpu_ref}")

  # ---- API level: the public autograd function, loss = out.sum() ----
  # (the reference's API benchmark pattern; includes the autograd
  # bookkeeping, output allocation and, for the sum, the stride-0 gradient)
  api = None
  if with_bwd and not a.no_api:
    import associative_scan_triton as ast
    args = {"cu_seqlens": cu, "chunk_size": 128,
            "grid": ast.get_grid(B + 1, int((cu[1:] - cu[:-1]).max()), 128, C)}
    leaves = [t.detach().requires_grad_(True) for t in (g + x)]

    def api_step():
      for t in leaves:
        t.grad = None
      if kind == "bidi":
        yf, yb = ast.scan_bidirectional_branched(leaves[0], leaves[2],
                                                 leaves[1], leaves[3], args)
        (yf.sum() + yb.sum()).backward()
      else:
        ast.scan_causal(leaves[0], leaves[1], args).sum().backward()

    for _ in range(a.warmup):
      api_step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(a.steps):
      api_step()
    e1.record(stream)
    torch.cuda.synchronize()
    api_ms = e0.elapsed_time(e1) / a.steps
    api = {"ms_per_step": round(api_ms, 4),
           "what": ("scan_bidirectional_branched + (out_f.sum() + out_b.sum())"
                    ".backward()" if kind == "bidi" else
                    "scan_causal + out.sum().backward()"),
           "GBs_algorithmic": round(step_bytes / (api_ms * 1e-3) / 1e9, 2)}
    del leaves
    log(f"[bench] api level: {api}")

  # ---- recompute mode (causal configs): the backward reads (dy, g, x) and
  # per-chunk checkpoints instead of (dy, g, h).  Kernel level: forward +
  # checkpoints, then the recompute backward, K steps back to back; API
  # level: scan_causal(..., recompute_states=True).sum().backward() against
  # the default mode, with the memory each keeps between the forward and the
  # backward and the peak over the step (above what was allocated before) ----
  recompute = None
  if with_bwd and kind == "causal" and not a.no_recompute:
    import associative_scan_triton as ast
    in_kernel = _ops.recompute_in_kernel(g[0], x[0], cu)

    def fwd_rc():
      _ops.scan_fwd(g[0], x[0], h[0], cu, reverse=False)
      return _ops.scan_checkpoints(h[0], cu, reverse=False)

    ck = fwd_rc()

    def bwd_rc():
      _ops.scan_bwd_recompute(dy[0], g[0], x[0], ck if in_kernel else None,
                              dx[0], dg[0], cu, causal=True)

    for _ in range(a.warmup):
      fwd_rc()
      bwd_rc()
    torch.cuda.synchronize()
    evr = [[torch.cuda.Event(enable_timing=True) for _ in range(3)]
           for _ in range(a.steps)]
    for k in range(a.steps):
      evr[k][0].record(stream)
      fwd_rc()
      evr[k][1].record(stream)
      bwd_rc()
      evr[k][2].record(stream)
    torch.cuda.synchronize()
    rf = float(np.mean([e[0].elapsed_time(e[1]) for e in evr]))
    rb = float(np.mean([e[1].elapsed_time(e[2]) for e in evr]))
    args_rc = {"cu_seqlens": cu, "chunk_size": 128,
               "grid": ast.get_grid(B + 1, int((cu[1:] - cu[:-1]).max()), 128, C)}
    gl = g[0].detach().requires_grad_(True)
    xl = x[0].detach().requires_grad_(True)

    def api_mode(rc):
      def step():
        gl.grad = xl.grad = None
        loss = ast.scan_causal(gl, xl, args_rc, recompute_states=rc).sum()
        loss.backward()
      for _ in range(a.warmup):
        step()
      torch.cuda.synchronize()
      e0 = torch.cuda.Event(enable_timing=True)
      e1 = torch.cuda.Event(enable_timing=True)
      e0.record(stream)
      for _ in range(a.steps):
        step()
      e1.record(stream)
      torch.cuda.synchronize()
      ms = e0.elapsed_time(e1) / a.steps
      gl.grad = xl.grad = None
      torch.cuda.synchronize()
      base = torch.cuda.memory_allocated()
      torch.cuda.reset_peak_memory_stats()
      loss = ast.scan_causal(gl, xl, args_rc, recompute_states=rc).sum()
      torch.cuda.synchronize()
      held = torch.cuda.memory_allocated() - base
      loss.backward()
      torch.cuda.synchronize()
      peak = torch.cuda.max_memory_allocated() - base
      gl.grad = xl.grad = None
      del loss
      return {"ms_per_step": round(ms, 4),
              "held_between_fwd_and_bwd_bytes": int(held),
              "peak_above_inputs_bytes": int(peak)}

    recompute = {
      "what": "backward from (dy, g, x) + per-chunk checkpoints instead of "
              "(dy, g, h): scan_causal(..., recompute_states=True)",
      "backward": ("recompute kernels (chained walk)" if in_kernel else
                   "states recomputed by the forward scan into a temporary, "
                   "then the plain backward"),
      "kernel_fwd_ms": round(rf, 4), "kernel_bwd_ms": round(rb, 4),
      "kernel_fwd_bwd_ms": round(rf + rb, 4),
      "kernel_bwd_GBs": round(bwd_bytes / (rb * 1e-3) / 1e9, 2),
      "checkpoint_bytes": int(ck.numel() * 4),
      "api_default": api_mode(False), "api_recompute": api_mode(True)}
    if not a.no_check:
      from oracle import oracle
      rows = sorted({0, C // 2, C - 1})
      cu_np = cu.cpu().numpy().astype(np.int64)
      gs = g[0][rows].double().cpu().numpy()
      hs = h[0][rows].double().cpu().numpy()   # the stored states
      dxr, dgr = oracle.scan_bwd(dy[0][rows].double().cpu().numpy(), gs, hs,
                                 cu_np, causal=True)
      tol = 1e-5 if dtype == torch.float32 else 1e-2

      def ratio(got, ref):
        s_ = max(1.0, float(np.sqrt(np.mean(ref * ref))))
        return float(np.max(np.abs(got - ref) / (tol * s_ + tol * np.abs(ref))))

      recompute["check_max_err_over_bound"] = {
        "dx": ratio(dx[0][rows].double().cpu().numpy(), dxr),
        "dg": ratio(dg[0][rows].double().cpu().numpy(), dgr)}
    del gl, xl
    log(f"[bench] recompute mode: {recompute}")

  # HBM bytes per launch of the dominant kernel from a recorded rocprofv3
  # FETCH_SIZE / WRITE_SIZE profile of this configuration (counters cannot
  # be read from inside the run; the file names the kernel and its copy
  # calibration); null when no profile of this configuration is recorded
  traffic = traffic_src = None
  tf = ROOT / "profiles" / f"traffic_{a.config}.json"
  if tf.exists():
    import hashlib
    rec = json.loads(tf.read_text())
    traffic = rec.get(dom)
    if traffic is not None:
      traffic_src = {"file": f"profiles/{tf.name}",
                     "sha256": hashlib.sha256(tf.read_bytes()).hexdigest()[:16],
                     "kernel": rec.get("kernels", {}).get(dom),
                     "recorded": True}

  out = {
    "metric": METRIC,
    "value": round(gbs, 2),
    "unit": "GB/s",
    "n_gpus": 1,
    "steps": a.steps,
    "warmup": a.warmup,
    "ms_per_step": round(step_ms, 4),
    "ms_per_step_flushed_median": round(flushed_ms, 4),
    "higher_is_better": True,
    "scaling": "weak",
    "vs_baseline": None,
    "dtype": {"float32": "f32", "bfloat16": "bf16"}[dts],
    "data": "synthetic (seeded device RNG)",
    "config": {"workload": f"{a.config}: {desc}", "B": B, "C": C,
               "T": T, "elements_per_tensor": N, "chunk_size": 128},
    "pct_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
    "elements_per_s": round(N * nbr / (step_ms * 1e-3), 1),
    "fwd_ms": round(f_ms, 4),
    "bwd_ms": round(b_ms, 4),
    "fwd_gbs": round(fwd_bytes / (f_ms * 1e-3) / 1e9, 2),
    "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 2),
                 "peak": PEAK_HBM_GBS, "unit": "GB/s",
                 "frac": round(achieved / PEAK_HBM_GBS, 4),
                 "traffic": traffic,
                 "traffic_source": traffic_src,
                 "algorithmic_bytes": dom_bytes},
    "cpu_baseline": cpu,
    "cpu_baseline_reference_method": cpu_ref,
    "api": api,
    "recompute": recompute,
    "check": check,
  }
  if a.config == "cfg5":
    # the reference's published kernel-level time for this shape (H100 80GB,
    # chunk 512, U(0,1) inputs; README.md:142-187); its GB/s are not
    # published, so vs_baseline stays null
    out["reference_published"] = {
      "hardware": "H100 80GB", "fwd_bwd_ms": H100_SWEEP[T][0],
      "speedup": round(H100_SWEEP[T][0] / step_ms, 3)}
  print(json.dumps(out), flush=True)


# The reference's published kernel-level sweep (H100 80GB, README.md:142-187):
# T -> (fwd+bwd, fwd, bwd) ms at B=8, C=1536, fp32, gates and tokens ~ U(0,1).
H100_SWEEP = {
  128: (0.027, 0.014, 0.020), 256: (0.043, 0.020, 0.029),
  512: (0.077, 0.033, 0.049), 1024: (0.161, 0.068, 0.099),
  2048: (0.306, 0.126, 0.186), 4096: (0.602, 0.240, 0.366),
  8192: (1.186, 0.455, 0.722), 16384: (2.322, 0.926, 1.429),
  32768: (4.602, 1.811, 2.821), 65536: (9.212, 3.606, 5.623),
}
# and its API-level fwd+bwd (H100 80GB, README.md:97-108): T -> ms for
# bench_vs_warpscan.py:214-220's subject (clone both inputs, scan_causal,
# out.sum().backward()).
H100_API = {128: 0.143, 256: 0.136, 512: 0.152, 1024: 0.300, 2048: 0.555,
            4096: 1.069, 8192: 2.070, 16384: 4.087, 32768: 8.126,
            65536: 16.238}


def sweep(a):
  """The reference's kernel benchmark sweep (bench/bench_kernels.py:279-312):
  for each T, B=8 sequences of T packed along time, C=1536, fp32, gates and
  tokens ~ U(0,1), dy = rand_like; the subjects forward, backward and
  forward + backward are timed separately.  As the reference's
  triton.testing.do_bench does, caches are flushed before every repetition
  (here a 1 GiB write, four times the 256 MB MALL) and only the subject sits
  between the two events; the median of the repetitions is reported.  The
  API leg times the reference's API subject (bench_vs_warpscan.py:214-220):
  clone gates and tokens with requires_grad, scan_causal, out.sum() and
  backward, chunk_size min(next_pow2(T), 512)."""
  import numpy as np
  import torch

  import associative_scan_triton as ast
  from associative_scan_triton import _ops

  dev = torch.device("cuda:0")
  stream = torch.cuda.current_stream(dev)
  B, C = 8, 1536
  flush = torch.empty(1 << 28, dtype=torch.int32, device=dev)
  reps = max(5, a.steps)
  rows = []
  for T in sorted(H100_SWEEP):
    Tt = B * T
    N = C * Tt
    gen = torch.Generator(device=dev).manual_seed(1155)
    cu = (torch.arange(B + 1, dtype=torch.int32) * T).to(dev)
    g = torch.rand(C, Tt, device=dev, generator=gen)
    x = torch.rand(C, Tt, device=dev, generator=gen)
    dy = torch.rand(C, Tt, device=dev, generator=gen)
    h, dx, dg = (torch.empty_like(x) for _ in range(3))

    def fwd():
      _ops.scan_fwd(g, x, h, cu, reverse=False)

    def bwd():
      _ops.scan_bwd(dy, g, h, dx, dg, cu, causal=True)

    def both():
      fwd()
      bwd()

    chunk = min(ast.next_power_of_2(T), 512)
    args = {"cu_seqlens": cu, "chunk_size": chunk,
            "grid": ast.get_grid(B + 1, T, chunk, C)}

    def api():
      gc = g.clone().requires_grad_(True)
      xc = x.clone().requires_grad_(True)
      ast.scan_causal(gc, xc, args).sum().backward()

    res = {}
    for name, fn in (("fwd", fwd), ("bwd", bwd), ("fwd+bwd", both),
                     ("api", api)):
      for _ in range(a.warmup):
        fn()
      ts = []
      for _ in range(reps):
        flush.fill_(0)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn()
        e1.record(stream)
        e1.synchronize()
        ts.append(e0.elapsed_time(e1))
      res[name] = float(np.median(ts))
    ref = H100_SWEEP[T]
    nbytes = 32 * N
    row = {"T": T, "elements_per_tensor": N,
           "fwd_ms": round(res["fwd"], 4), "bwd_ms": round(res["bwd"], 4),
           "fwd_bwd_ms": round(res["fwd+bwd"], 4),
           "fwd_bwd_GBs": round(nbytes / (res["fwd+bwd"] * 1e-3) / 1e9, 1),
           "pct_peak": round(100 * nbytes / (res["fwd+bwd"] * 1e-3) / 1e9
                             / PEAK_HBM_GBS, 1),
           "h100_fwd_bwd_ms": ref[0],
           "speedup_vs_h100": round(ref[0] / res["fwd+bwd"], 2),
           "api_fwd_bwd_ms": round(res["api"], 4),
           "h100_api_ms": H100_API[T],
           "api_speedup_vs_h100": round(H100_API[T] / res["api"], 2)}
    rows.append(row)
    log(f"[sweep] {row}")
    del g, x, dy, h, dx, dg
    torch.cuda.empty_cache()
  out = {"metric": "kernel-level fwd / bwd / fwd+bwd and API-level fwd+bwd "
                   "ms per T (median, caches flushed), B=8 C=1536 fp32",
         "unit": "ms", "n_gpus": 1, "higher_is_better": False,
         "dtype": "f32", "data": "synthetic (seeded device RNG, U(0,1))",
         "config": {"workload": "sweep: the reference's kernel benchmark "
                                "sweep over T, B=8 C=1536 fp32"},
         "reps": reps, "warmup": a.warmup, "rows": rows}
  print(json.dumps(out), flush=True)


# The reference's published forward RMSE against the sequential fp64 gold
# (H100, C=4, seed 42; README.md:266-281).
PUBLISHED_RMSE = {
  "fp32": {128: 6.55e-08, 512: 6.46e-08, 2048: 6.62e-08, 8192: 6.69e-08},
  "fp16": {128: 4.51e-04, 512: 4.89e-04, 2048: 2.58e-04, 8192: 2.58e-04},
  "bf16": {128: 3.59e-03, 512: 3.68e-03, 2048: 2.07e-03, 8192: 2.06e-03},
}


def accuracy(a):
  """The reference's accuracy benchmark (bench/bench_accuracy.py:31-37,
  76-95, 129-160): C=4 channels, one sequence of T in 128 ... 8192, for
  fp32 / fp16 / bf16 storage; torch.manual_seed(42) before each case, gates
  ~ U(0,1) and tokens ~ N(0,1) drawn on the device in fp32 and cast; the
  forward output against the sequential fp64 scan of the cast inputs:
  max abs error, max relative error where |gold| > eps(dtype), mean abs
  error and RMSE, beside the reference's published RMSE where it has one.
  The fused backward's RMSE (dy ~ N(0,1), against the fp64 adjoint of the
  same stored states) is reported too; the reference publishes none.  The
  fp64 sequential scans are the test oracle, used here as the checker."""
  import numpy as np
  import torch

  import associative_scan_triton as ast
  from associative_scan_triton import _ops
  from oracle import oracle

  dev = torch.device("cuda:0")
  C = 4
  rows = []
  for T in (128, 256, 512, 1024, 2048, 4096, 8192):
    for dt, name in ((torch.float32, "fp32"), (torch.float16, "fp16"),
                     (torch.bfloat16, "bf16")):
      torch.manual_seed(42)
      g32 = torch.rand(C, T, device=dev)
      x32 = torch.randn(C, T, device=dev)
      g, x = g32.to(dt).contiguous(), x32.to(dt).contiguous()
      cu = torch.tensor([0, T], device=dev, dtype=torch.int32)
      cs = min(ast.next_power_of_2(T), 512)
      out = torch.empty_like(x)
      ast.forward_scan_full(g, x, cu, ast.get_grid(2, T, cs, C),
                            REVERSE=False, CHUNK_SIZE=cs, TESTING=False,
                            tokens_out=out)
      dy = torch.randn(C, T, device=dev).to(dt)
      dx, dg = torch.empty_like(x), torch.empty_like(x)
      _ops.scan_bwd(dy, g, out, dx, dg, cu, causal=True)
      torch.cuda.synchronize()
      f64 = lambda t: t.detach().cpu().double().numpy()
      cu_np = np.array([0, T], dtype=np.int64)
      gold = oracle.scan_fwd(f64(g), f64(x), cu_np, False)
      diff = np.abs(f64(out) - gold)
      eps = float(torch.finfo(dt).eps)
      safe = np.abs(gold) > eps
      dx_ref, dg_ref = oracle.scan_bwd(f64(dy), f64(g), f64(out), cu_np, True)
      pub = PUBLISHED_RMSE[name].get(T)
      rmse = float(np.sqrt(np.mean(diff ** 2)))
      row = {"T": T, "dtype": name,
             "max_abs_err": float(diff.max()),
             "max_rel_err": float((diff[safe] / np.abs(gold[safe])).max())
             if safe.any() else 0.0,
             "mean_abs_err": float(diff.mean()), "rmse": rmse,
             "published_rmse": pub,
             "rmse_over_published": round(rmse / pub, 3) if pub else None,
             "bwd_rmse_dx": float(np.sqrt(np.mean((f64(dx) - dx_ref) ** 2))),
             "bwd_rmse_dg": float(np.sqrt(np.mean((f64(dg) - dg_ref) ** 2))),
             "finite": bool(torch.isfinite(out).all())}
      rows.append(row)
      log(f"[accuracy] {row}")
  out = {"metric": "forward RMSE vs sequential fp64 gold, C=4, seed 42 "
                   "(the reference's accuracy benchmark)",
         "unit": "rmse", "n_gpus": 1, "higher_is_better": False,
         "data": "synthetic (torch.manual_seed(42), device RNG)",
         "config": {"workload": "accuracy: C=4, one sequence of T, "
                                "fp32/fp16/bf16 storage, fp32 accumulation"},
         "rows": rows}
  print(json.dumps(out), flush=True)


if __name__ == "__main__":
  main()
