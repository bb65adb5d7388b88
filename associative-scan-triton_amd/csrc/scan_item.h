// One wave per (segment, channel) item: device code and kernel templates,
// shared by the deep-pipeline (scan_item.hip) and shallow-pipeline
// (scan_item_short.hip) units.  The carry lives in a register and the
// item is walked sub-tile by sub-tile, interior sub-tiles software-
// pipelined (loads of the next U sub-tiles issued before the current ones
// are scanned).  The two depths are compiled in separate units: in one
// unit the shared helpers were register-allocated less tightly (bf16
// backward 100 instead of 96 VGPRs, one wave per SIMD fewer).

#ifndef ASC_SCAN_ITEM_H
#define ASC_SCAN_ITEM_H

#include "asc_common.h"

namespace asc {
namespace {

// Pipeline depths (sub-tiles per block): deep for long items
// (scan_item.hip), shallow for short ones (scan_item_short.hip).  Only the
// deep kernels (16-byte aligned tensors, no gate product) can run before
// the chained walk, which takes segments of a chunk or more.
constexpr int kFwdDeep = 4, kBwdDeep = 2, kFwdShallow = 2, kBwdShallow = 1;

// BATCH: the masked loads of a sub-tile go through load_vecs (all tensors'
// loads issued before any is masked): ragged fp32 segments of 16-600
// elements 65.5 / 99.1 -> 54.0 / 81.9 us fwd / bwd, bf16 segments of
// 300-1200 elements 96.1 / 162.1 -> 69.5 / 124.2, bf16 segments of 2047
// 48.3 / 85.8 -> 40.8 / 72.6 (C = 1024-1536, caches flushed).  Not in the
// deep fp16/bf16 backward: its 113-124 VGPRs leave no room (cfg3 backward
// 451 -> 464 us with it).
template <class IO, bool SHALLOW>
constexpr bool batch_masked_bwd() {
  return IO::V == 4 || SHALLOW;
}

template <class IO, bool REV, bool ALN, bool WA, bool MASKED, int NS>
__device__ inline void fwd_block(const FwdPtrs& t, const Walk<IO, REV>& w,
                                 int64_t k0, int lane, float& carry,
                                 float& carry_a) {
  constexpr int V = IO::V;
  float g[NS][V], x[NS][V];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int64_t vi = w.vec(k0 + u, lane);
    const bool ok = !MASKED || w.lane_valid(k0 + u, lane);
    if (ALN && MASKED) {
      const char* const src[2] = {t.g, t.x};
      const float ident[2] = {1.0f, 0.0f};
      float gx[2][V];
      load_vecs<IO, 2>(src, vi, ok, w.P0, w.P1, ident, gx, w.pend);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        g[u][e] = gx[0][e];
        x[u][e] = gx[1][e];
      }
    } else {
      load_vec<IO, ALN, MASKED, true>(t.g, vi, ok, w.P0, w.P1, 1.0f, g[u], w.pend);
      load_vec<IO, ALN, MASKED, true>(t.x, vi, ok, w.P0, w.P1, 0.0f, x[u], w.pend);
    }
  }
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int64_t vi = w.vec(k0 + u, lane);
    const bool ok = !MASKED || w.lane_valid(k0 + u, lane);
    float h[V], a[V];
    fwd_subtile<IO, REV, MASKED, WA>(g[u], x[u], vi * V, w.head(), carry,
                                     carry_a, h, a);
    store_vec<IO, ALN, MASKED>(t.h, vi, ok, w.P0, w.P1, h);
    if (WA) store_vec<IO, ALN, MASKED>(t.a, vi, ok, w.P0, w.P1, a);
  }
}

// Interior sub-tiles [k, kend) ((kend - k) a positive multiple of U), all
// full and aligned.  Software-pipelined: the loads of the next block of U
// sub-tiles are issued before the current block is scanned, so each wave
// keeps 2*U*16 bytes per lane and tensor in flight while it computes.
template <class IO, bool REV, bool WA, int U>
__device__ inline void fwd_fast(const FwdPtrs& t, const Walk<IO, REV>& w,
                                int64_t k, int64_t kend, int lane,
                                float& carry, float& carry_a) {
  constexpr int V = IO::V;
  constexpr int STEP = REV ? -kWave * 16 : kWave * 16;  // bytes per sub-tile
  const uint32_t lo = lane_off<REV>(lane);
  uint4 ga[U], xa[U], gb[U], xb[U];
  auto load = [&](uint4(&g)[U], uint4(&x)[U], int64_t kk) {
    const int64_t b = sub_lo(w, kk) * 16;
    const char* gp = t.g + b + lo;
    const char* xp = t.x + b + lo;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      g[u] = ld16(gp + u * STEP);
      x[u] = ld16(xp + u * STEP);
    }
  };
  auto run = [&](const uint4(&g)[U], const uint4(&x)[U], int64_t kk) {
    const int64_t b = sub_lo(w, kk) * 16;
    char* hp = t.h + b + lo;
    char* ap = WA ? t.a + b + lo : nullptr;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float gf[V], xf[V], hf[V], af[V];
      IO::unpack(g[u], gf);
      IO::unpack(x[u], xf);
      fwd_subtile<IO, REV, false, WA>(gf, xf, 0, 0, carry, carry_a, hf, af);
      st16(hp + u * STEP, IO::pack(hf));
      if (WA) st16(ap + u * STEP, IO::pack(af));
    }
  };
  load(ga, xa, k);
  while (true) {
    const bool more = k + U < kend;
    if (more) load(gb, xb, k + U);
    run(ga, xa, k);
    k += U;
    if (!more) break;
    const bool more2 = k + U < kend;
    if (more2) load(ga, xa, k + U);
    run(gb, xb, k);
    k += U;
    if (!more2) break;
  }
}

template <class IO, bool REV, bool ALN, bool WA, int U>
__device__ void fwd_item(const FwdPtrs& t, int64_t P0, int64_t P1, int lane) {
  const Walk<IO, REV> w(P0, P1, t.pend);
  float carry = 0.0f, carry_a = 1.0f;
  fwd_block<IO, REV, ALN, WA, true, 1>(t, w, 0, lane, carry, carry_a);
  int64_t k = 1;
  if (ALN) {
    const int64_t nfull = (w.kfast - 1) / U * U;
    if (nfull > 0) {
      fwd_fast<IO, REV, WA, U>(t, w, 1, 1 + nfull, lane, carry, carry_a);
      k = 1 + nfull;
    }
  } else {
    for (; k + U <= w.kfast; k += U)
      fwd_block<IO, REV, ALN, WA, false, U>(t, w, k, lane, carry, carry_a);
  }
  for (; k < w.kfast; ++k)
    fwd_block<IO, REV, ALN, WA, false, 1>(t, w, k, lane, carry, carry_a);
  for (; k < w.nsub; ++k)
    fwd_block<IO, REV, ALN, WA, true, 1>(t, w, k, lane, carry, carry_a);
}


// DYC: the gradient is the constant dyv along the item (dy is not read).
template <class IO, bool RB, bool ALN, bool MASKED, int NS, bool DYC,
          bool BATCH = true>
__device__ inline void bwd_block(const BwdPtrs& t, const Walk<IO, RB>& w,
                                 int64_t k0, int lane, float& carry,
                                 float& carry_g, float dyv) {
  constexpr int V = IO::V;
  float g[NS][V], dy[NS][V], h[NS][V];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int64_t vi = w.vec(k0 + u, lane);
    const bool ok = !MASKED || w.lane_valid(k0 + u, lane);
    if (ALN && MASKED && BATCH && !DYC) {
      const char* const src[3] = {t.dy, t.g, t.h};
      const float ident[3] = {0.0f, 1.0f, 0.0f};
      float ygh[3][V];
      load_vecs<IO, 3>(src, vi, ok, w.P0, w.P1, ident, ygh, w.pend);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        dy[u][e] = ygh[0][e];
        g[u][e] = ygh[1][e];
        h[u][e] = ygh[2][e];
      }
    } else if (ALN && MASKED && BATCH) {
      const char* const src[2] = {t.g, t.h};
      const float ident[2] = {1.0f, 0.0f};
      float gh[2][V];
      load_vecs<IO, 2>(src, vi, ok, w.P0, w.P1, ident, gh, w.pend);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        g[u][e] = gh[0][e];
        h[u][e] = gh[1][e];
      }
      dyc_vec<IO, MASKED>(dyv, vi, ok, w.P0, w.P1, dy[u]);
    } else {
      if (DYC)
        dyc_vec<IO, MASKED>(dyv, vi, ok, w.P0, w.P1, dy[u]);
      else
        load_vec<IO, ALN, MASKED, true>(t.dy, vi, ok, w.P0, w.P1, 0.0f, dy[u], w.pend);
      load_vec<IO, ALN, MASKED, true>(t.g, vi, ok, w.P0, w.P1, 1.0f, g[u], w.pend);
      load_vec<IO, ALN, MASKED, true>(t.h, vi, ok, w.P0, w.P1, 0.0f, h[u], w.pend);
    }
  }
  // state just past this block in B order (pad 0 outside the segment)
  float halo = 0.0f;
  if (k0 + NS < w.nsub) {
    const int64_t vlast = w.vec(k0 + NS - 1, kWave - 1);
    const int64_t pn = RB ? vlast * V - 1 : vlast * V + V;
    if (pn >= w.P0 && pn < w.P1) halo = IO::load1(t.h + pn * IO::ES);
  }
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int64_t vi = w.vec(k0 + u, lane);
    const bool ok = !MASKED || w.lane_valid(k0 + u, lane);
    const float hin =
        (u + 1 < NS) ? readlane(h[u + 1][mem_idx<V, RB>(0)], 0) : halo;
    float dx[V], dg[V];
    bwd_subtile<IO, RB, MASKED>(g[u], dy[u], h[u], vi * V, w.head(), w.tail(),
                                carry, carry_g, hin, dx, dg);
    store_vec<IO, ALN, MASKED>(t.dx, vi, ok, w.P0, w.P1, dx);
    store_vec<IO, ALN, MASKED>(t.dg, vi, ok, w.P0, w.P1, dg);
  }
}

// Interior sub-tiles of the backward, software-pipelined like fwd_fast.
template <class IO, bool RB, int U, bool DYC>
__device__ inline void bwd_fast(const BwdPtrs& t, const Walk<IO, RB>& w,
                                int64_t k, int64_t kend, int lane,
                                float& carry, float& carry_g, float dyv) {
  constexpr int V = IO::V;
  constexpr int STEP = RB ? -kWave * 16 : kWave * 16;
  const uint32_t lo = lane_off<RB>(lane);
  uint4 ya[U], ga[U], ha[U], yb[U], gb[U], hb[U];
  float halo_a, halo_b;
  auto load = [&](uint4(&y)[U], uint4(&g)[U], uint4(&h)[U], float& halo,
                  int64_t kk) {
    const int64_t b = sub_lo(w, kk) * 16;
    const char* yp = t.dy + b + lo;
    const char* gp = t.g + b + lo;
    const char* hp = t.h + b + lo;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!DYC) y[u] = ld16(yp + u * STEP);
      g[u] = ld16(gp + u * STEP);
      h[u] = ld16(hp + u * STEP);
    }
    halo = bwd_halo(t, w, kk, U);
  };
  auto run = [&](const uint4(&y)[U], const uint4(&g)[U], const uint4(&h)[U],
                 float halo, int64_t kk) {
    const int64_t b = sub_lo(w, kk) * 16;
    char* xp = t.dx + b + lo;
    char* dp = t.dg + b + lo;
    float hf[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u) IO::unpack(h[u], hf[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float yf[V], gf[V], dx[V], dg[V];
      if (DYC) {
#pragma unroll
        for (int j = 0; j < V; ++j) yf[j] = dyv;
      } else {
        IO::unpack(y[u], yf);
      }
      IO::unpack(g[u], gf);
      const float hin =
          (u + 1 < U) ? readlane(hf[u + 1][mem_idx<V, RB>(0)], 0) : halo;
      bwd_subtile<IO, RB, false>(gf, yf, hf[u], 0, 0, 0, carry, carry_g, hin,
                                 dx, dg);
      st16(xp + u * STEP, IO::pack(dx));
      st16(dp + u * STEP, IO::pack(dg));
    }
  };
  load(ya, ga, ha, halo_a, k);
  while (true) {
    const bool more = k + U < kend;
    if (more) load(yb, gb, hb, halo_b, k + U);
    run(ya, ga, ha, halo_a, k);
    k += U;
    if (!more) break;
    const bool more2 = k + U < kend;
    if (more2) load(ya, ga, ha, halo_a, k + U);
    run(yb, gb, hb, halo_b, k);
    k += U;
    if (!more2) break;
  }
}

template <class IO, bool RB, bool ALN, bool DYC, int U>
__device__ void bwd_item(const BwdPtrs& t, int64_t P0, int64_t P1, int lane,
                         float dyv) {
  const Walk<IO, RB> w(P0, P1, t.pend);
  float carry = 0.0f, carry_g = 1.0f;
  constexpr bool B = batch_masked_bwd<IO, U == kBwdShallow>();
  bwd_block<IO, RB, ALN, true, 1, DYC, B>(t, w, 0, lane, carry, carry_g, dyv);
  int64_t k = 1;
  if (ALN) {
    const int64_t nfull = (w.kfast - 1) / U * U;
    if (nfull > 0) {
      bwd_fast<IO, RB, U, DYC>(t, w, 1, 1 + nfull, lane, carry, carry_g, dyv);
      k = 1 + nfull;
    }
  } else {
    for (; k + U <= w.kfast; k += U)
      bwd_block<IO, RB, ALN, false, U, DYC>(t, w, k, lane, carry, carry_g, dyv);
  }
  for (; k < w.kfast; ++k)
    bwd_block<IO, RB, ALN, false, 1, DYC>(t, w, k, lane, carry, carry_g, dyv);
  for (; k < w.nsub; ++k)
    bwd_block<IO, RB, ALN, true, 1, DYC, B>(t, w, k, lane, carry, carry_g, dyv);
}

// U: sub-tiles per pipelined block (deep for long items; shallow for short
// ones, which never reach the pipelined loop but would pay its registers in
// occupancy).
template <class IO, int DIRS, bool ALN, bool WA, int U>
__global__ void __launch_bounds__(kWPB* kWave) k_scan_fwd(FwdParams p) {
  constexpr bool CHAIN = ALN && !WA && U == kFwdDeep;
  if (skipped(p)) return;
  const int lane = threadIdx.x % kWave;
  const int64_t W = p.geo.items * p.geo.nbranch;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWPB;
  if (CHAIN && p.geo.chain_ch > 0 &&
      chain_prologue(p.geo, static_cast<int64_t>(blockIdx.x) * kWPB + wave_id(),
                     stride, lane))
    return;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * kWPB + wave_id(); w < W;
       w += stride) {
    int br;
    int64_t P0, P1, row;
    if (!item_range<CHAIN>(p.geo, w, br, P0, P1, row, true)) continue;
    const FwdPtrs& t = p.br[br];
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      fwd_item<IO, false, ALN, WA, U>(t, P0, P1, lane);
    else
      fwd_item<IO, true, ALN, WA, U>(t, P0, P1, lane);
  }
}

// DIRS refers to the forward scan being differentiated: 1 = causal forward
// (adjoint runs in reverse), 2 = reverse forward (adjoint runs forward),
// 3 = branch 0 causal / branch 1 reverse.
template <class IO, int DIRS, bool ALN, bool DYC, int U>
__global__ void __launch_bounds__(kWPB* kWave) k_scan_bwd(BwdParams p) {
  constexpr bool CHAIN = ALN && U == kBwdDeep;
  if (skipped(p)) return;
  const int lane = threadIdx.x % kWave;
  const int64_t W = p.geo.items * p.geo.nbranch;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWPB;
  if (CHAIN && p.geo.chain_ch > 0 &&
      chain_prologue(p.geo, static_cast<int64_t>(blockIdx.x) * kWPB + wave_id(),
                     stride, lane))
    return;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * kWPB + wave_id(); w < W;
       w += stride) {
    int br;
    int64_t P0, P1, row;
    if (!item_range<CHAIN>(p.geo, w, br, P0, P1, row, true)) continue;
    const BwdPtrs& t = p.br[br];
    const float dyv = dyc_value<IO, DYC>(p, br, row);
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      bwd_item<IO, true, ALN, DYC, U>(t, P0, P1, lane, dyv);
    else
      bwd_item<IO, false, ALN, DYC, U>(t, P0, P1, lane, dyv);
  }
}


template <class IO, int U>
const void* pick_fwd(int dirs, bool aln, bool wa) {
#define ASC_F(D, A, W) reinterpret_cast<const void*>(&k_scan_fwd<IO, D, A, W, U>)
  if (dirs == 1) {
    if (aln) return wa ? ASC_F(1, true, true) : ASC_F(1, true, false);
    return wa ? ASC_F(1, false, true) : ASC_F(1, false, false);
  }
  if (dirs == 2) {
    if (aln) return wa ? ASC_F(2, true, true) : ASC_F(2, true, false);
    return wa ? ASC_F(2, false, true) : ASC_F(2, false, false);
  }
  return aln ? ASC_F(3, true, false) : ASC_F(3, false, false);
#undef ASC_F
}

template <class IO, int U>
const void* pick_bwd(int dirs, bool aln, bool dyc) {
#define ASC_B(D, A, Y) reinterpret_cast<const void*>(&k_scan_bwd<IO, D, A, Y, U>)
  if (dyc) {
    if (dirs == 1) return aln ? ASC_B(1, true, true) : ASC_B(1, false, true);
    if (dirs == 2) return aln ? ASC_B(2, true, true) : ASC_B(2, false, true);
    return aln ? ASC_B(3, true, true) : ASC_B(3, false, true);
  }
  if (dirs == 1) return aln ? ASC_B(1, true, false) : ASC_B(1, false, false);
  if (dirs == 2) return aln ? ASC_B(2, true, false) : ASC_B(2, false, false);
  return aln ? ASC_B(3, true, false) : ASC_B(3, false, false);
#undef ASC_B
}

}  // namespace

// Shallow-pipeline kernels for short items (scan_item_short.hip).
const void* item_fwd_short_kernel(int dtype, int dirs, bool aln, bool wa);
const void* item_bwd_short_kernel(int dtype, int dirs, bool aln, bool dyc);

}  // namespace asc

#endif  // ASC_SCAN_ITEM_H
