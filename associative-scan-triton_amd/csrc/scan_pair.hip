// Two items per wave for short segments: each 32-lane half of a wave walks
// one (segment, channel) item, 32 vectors (128 fp32 / 256 fp16-bf16
// elements) per step.  A launch of short items is bound by how fast waves
// start (about 2000 per us on MI355X, 12288 one-wave items of 128 fp32
// elements: the last of them starts after 6 us, each lives 2-3 us); pairing
// halves the waves for the same instructions per item, since the halves
// scan in one pass: the DPP scan stops before the step that joins the two
// halves (row_bcast:31), and the three lane shifts that cross lane 31/32
// (the exclusive prefix, the shifted gate, the shifted state) take the
// half's own value there instead.  Every element is tested against its
// item's edges (both edges of a short item usually fall in one step).

#include "asc_common.h"

namespace asc {
namespace {

constexpr int kHalf = 32;

// The half's value at its last lane (31 or 63).
__device__ inline float half_last(float v, bool upper) {
  const float lo = readlane(v, kHalf - 1), hi = readlane(v, kWave - 1);
  return upper ? hi : lo;
}

// The lane's start value from its half's carry (carried_start within each
// half: lane 0 of a half takes the carry, not lane 31's value) and the
// half's carry out.
__device__ inline float half_carried_start(float A, float X, int hl,
                                           bool upper, float& carry) {
  half_scan_affine(A, X);
  const float y = fmaf(A, carry, X);
  float start = dpp<kWaveShr1, 0xf>(carry, y);
  if (hl == 0) start = carry;
  carry = half_last(y, upper);
  return start;
}

// Vectors of a half's item in scan order: vector i is v0 + i (forward) or
// v1 - i (reverse).
struct HalfItem {
  int64_t P0, P1;  // element range (empty: P0 = P1 = 0)
  int64_t v0, v1, nv;
  __device__ inline HalfItem(int64_t p0, int64_t p1, int V) : P0(p0), P1(p1) {
    if (P1 > P0) {
      v0 = P0 / V;
      v1 = (P1 - 1) / V;
      nv = v1 - v0 + 1;
    } else {
      v0 = v1 = 0;
      nv = 0;
    }
  }
};

template <class IO, bool REV>
__device__ inline void pair_fwd(const FwdPtrs& t, const HalfItem& it, int hl,
                                bool upper) {
  constexpr int V = IO::V;
  const int64_t nsub = (it.nv + kHalf - 1) / kHalf;
  const int64_t n0 = __builtin_amdgcn_readlane(static_cast<int>(nsub), 0);
  const int64_t n1 = __builtin_amdgcn_readlane(static_cast<int>(nsub), kHalf);
  const int64_t nmax = n0 > n1 ? n0 : n1;
  const int64_t head = REV ? it.P1 - 1 : it.P0;
  float carry = 0.0f;
  for (int64_t k = 0; k < nmax; ++k) {
    const int64_t i = k * kHalf + hl;
    const bool ok = i < it.nv;
    const int64_t vi = REV ? it.v1 - i : it.v0 + i;
    const int64_t pv = vi * V;
    float g[V], x[V];
    load_vec<IO, true, true, true>(t.g, vi, ok, it.P0, it.P1, 1.0f, g, t.pend);
    load_vec<IO, true, true, true>(t.x, vi, ok, it.P0, it.P1, 0.0f, x, t.pend);
    float A = 1.0f, X = 0.0f;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int j = mem_idx<V, REV>(e);
      if (pv + j == head) {
        A = 0.0f;
        X = x[j];
      } else {
        X = fmaf(g[j], X, x[j]);
        A = A * g[j];
      }
    }
    float h[V];
    float hh = half_carried_start(A, X, hl, upper, carry);
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int j = mem_idx<V, REV>(e);
      hh = pv + j == head ? x[j] : fmaf(g[j], hh, x[j]);
      h[j] = hh;
    }
    store_vec<IO, true, true>(t.h, vi, ok, it.P0, it.P1, h);
  }
}

// RB: B order (the adjoint's scan order) is reverse memory order.
template <class IO, bool RB, bool DYC>
__device__ inline void pair_bwd(const BwdPtrs& t, const HalfItem& it, int hl,
                                bool upper, float dyv) {
  constexpr int V = IO::V;
  constexpr int jl = mem_idx<V, RB>(V - 1);  // last element in B order
  constexpr int jf = mem_idx<V, RB>(0);      // first element in B order
  const int64_t nsub = (it.nv + kHalf - 1) / kHalf;
  const int64_t n0 = __builtin_amdgcn_readlane(static_cast<int>(nsub), 0);
  const int64_t n1 = __builtin_amdgcn_readlane(static_cast<int>(nsub), kHalf);
  const int64_t nmax = n0 > n1 ? n0 : n1;
  const int64_t head = RB ? it.P1 - 1 : it.P0;
  const int64_t tail = RB ? it.P0 : it.P1 - 1;
  float carry = 0.0f, carry_g = 1.0f;
  for (int64_t k = 0; k < nmax; ++k) {
    const int64_t i = k * kHalf + hl;
    const bool ok = i < it.nv;
    const int64_t vi = RB ? it.v1 - i : it.v0 + i;
    const int64_t pv = vi * V;
    float g[V], dy[V], h[V];
    // (DYC: the row value fills dy after the loads are issued, so that its
    // own load does not hold them back)
    if (!DYC)
      load_vec<IO, true, true, true>(t.dy, vi, ok, it.P0, it.P1, 0.0f, dy, t.pend);
    load_vec<IO, true, true, true>(t.g, vi, ok, it.P0, it.P1, 1.0f, g, t.pend);
    load_vec<IO, true, true, true>(t.h, vi, ok, it.P0, it.P1, 0.0f, h, t.pend);
    if (DYC) dyc_vec<IO, true>(dyv, vi, ok, it.P0, it.P1, dy);
    // the state just past this step in B order (0 past the item)
    const int64_t il = k * kHalf + kHalf - 1;
    const int64_t vl = RB ? it.v1 - il : it.v0 + il;
    const int64_t pn = RB ? vl * V - 1 : vl * V + V;
    const float halo =
        (pn >= it.P0 && pn < it.P1) ? IO::load1(t.h + pn * IO::ES) : 0.0f;
    // first phase: shifted gates (lane 0 of each half takes its half's
    // carry_g), the adjoint's maps
    float gprev = dpp<kWaveShr1, 0xf>(carry_g, g[jl]);
    if (hl == 0) gprev = carry_g;
    float A = 1.0f, X = 0.0f;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int j = mem_idx<V, RB>(e);
      const float gs = (e == 0) ? gprev : g[mem_idx<V, RB>(e - 1)];
      if (pv + j == head) {
        A = 0.0f;
        X = dy[j];
      } else {
        X = fmaf(gs, X, dy[j]);
        A = A * gs;
      }
    }
    float d = half_carried_start(A, X, hl, upper, carry);
    // second phase: dx, and dg from the shifted state (lane 31 of each
    // half takes its half's halo)
    float hnx = dpp<kWaveShl1, 0xf>(halo, h[jf]);
    if (hl == kHalf - 1) hnx = halo;
    float dx[V], dg[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int j = mem_idx<V, RB>(e);
      const float gs = (e == 0) ? gprev : g[mem_idx<V, RB>(e - 1)];
      d = pv + j == head ? dy[j] : fmaf(gs, d, dy[j]);
      float hn = (e == V - 1) ? hnx : h[mem_idx<V, RB>(e + 1)];
      if (pv + j == tail) hn = 0.0f;
      dx[j] = d;
      dg[j] = hn * d;
    }
    store_vec<IO, true, true>(t.dx, vi, ok, it.P0, it.P1, dx);
    store_vec<IO, true, true>(t.dg, vi, ok, it.P0, it.P1, dg);
    carry_g = half_last(g[jl], upper);
  }
}

// Pair w of a branch: items 2w and 2w + 1 of that branch (the second may
// not exist).  Both are decoded before any cu_seqlens value is read (the
// two usually share their segment: the item order pairs neighbouring
// channels), so the wave waits on one round of scalar loads.  Returns the
// lane's half's item range (empty: P0 = P1 = 0) and row.
__device__ inline void pair_items(const Geometry& geo, int64_t w, int& br,
                                  bool upper, int64_t& P0, int64_t& P1,
                                  int64_t& row) {
  const int64_t ppb = (geo.items + 1) / 2;  // pairs per branch
  br = w >= ppb ? 1 : 0;
  const int64_t loc = w - br * ppb;
  const bool two = 2 * loc + 1 < geo.items;
  int64_t s0, c0, s1 = 0, c1 = 0;
  item_seg_chan(geo, 2 * loc, true, s0, c0);
  if (two) item_seg_chan(geo, 2 * loc + 1, true, s1, c1);
  const int64_t a0 = cu_at(geo, s0), a1 = cu_at(geo, s0 + 1);
  int64_t b0 = a0, b1 = a1;
  if (two && s1 != s0) {
    b0 = cu_at(geo, s1);
    b1 = cu_at(geo, s1 + 1);
  }
  auto range = [&](int64_t t0, int64_t t1, int64_t c, int64_t& q0,
                   int64_t& q1) {
    t0 = t0 < 0 ? 0 : (t0 > geo.T ? geo.T : t0);
    t1 = t1 < t0 ? t0 : (t1 > geo.T ? geo.T : t1);
    const int64_t base = c * geo.T + geo.phase;
    q0 = t1 > t0 ? base + t0 : 0;
    q1 = t1 > t0 ? base + t1 : 0;
  };
  int64_t p0a, p1a, p0b = 0, p1b = 0;
  range(a0, a1, c0, p0a, p1a);
  if (two) range(b0, b1, c1, p0b, p1b);
  P0 = upper ? p0b : p0a;
  P1 = upper ? p1b : p1a;
  row = upper ? c1 : c0;
}

template <class IO, int DIRS>
__global__ void __launch_bounds__(kWave) k_scan_fwd_pair(FwdParams p) {
  if (skipped(p)) return;
  const int lane = threadIdx.x;
  const int hl = lane & (kHalf - 1);
  const bool upper = lane >= kHalf;
  const int64_t W = (p.geo.items + 1) / 2 * p.geo.nbranch;
  for (int64_t w = blockIdx.x; w < W; w += gridDim.x) {
    int br;
    int64_t P0, P1, row;
    pair_items(p.geo, w, br, upper, P0, P1, row);
    const HalfItem it(P0, P1, IO::V);
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      pair_fwd<IO, false>(p.br[br], it, hl, upper);
    else
      pair_fwd<IO, true>(p.br[br], it, hl, upper);
  }
}

// DIRS: the forward scan's direction, as for the other backward kernels.
template <class IO, int DIRS, bool DYC>
__global__ void __launch_bounds__(kWave) k_scan_bwd_pair(BwdParams p) {
  if (skipped(p)) return;
  const int lane = threadIdx.x;
  const int hl = lane & (kHalf - 1);
  const bool upper = lane >= kHalf;
  const int64_t W = (p.geo.items + 1) / 2 * p.geo.nbranch;
  for (int64_t w = blockIdx.x; w < W; w += gridDim.x) {
    int br;
    int64_t P0, P1, row;
    pair_items(p.geo, w, br, upper, P0, P1, row);
    const HalfItem it(P0, P1, IO::V);
    // DYC: each half's row value (read by every lane of the half)
    float dyv = 0.0f;
    if (DYC && P1 > P0) dyv = IO::load1(p.br[br].dy + row * p.dy_rs[br] * IO::ES);
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      pair_bwd<IO, true, DYC>(p.br[br], it, hl, upper, dyv);
    else
      pair_bwd<IO, false, DYC>(p.br[br], it, hl, upper, dyv);
  }
}

template <class IO>
const void* pick_fwd_pair(int dirs) {
  if (dirs == 1) return reinterpret_cast<const void*>(&k_scan_fwd_pair<IO, 1>);
  if (dirs == 2) return reinterpret_cast<const void*>(&k_scan_fwd_pair<IO, 2>);
  return reinterpret_cast<const void*>(&k_scan_fwd_pair<IO, 3>);
}

template <class IO, bool DYC>
const void* pick_bwd_pair(int dirs) {
  if (dirs == 1) return reinterpret_cast<const void*>(&k_scan_bwd_pair<IO, 1, DYC>);
  if (dirs == 2) return reinterpret_cast<const void*>(&k_scan_bwd_pair<IO, 2, DYC>);
  return reinterpret_cast<const void*>(&k_scan_bwd_pair<IO, 3, DYC>);
}

}  // namespace

// A mean segment of at most one step of a half.  Up to two or four steps
// (T = 256 / 512 fp32, 512 / 1024 bf16 and ragged segments of those means)
// ran at best even with one wave per item and lost up to 25% in the
// backward (the halves of a pair wait for the longer item).
bool pair_use(const Geometry& geo, int v) {
  return geo.T <= (geo.S > 0 ? geo.S : 1) * static_cast<int64_t>(kHalf) * v;
}

int pair_fwd(const FwdParams& p, int dtype, int dirs, void* stream) {
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = pick_fwd_pair<IoF32>(dirs); break;
    case ASC_F16: fn = pick_fwd_pair<IoF16>(dirs); break;
    default: fn = pick_fwd_pair<IoBF16>(dirs); break;
  }
  const int64_t pairs = (p.geo.items + 1) / 2 * p.geo.nbranch;
  return launch(fn, walk_grid(p, pairs, 1), 1, p, stream);
}

int pair_bwd(const BwdParams& p, int dtype, int dirs, bool dyc, void* stream) {
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = dyc ? pick_bwd_pair<IoF32, true>(dirs) : pick_bwd_pair<IoF32, false>(dirs); break;
    case ASC_F16: fn = dyc ? pick_bwd_pair<IoF16, true>(dirs) : pick_bwd_pair<IoF16, false>(dirs); break;
    default: fn = dyc ? pick_bwd_pair<IoBF16, true>(dirs) : pick_bwd_pair<IoBF16, false>(dirs); break;
  }
  const int64_t pairs = (p.geo.items + 1) / 2 * p.geo.nbranch;
  return launch(fn, walk_grid(p, pairs, 1), 1, p, stream);
}

}  // namespace asc
