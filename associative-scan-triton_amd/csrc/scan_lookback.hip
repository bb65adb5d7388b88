#include <atomic>

#include "seg_common.h"

namespace asc {
namespace {

// ===========================================================================
// Decoupled look-back walk (single pass over in-order tiles).
//
// The per-item walks give each (segment, channel) item to one wave or one
// workgroup, so a problem with few items (one long sequence, a handful of
// channels) leaves most of the 256 CUs idle.  This walk cuts the flat array
// of all rows into tiles of 16384 elements instead, so its parallelism is
// the element count.  Workgroup b (kLbWaves waves) owns tile b in scan order
// (address order, or reverse address order for a reverse-direction scan);
// wave w owns part w of it, 1024 elements.  A part may hold the end of one
// segment and the start of others (or the end of one row and the start of
// the next): segment heads reset the scan inside it.  Each tile
//   1. loads its data and scans it locally, one part per wave, and the part
//      maps meet in LDS;
//   2. (wave 0) publishes the tile's aggregate map (A, X) in its workspace
//      slot -- or, if a segment starts inside the tile, directly its
//      inclusive value, which no longer depends on earlier tiles;
//   3. (wave 0) unless its first element in a segment is a head, looks back
//      over the slots of the preceding tiles, 64 at a time (one per lane),
//      composing aggregates with the same DPP scan until it meets an
//      inclusive value, and publishes its own inclusive value;
//   4. every wave takes the tile carry through the parts before its own and
//      writes its outputs.
// Slot words are (status << 32 | float bits), written and read with
// agent-scope atomics (the 8 XCDs have separate L2 caches, so every poll is
// a round trip past them); the workspace is zero-filled by a small kernel
// before every launch.  Every wait is bounded: after g_spin_limit (2^14 by
// default) unsuccessful polls the waiting wave computes the missing
// predecessor's map from that tile's inputs itself, so progress never
// depends on the order in which workgroups are scheduled.
//
// Measured on MI355X, a poll round trip under full HBM load costs about as
// much as a tile's own loads, so with many items the per-item walks (which
// need no inter-workgroup communication) stream faster; the host picks this
// walk only for problems with few items (lb_use).  Which predecessor a tile
// meets as inclusive depends on timing, so the last bits of the results can
// vary from run to run.
// ===========================================================================
// Parts are 1024 elements for every element type: 4 sub-tiles of 64 lanes x
// 4 fp32, or 2 sub-tiles of 64 lanes x 8 fp16/bf16 (ASC_LB_U_F32 sets the
// fp32 part for experiments).
#ifndef ASC_LB_U_F32
#define ASC_LB_U_F32 4
#endif
template <class IO>
constexpr int LbU = IO::V == 4 ? ASC_LB_U_F32 : 2;  // sub-tiles per part
template <class IO>
constexpr int64_t LbTileVec = static_cast<int64_t>(LbU<IO>) * kWave;  // per part
// 16 waves (16384-element tiles): a poll costs the same for any tile size,
// so fewer, larger tiles stream faster (measured with one 2^27-element row:
// 4.1 / 4.7 TB/s fwd / bwd fp32 against 3.3 / 4.0 with 4 waves; 8 waves
// were no better than 4 at the occupancy their register use allows).
#ifndef ASC_LB_WAVES
#define ASC_LB_WAVES 16
#endif
constexpr int kLbWaves = ASC_LB_WAVES;  // parts (waves) per workgroup tile
// Elements per part for v elements per vector (host side; matches LbU).
constexpr int64_t lb_part_elems(int v) {
  return v == 4 ? 256 * ASC_LB_U_F32 : 2 * 512;
}

// Vector owned by `lane` in sub-tile u of tile t (scan order).
template <class IO, bool REV>
__device__ inline int64_t lb_vec(const LbGeo& g, int64_t t, int u, int lane) {
  const int64_t i = t * LbTileVec<IO> + static_cast<int64_t>(u) * kWave + lane;
  return REV ? g.nvec - 1 - i : i;
}


template <class IO, bool REV>
__device__ inline LbTile lb_classify(const LbGeo& g, int64_t t) {
  constexpr int V = IO::V;
  LbTile r{false, -1, -1, 0, 0, 0};
  const int64_t v_lo = REV ? g.nvec - (t + 1) * LbTileVec<IO> : t * LbTileVec<IO>;
  const int64_t e_lo = uniform(v_lo * V - g.phase);
  const int64_t e_hi = e_lo + LbTileVec<IO> * V;
  r.ebase = e_lo < 0 ? 0 : e_lo;
  r.c0 = uniform(r.ebase / g.T);
  r.t0 = static_cast<int32_t>(r.ebase - r.c0 * g.T);
  if (v_lo < 0 || e_lo < 0 || e_hi > g.n) return r;
  if ((e_hi - 1) / g.T != r.c0) return r;
  const int64_t c = r.c0;
  const int64_t tl = e_lo - c * g.T, th = e_hi - c * g.T;
  const int64_t s = uniform(lb_find(g, tl));
  if (s < 0 || s >= g.S) return r;
  const int64_t cs = uniform(lb_cu(g, s)), ce = uniform(lb_cu(g, s + 1));
  if (ce < th) return r;
  r.fast = true;
  const int64_t base = c * g.T + g.phase;
  const int64_t hd = REV ? ce - 1 : cs;   // segment's first scan element
  const int64_t tl_ = REV ? cs : ce - 1;  // segment's last scan element
  if (hd == (REV ? th - 1 : tl)) r.phead = base + hd;
  if (tl_ == (REV ? tl : th - 1)) r.ptail = base + tl_;
  return r;
}

// Per-tile scan state of the forward kernel.
template <class IO>
struct FwdTile {
  float g[LbU<IO>][IO::V], x[LbU<IO>][IO::V];
  uint32_t valid[LbU<IO>], head[LbU<IO>];
  SegScan sc[LbU<IO>];
  float A, X;
  int F;
  bool need_carry;
  bool any;  // some element of the part lies in a segment
};

// Whether the tile needs a carry: it does unless the first element (scan
// order) that lies in a segment is a segment head.  Slow path only.
template <class IO, bool REV>
__device__ inline bool lb_needs_carry(const uint32_t* valid, const uint32_t* head) {
  constexpr int V = IO::V;
#pragma unroll
  for (int u = 0; u < LbU<IO>; ++u) {
    const u64 any = __builtin_amdgcn_ballot_w64(valid[u] != 0);
    if (!any) continue;
    const int l0 = __builtin_ctzll(any);
    int fh = 0;
    bool got = false;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int j = mem_idx<V, REV>(i);
      if (!got && (valid[u] & (1u << j))) {
        got = true;
        fh = (head[u] >> j) & 1;
      }
    }
    return !__builtin_amdgcn_readlane(fh, l0);
  }
  return false;
}

// Loads and scans tile t locally (no stores); fills the tile map.  The data
// loads depend on the tensor bounds only, so they are issued before the
// segment lookup and their latency covers it.
template <class IO, bool REV, bool ALN>
__device__ inline void fwd_tile_local(const FwdPtrs& p, const LbGeo& geo,
                                      int64_t t, int lane, FwdTile<IO>& s) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  uint32_t inten[LbU<IO>];
#pragma unroll
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    inten[u] = lb_inten<IO>(geo, vi);
    lb_load<IO, ALN>(p.g, vi, inten[u], 1.0f, s.g[u]);
    lb_load<IO, ALN>(p.x, vi, inten[u], 0.0f, s.x[u]);
  }
  const LbTile ti = lb_classify<IO, REV>(geo, t);
  s.A = 1.0f;
  s.X = 0.0f;
  s.F = 0;
  if (ti.fast) {
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      s.valid[u] = full;
      s.head[u] = 0;
    }
    if (ti.phead >= 0 && lane == 0) s.head[0] = 1u << mem_idx<V, REV>(0);
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      const int64_t pv = lb_vec<IO, REV>(geo, t, u, lane) * V;
      SubScan ss;
      if (u == 0)
        ss = fwd_local<IO, REV, true>(s.g[u], s.x[u], pv, ti.phead);
      else
        ss = fwd_local<IO, REV, false>(s.g[u], s.x[u], pv, -1);
      s.sc[u] = seg_from(ss, u == 0 && ti.phead >= 0);
      lb_compose(s.A, s.X, s.F, s.sc[u].ta, s.sc[u].tx, s.sc[u].tf);
    }
    s.need_carry = ti.phead < 0;
    s.any = true;
    return;
  }
  uint32_t anyv = 0;
#pragma unroll
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    uint32_t in2, tail;
    lb_flags<IO, REV>(geo, ti, vi, in2, s.valid[u], s.head[u], tail);
    anyv |= s.valid[u];
    s.sc[u] = fwd_local_seg<IO, REV>(s.g[u], s.x[u], s.valid[u], s.head[u]);
    lb_compose(s.A, s.X, s.F, s.sc[u].ta, s.sc[u].tx, s.sc[u].tf);
  }
  s.need_carry = lb_needs_carry<IO, REV>(s.valid, s.head);
  s.any = __builtin_amdgcn_ballot_w64(anyv != 0) != 0;
}

// Composes the maps of the tiles before t (scan order) until an inclusive
// value; returns the carry into tile t.  Window of 64 tiles: lane r polls
// tile top - 63 + r, so lane 63 is the nearest and one DPP scan composes
// the window in scan order.  (Wider windows, several slots per lane, were
// slower: every extra slot is another device-coherent load per poll.)
// `compute(j, A, X, F)` recomputes tile j's map from its inputs (the
// bounded-wait fallback).
template <class Compute>
__device__ float lb_lookback(const LbGeo& geo, LbSlot* slots, int64_t t,
                             int lane, Compute compute) {
  float acc_a = 1.0f, acc_x = 0.0f;
  int64_t top = t - 1;
  uint32_t spins = 0;
  while (true) {
    const int64_t j = top - (kWave - 1) + lane;
    float a, x;
    int kind = lb_read(&slots[j < 0 ? 0 : j], a, x);
    if (j < 0) {  // before the first tile: inclusive 0
      kind = kLbIncl;
      x = 0.0f;
    }
    u64 incl = __builtin_amdgcn_ballot_w64(kind == kLbIncl);
    int r_inc = incl ? 63 - __builtin_clzll(incl) : -1;
    u64 above = r_inc >= 63 ? 0ull : (~0ull << (r_inc + 1));
    u64 missing = __builtin_amdgcn_ballot_w64(kind == kLbNone) & above;
    if (missing) {
      if (++spins <= geo.spin_limit) {
        __builtin_amdgcn_s_sleep(2);
        continue;
      }
      // Bounded wait expired: compute the missing maps from the tiles'
      // inputs, nearest first (a tile with a segment head is inclusive).
      while (missing) {
        const int r = 63 - __builtin_clzll(missing);
        float ma, mx;
        int mf;
        compute(top - (kWave - 1) + r, ma, mx, mf);
        if (lane == r) {
          kind = mf ? kLbIncl : kLbAgg;
          a = ma;
          x = mx;
        }
        incl = __builtin_amdgcn_ballot_w64(kind == kLbIncl);
        r_inc = incl ? 63 - __builtin_clzll(incl) : -1;
        above = r_inc >= 63 ? 0ull : (~0ull << (r_inc + 1));
        missing = __builtin_amdgcn_ballot_w64(kind == kLbNone) & above;
      }
      spins = 0;
    }
    float ma = a, mx = x;
    if (lane < r_inc) {
      ma = 1.0f;
      mx = 0.0f;
    } else if (lane == r_inc) {
      ma = 0.0f;
    }
    wave_scan_affine(ma, mx);
    const float ra = readlane(ma, kWave - 1);
    const float rx = readlane(mx, kWave - 1);
    acc_x = fmaf(acc_a, rx, acc_x);
    acc_a = acc_a * ra;
    if (r_inc >= 0) return acc_x;
    top -= kWave;
  }
}

// The map (A, X, F) of tile t computed from its inputs one sub-tile at a
// time (the bounded-wait fallback of the look-back; nothing is stored).
template <class IO, bool REV, bool ALN>
__device__ __attribute__((noinline)) void fwd_tile_map(const FwdPtrs p, const LbGeo geo,
                                                       int64_t t, int lane, float& A,
                                                       float& X, int& F) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  const LbTile ti = lb_classify<IO, REV>(geo, t);
  A = 1.0f;
  X = 0.0f;
  F = 0;
#pragma unroll 1
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    float g[V], x[V];
    if (ti.fast) {
      lb_load<IO, ALN>(p.g, vi, full, 1.0f, g);
      lb_load<IO, ALN>(p.x, vi, full, 0.0f, x);
      const SubScan ss = fwd_local<IO, REV, true>(g, x, vi * V,
                                                  u == 0 ? ti.phead : -1);
      lb_compose(A, X, F, ss.ta, ss.tx, u == 0 && ti.phead >= 0);
    } else {
      uint32_t inten, valid, head, tail;
      lb_flags<IO, REV>(geo, ti, vi, inten, valid, head, tail);
      lb_load<IO, ALN>(p.g, vi, inten, 1.0f, g);
      lb_load<IO, ALN>(p.x, vi, inten, 0.0f, x);
      const SegScan sc = fwd_local_seg<IO, REV>(g, x, valid, head);
      lb_compose(A, X, F, sc.ta, sc.tx, sc.tf);
    }
  }
}

// A workgroup tile is kLbWaves consecutive parts, one per wave.  The waves
// share their part maps through LDS; wave 0 composes them into the tile
// map, publishes it, looks back and hands the tile's carry-in to the others.
struct LbPart {
  float a, x;
  int f;      // a segment head lies inside the part
  int flags;  // bit 1: some element lies in a segment; bit 0: needs a carry
};

// Tile map (A, X, F) from the parts and whether the tile needs a carry (the
// first part that holds segment elements needs one).
__device__ inline bool lb_tile_from_parts(const LbPart* parts, float& A,
                                          float& X, int& F) {
  A = 1.0f;
  X = 0.0f;
  F = 0;
  int nc = -1;
#pragma unroll
  for (int k = 0; k < kLbWaves; ++k) {
    const LbPart q = parts[k];
    lb_compose(A, X, F, q.a, q.x, q.f);
    if (nc < 0 && (q.flags & 2)) nc = q.flags & 1;
  }
  return nc > 0;
}

// Carry into part wv from the tile's carry-in.
__device__ inline float lb_part_carry(const LbPart* parts, int wv, float carry) {
  for (int k = 0; k < wv; ++k) {
    const LbPart q = parts[k];
    carry = q.f ? q.x : fmaf(q.a, carry, q.x);
  }
  return carry;
}

struct LbFwdParams {
  LbGeo geo;
  FwdPtrs br[2];
  LbSlot* slots;  // nbranch * ntiles
};

template <class IO, int DIRS, bool ALN>
__global__ void __launch_bounds__(kLbWaves* kWave) k_scan_fwd_lb(LbFwdParams p) {
  __shared__ LbPart parts[kLbWaves];
  __shared__ float tile_carry;
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  const int64_t gt = blockIdx.x;
  const int br = gt >= p.geo.ntiles ? 1 : 0;
  const int64_t t = gt - br * p.geo.ntiles;
  if (br >= p.geo.nbranch) return;  // whole workgroup
  LbSlot* slots = p.slots + br * p.geo.ntiles;
  auto run = [&](auto rev_tag) {
    constexpr bool REV = decltype(rev_tag)::value;
    constexpr int V = IO::V;
    const FwdPtrs q = p.br[br];
    FwdTile<IO> s;
    fwd_tile_local<IO, REV, ALN>(q, p.geo, t * kLbWaves + wv, lane, s);
    if (lane == 0)
      parts[wv] = LbPart{s.A, s.X, s.F, (s.any ? 2 : 0) | (s.need_carry ? 1 : 0)};
    __syncthreads();
    if (wv == 0) {
      float A, X;
      int F;
      const bool need = lb_tile_from_parts(parts, A, X, F);
      if (lane == 0) {
        if (F) {
          lb_put(&slots[t].x, kLbIncl, X);
        } else {
          lb_put(&slots[t].a, kLbAgg, A);
          lb_put(&slots[t].x, kLbAgg, X);
        }
      }
      float carry = 0.0f;
      if (need)
        carry = lb_lookback(p.geo, slots, t, lane,
                            [&](int64_t j, float& a, float& x, int& f) {
                              a = 1.0f;
                              x = 0.0f;
                              f = 0;
                              for (int k = 0; k < kLbWaves; ++k) {
                                float ma, mx;
                                int mf;
                                fwd_tile_map<IO, REV, ALN>(q, p.geo, j * kLbWaves + k,
                                                           lane, ma, mx, mf);
                                lb_compose(a, x, f, ma, mx, mf);
                              }
                            });
      if (lane == 0) {
        if (!F) lb_put(&slots[t].x, kLbIncl, fmaf(A, carry, X));
        tile_carry = carry;
      }
    }
    __syncthreads();
    float carry = lb_part_carry(parts, wv, tile_carry);
    const int64_t pt = t * kLbWaves + wv;
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      const int64_t vi = lb_vec<IO, REV>(p.geo, pt, u, lane);
      float hf[V];
      fwd_apply_seg<IO, REV>(s.g[u], s.x[u], s.valid[u], s.head[u], s.sc[u],
                             carry, hf);
      lb_store<IO, ALN>(q.h, vi, s.valid[u], hf);
      carry = seg_apply_total(s.sc[u].ta, s.sc[u].tx, s.sc[u].tf, carry);
    }
  };
  if (DIRS == 1 || (DIRS == 3 && br == 0))
    run(std::integral_constant<bool, false>{});
  else
    run(std::integral_constant<bool, true>{});
}

// Per-tile scan state of the backward kernel (B order = REV).
template <class IO>
struct BwdTile {
  float y[LbU<IO>][IO::V], g[LbU<IO>][IO::V], h[LbU<IO>][IO::V];
  uint32_t valid[LbU<IO>], head[LbU<IO>], tail[LbU<IO>];
  float gprev[LbU<IO>];
  SegScan sc[LbU<IO>];
  float hn;  // state just after the part in B order (0 outside the tensor)
  float A, X;
  int F;
  bool need_carry;
  bool any;  // some element of the part lies in a segment
};

template <class IO, bool REV, bool ALN>
__device__ inline void bwd_tile_local(const BwdPtrs& p, const LbGeo& geo,
                                      int64_t t, int lane, BwdTile<IO>& s) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  constexpr int jl = mem_idx<V, REV>(V - 1);
  // data and halos first (tensor bounds only): the gate before the tile and
  // the state after it (B order)
  uint32_t inten[LbU<IO>];
#pragma unroll
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    inten[u] = lb_inten<IO>(geo, vi);
    lb_load<IO, ALN>(p.dy, vi, inten[u], 0.0f, s.y[u]);
    lb_load<IO, ALN>(p.g, vi, inten[u], 1.0f, s.g[u]);
    lb_load<IO, ALN>(p.h, vi, inten[u], 0.0f, s.h[u]);
  }
  float cg = 1.0f;
  {
    const int64_t pf = lb_vec<IO, REV>(geo, t, 0, 0) * V + mem_idx<V, REV>(0);
    const int64_t pp = REV ? pf + 1 : pf - 1;
    const int64_t e = pp - geo.phase;
    if (e >= 0 && e < geo.n) cg = IO::load1(p.g + pp * IO::ES);
    const int64_t pl =
        lb_vec<IO, REV>(geo, t, LbU<IO> - 1, kWave - 1) * V + mem_idx<V, REV>(V - 1);
    const int64_t pn = REV ? pl - 1 : pl + 1;
    const int64_t en = pn - geo.phase;
    s.hn = (en >= 0 && en < geo.n) ? IO::load1(p.h + pn * IO::ES) : 0.0f;
  }
  const LbTile ti = lb_classify<IO, REV>(geo, t);
  s.A = 1.0f;
  s.X = 0.0f;
  s.F = 0;
  if (ti.fast) {
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      s.valid[u] = full;
      s.head[u] = 0;
      s.tail[u] = 0;
    }
    if (ti.phead >= 0 && lane == 0) s.head[0] = 1u << mem_idx<V, REV>(0);
    if (ti.ptail >= 0 && lane == kWave - 1)
      s.tail[LbU<IO> - 1] = 1u << mem_idx<V, REV>(V - 1);
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      const int64_t pv = lb_vec<IO, REV>(geo, t, u, lane) * V;
      SubScan ss;
      if (u == 0)
        ss = bwd_local<IO, REV, true>(s.g[u], s.y[u], pv, ti.phead, cg, s.gprev[u]);
      else
        ss = bwd_local<IO, REV, false>(s.g[u], s.y[u], pv, -1, cg, s.gprev[u]);
      cg = readlane(s.g[u][jl], kWave - 1);
      s.sc[u] = seg_from(ss, u == 0 && ti.phead >= 0);
      lb_compose(s.A, s.X, s.F, s.sc[u].ta, s.sc[u].tx, s.sc[u].tf);
    }
    s.need_carry = ti.phead < 0;
    s.any = true;
    return;
  }
  uint32_t anyv = 0;
#pragma unroll
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    uint32_t in2;
    lb_flags<IO, REV>(geo, ti, vi, in2, s.valid[u], s.head[u], s.tail[u]);
    anyv |= s.valid[u];
    s.sc[u] = bwd_local_seg<IO, REV>(s.g[u], s.y[u], s.valid[u], s.head[u], cg,
                                     s.gprev[u]);
    cg = readlane(s.g[u][jl], kWave - 1);
    lb_compose(s.A, s.X, s.F, s.sc[u].ta, s.sc[u].tx, s.sc[u].tf);
  }
  s.need_carry = lb_needs_carry<IO, REV>(s.valid, s.head);
  s.any = __builtin_amdgcn_ballot_w64(anyv != 0) != 0;
}

template <class IO, bool REV, bool ALN>
__device__ __attribute__((noinline)) void bwd_tile_map(const BwdPtrs p, const LbGeo geo,
                                                       int64_t t, int lane, float& A,
                                                       float& X, int& F) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  constexpr int jl = mem_idx<V, REV>(V - 1);
  const LbTile ti = lb_classify<IO, REV>(geo, t);
  float cg = 1.0f;
  {
    const int64_t pf = lb_vec<IO, REV>(geo, t, 0, 0) * V + mem_idx<V, REV>(0);
    const int64_t pp = REV ? pf + 1 : pf - 1;
    const int64_t e = pp - geo.phase;
    if (e >= 0 && e < geo.n) cg = IO::load1(p.g + pp * IO::ES);
  }
  A = 1.0f;
  X = 0.0f;
  F = 0;
#pragma unroll 1
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    float g[V], y[V], gprev;
    if (ti.fast) {
      lb_load<IO, ALN>(p.g, vi, full, 1.0f, g);
      lb_load<IO, ALN>(p.dy, vi, full, 0.0f, y);
      const SubScan ss = bwd_local<IO, REV, true>(g, y, vi * V,
                                                  u == 0 ? ti.phead : -1, cg, gprev);
      lb_compose(A, X, F, ss.ta, ss.tx, u == 0 && ti.phead >= 0);
    } else {
      uint32_t inten, valid, head, tail;
      lb_flags<IO, REV>(geo, ti, vi, inten, valid, head, tail);
      lb_load<IO, ALN>(p.g, vi, inten, 1.0f, g);
      lb_load<IO, ALN>(p.dy, vi, inten, 0.0f, y);
      const SegScan sc = bwd_local_seg<IO, REV>(g, y, valid, head, cg, gprev);
      lb_compose(A, X, F, sc.ta, sc.tx, sc.tf);
    }
    cg = readlane(g[jl], kWave - 1);
  }
}

struct LbBwdParams {
  LbGeo geo;
  BwdPtrs br[2];
  LbSlot* slots;
};

// DIRS as k_scan_bwd: 1 = causal (B order reverse), 2 = anti-causal,
// 3 = branch 0 causal / branch 1 anti-causal.
template <class IO, int DIRS, bool ALN>
__global__ void __launch_bounds__(kLbWaves* kWave) k_scan_bwd_lb(LbBwdParams p) {
  __shared__ LbPart parts[kLbWaves];
  __shared__ float tile_carry;
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  const int64_t gt = blockIdx.x;
  const int br = gt >= p.geo.ntiles ? 1 : 0;
  const int64_t t = gt - br * p.geo.ntiles;
  if (br >= p.geo.nbranch) return;  // whole workgroup
  LbSlot* slots = p.slots + br * p.geo.ntiles;
  auto run = [&](auto rev_tag) {
    constexpr bool REV = decltype(rev_tag)::value;
    constexpr int V = IO::V;
    constexpr int jf = mem_idx<V, REV>(0);
    const BwdPtrs q = p.br[br];
    const int64_t pt = t * kLbWaves + wv;
    BwdTile<IO> s;
    bwd_tile_local<IO, REV, ALN>(q, p.geo, pt, lane, s);
    if (lane == 0)
      parts[wv] = LbPart{s.A, s.X, s.F, (s.any ? 2 : 0) | (s.need_carry ? 1 : 0)};
    __syncthreads();
    if (wv == 0) {
      float A, X;
      int F;
      const bool need = lb_tile_from_parts(parts, A, X, F);
      if (lane == 0) {
        if (F) {
          lb_put(&slots[t].x, kLbIncl, X);
        } else {
          lb_put(&slots[t].a, kLbAgg, A);
          lb_put(&slots[t].x, kLbAgg, X);
        }
      }
      float carry = 0.0f;
      if (need)
        carry = lb_lookback(p.geo, slots, t, lane,
                            [&](int64_t j, float& a, float& x, int& f) {
                              a = 1.0f;
                              x = 0.0f;
                              f = 0;
                              for (int k = 0; k < kLbWaves; ++k) {
                                float ma, mx;
                                int mf;
                                bwd_tile_map<IO, REV, ALN>(q, p.geo, j * kLbWaves + k,
                                                           lane, ma, mx, mf);
                                lb_compose(a, x, f, ma, mx, mf);
                              }
                            });
      if (lane == 0) {
        if (!F) lb_put(&slots[t].x, kLbIncl, fmaf(A, carry, X));
        tile_carry = carry;
      }
    }
    __syncthreads();
    float carry = lb_part_carry(parts, wv, tile_carry);
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      const int64_t vi = lb_vec<IO, REV>(p.geo, pt, u, lane);
      const float hin = (u + 1 < LbU<IO>) ? readlane(s.h[u + 1][jf], 0) : s.hn;
      float dx[V], dg[V];
      bwd_apply_seg<IO, REV>(s.g[u], s.y[u], s.h[u], s.valid[u], s.head[u],
                             s.tail[u], s.gprev[u], hin, s.sc[u], carry, dx, dg);
      lb_store<IO, ALN>(q.dx, vi, s.valid[u], dx);
      lb_store<IO, ALN>(q.dg, vi, s.valid[u], dg);
      carry = seg_apply_total(s.sc[u].ta, s.sc[u].tx, s.sc[u].tf, carry);
    }
  };
  if (DIRS == 1 || (DIRS == 3 && br == 0))
    run(std::integral_constant<bool, true>{});
  else
    run(std::integral_constant<bool, false>{});
}

__global__ void __launch_bounds__(256) k_fill_zero(u64* p, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += stride)
    p[i] = 0;
}

// Look-back and chained walks: polls before a waiting wave computes a
// missing predecessor itself (a test hook can lower it to exercise that
// path).  Process-wide; read once per launch on the host, so an atomic with
// relaxed order is enough for concurrent callers on several host threads.
std::atomic<uint32_t> g_spin_limit{1u << 14};

// Tiles of the look-back walk: kLbWaves parts each, from the start of the
// phase frame (the vectors of every element type divide 1024).
int64_t lb_ntiles(int64_t n, int phase, int v) {
  const int64_t te = lb_part_elems(v) * kLbWaves;
  return (phase + n + te - 1) / te;
}


template <class IO>
const void* pick_fwd_lb(int dirs, bool aln) {
#define ASC_F(D, A) reinterpret_cast<const void*>(&k_scan_fwd_lb<IO, D, A>)
  if (dirs == 1) return aln ? ASC_F(1, true) : ASC_F(1, false);
  if (dirs == 2) return aln ? ASC_F(2, true) : ASC_F(2, false);
  return aln ? ASC_F(3, true) : ASC_F(3, false);
#undef ASC_F
}

template <class IO>
const void* pick_bwd_lb(int dirs, bool aln) {
#define ASC_B(D, A) reinterpret_cast<const void*>(&k_scan_bwd_lb<IO, D, A>)
  if (dirs == 1) return aln ? ASC_B(1, true) : ASC_B(1, false);
  if (dirs == 2) return aln ? ASC_B(2, true) : ASC_B(2, false);
  return aln ? ASC_B(3, true) : ASC_B(3, false);
#undef ASC_B
}

// Look-back geometry of a call whose per-item parameters are `geo`; false
// when the workspace is missing, misaligned or too small for it.
bool lb_prepare(const Geometry& geo, int v, void* ws, int64_t ws_bytes,
                LbGeo& lg, int64_t& need) {
  if (!ws || reinterpret_cast<uintptr_t>(ws) % 32 != 0) return false;
  lg = LbGeo{geo.cu, geo.cu64, geo.S, geo.C, geo.T, geo.C * geo.T, geo.phase,
             0, 0, geo.nbranch, g_spin_limit.load(std::memory_order_relaxed)};
  lg.nvec = (lg.phase + lg.n + v - 1) / v;
  lg.ntiles = lb_ntiles(lg.n, lg.phase, v);
  need = lg.ntiles * geo.nbranch * static_cast<int64_t>(sizeof(LbSlot));
  return ws_bytes >= need;
}

}  // namespace

int fill_zero(void* ws, int64_t bytes, void* stream) {
  const int64_t words = bytes / 8;
  int64_t blocks = (words + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  u64* p = static_cast<u64*>(ws);
  int64_t n = words;
  void* args[] = {&p, &n};
  const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&k_fill_zero),
                                       dim3(static_cast<unsigned>(blocks)), dim3(256),
                                       args, 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ASC_OK : static_cast<int>(e);
}

// Walk choice: the look-back walk for problems with few (segment, channel)
// items (each item of the other walks is one wave or one workgroup, which
// leaves most CUs idle), the per-item walks otherwise.  Measured on MI355X
// (2^27 elements): the look-back walk streams about 4.1 / 4.7 TB/s (fwd /
// bwd) fp32 and 2.4 / 3.0 bf16 at any item count; 16-wave workgroups per
// item reach 2.4 / 2.6 (fp32) and 1.5 / 1.3 (bf16) at 64 items, 4.4 / 4.6
// and 2.8 / 2.3 at 128, and overtake beyond.  The look-back kernels also
// keep row offsets and segment indices in 32 bits, and need one workgroup
// per tile (no grid-stride loop), so the tiles must fit one grid.
#ifndef ASC_LB_MAX_ITEMS_F32
#define ASC_LB_MAX_ITEMS_F32 128
#endif
#ifndef ASC_LB_MAX_ITEMS_HALF
#define ASC_LB_MAX_ITEMS_HALF 128
#endif
bool lb_use(int64_t S, int64_t C, int64_t T, int nbranch, int v) {
  if (S <= 0 || C <= 0 || T <= 0) return false;
  if (T >= (int64_t(1) << 30) || S >= (int64_t(1) << 30)) return false;
  const int64_t max_items = v == 4 ? ASC_LB_MAX_ITEMS_F32 : ASC_LB_MAX_ITEMS_HALF;
  if (S * C * nbranch > max_items) return false;
  return lb_ntiles(C * T, v - 1, v) * nbranch <= kMaxGrid;
}

// Workspace bytes for the worst-case phase (v - 1).
int64_t lb_bytes(int64_t n, int v, int nbranch) {
  return lb_ntiles(n, v - 1, v) * nbranch * static_cast<int64_t>(sizeof(LbSlot));
}

unsigned lb_spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }

unsigned lb_set_spin_limit(unsigned polls) {
  return g_spin_limit.exchange(polls, std::memory_order_relaxed);
}

bool lb_fwd(const FwdParams& p, int dtype, int dirs, bool aln, void* ws,
            int64_t ws_bytes, void* stream, int& status) {
  LbFwdParams q{};
  int64_t need = 0;
  if (!lb_prepare(p.geo, 16 / elem_size(dtype), ws, ws_bytes, q.geo, need))
    return false;
  for (int b = 0; b < p.geo.nbranch; ++b) q.br[b] = p.br[b];
  q.slots = static_cast<LbSlot*>(ws);
  if ((status = fill_zero(ws, need, stream))) return true;
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = pick_fwd_lb<IoF32>(dirs, aln); break;
    case ASC_F16: fn = pick_fwd_lb<IoF16>(dirs, aln); break;
    default: fn = pick_fwd_lb<IoBF16>(dirs, aln); break;
  }
  status = launch(fn, q.geo.ntiles * p.geo.nbranch, kLbWaves, q, stream);
  return true;
}

bool lb_bwd(const BwdParams& p, int dtype, int dirs, bool aln, void* ws,
            int64_t ws_bytes, void* stream, int& status) {
  LbBwdParams q{};
  int64_t need = 0;
  if (!lb_prepare(p.geo, 16 / elem_size(dtype), ws, ws_bytes, q.geo, need))
    return false;
  for (int b = 0; b < p.geo.nbranch; ++b) q.br[b] = p.br[b];
  q.slots = static_cast<LbSlot*>(ws);
  if ((status = fill_zero(ws, need, stream))) return true;
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = pick_bwd_lb<IoF32>(dirs, aln); break;
    case ASC_F16: fn = pick_bwd_lb<IoF16>(dirs, aln); break;
    default: fn = pick_bwd_lb<IoBF16>(dirs, aln); break;
  }
  status = launch(fn, q.geo.ntiles * p.geo.nbranch, kLbWaves, q, stream);
  return true;
}

}  // namespace asc
