// Segmented scans over tiles of the flat array that may hold several
// segments and row ends (per-element head / tail / validity flags), shared
// by the look-back walk (scan_lookback.hip) and the tree walk
// (scan_tree.hip).
#ifndef ASC_SEG_COMMON_H
#define ASC_SEG_COMMON_H

#include "asc_common.h"
#include "lookback_slots.h"

namespace asc {
namespace {

struct LbGeo {
  const void* cu;
  int cu64;
  int64_t S, C, T;
  int64_t n;       // C*T elements
  int phase;
  int64_t nvec;    // 16-byte vectors covering [phase, phase + n)
  int64_t ntiles;  // tiles per branch
  int nbranch;
  uint32_t spin_limit;
};

__device__ inline int64_t lb_cu(const LbGeo& g, int64_t i) {
  const int64_t v = g.cu64 ? reinterpret_cast<const int64_t*>(g.cu)[i]
                           : static_cast<int64_t>(reinterpret_cast<const int32_t*>(g.cu)[i]);
  return v < 0 ? 0 : (v > g.T ? g.T : v);
}

// Segment of row offset t: the last s with cu[s] <= t (-1 if t < cu[0];
// S if t >= cu[S]).
__device__ inline int64_t lb_find(const LbGeo& g, int64_t t) {
  int64_t lo = 0, hi = g.S + 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (lb_cu(g, mid) <= t)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo - 1;
}

// Tile classification (uniform).  fast: every element of the tile lies in
// one segment; then phead / ptail are the positions P of that segment's
// first / last element in scan order if they are the tile's first / last
// element, else -1.
struct LbTile {
  bool fast;
  int64_t phead, ptail;
  int64_t ebase;  // first in-tensor element of the tile (memory order)
  int64_t c0;     // its row ...
  int32_t t0;     // ... and offset in the row
};

// 32-bit row offsets (the host routes T >= 2^31 - tile to the other walks).
__device__ inline int32_t lb_cu32(const LbGeo& g, int32_t i) {
  return static_cast<int32_t>(lb_cu(g, i));
}
__device__ inline int32_t lb_find32(const LbGeo& g, int32_t t) {
  int32_t lo = 0, hi = static_cast<int32_t>(g.S) + 1;
  while (lo < hi) {
    const int32_t mid = (lo + hi) >> 1;
    if (lb_cu32(g, mid) <= t)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo - 1;
}

// Per-element flags of the lane's vector vi (bit j = memory index j):
// inside the tensor, inside a segment, segment head / tail in scan order.
template <class IO, bool REV>
__device__ inline void lb_flags(const LbGeo& g, const LbTile& ti, int64_t vi,
                                uint32_t& inten, uint32_t& valid,
                                uint32_t& head, uint32_t& tail) {
  constexpr int V = IO::V;
  inten = valid = head = tail = 0;
  const int64_t e0 = vi * V - g.phase;
  if (e0 >= g.n || e0 + V <= 0) return;
  const int32_t T = static_cast<int32_t>(g.T);
  const int32_t S = static_cast<int32_t>(g.S);
  const int32_t lead = e0 < 0 ? static_cast<int32_t>(-e0) : 0;  // elements before the tensor
  // row offset of the lane's first in-tensor element
  int32_t tt = ti.t0 + static_cast<int32_t>(e0 + lead - ti.ebase);
  if (tt >= T) tt %= T;
  int32_t s = lb_find32(g, tt);
  int32_t cs = (s >= 0 && s < S) ? lb_cu32(g, s) : 0;
  int32_t ce = (s >= 0 && s < S) ? lb_cu32(g, s + 1) : 0;
  const int64_t left = g.n - e0;  // elements of the vector inside the tensor
#pragma unroll
  for (int j = 0; j < V; ++j) {
    if (j < lead || j >= left) continue;
    if (j > lead) {  // advance one element
      ++tt;
      if (tt == T) {
        tt = 0;
        s = lb_find32(g, 0);
      } else {
        while (s < S && lb_cu32(g, s + 1) <= tt) ++s;
      }
      cs = (s >= 0 && s < S) ? lb_cu32(g, s) : 0;
      ce = (s >= 0 && s < S) ? lb_cu32(g, s + 1) : 0;
    }
    inten |= 1u << j;
    if (s >= 0 && s < S && tt >= cs && tt < ce) {
      valid |= 1u << j;
      if (tt == (REV ? ce - 1 : cs)) head |= 1u << j;
      if (tt == (REV ? cs : ce - 1)) tail |= 1u << j;
    }
  }
}

// Loads the elements of vector vi that lie inside the tensor (others read
// `ident`); a full in-tensor aligned vector is one 16-byte load.
template <class IO, bool ALN>
__device__ inline void lb_load(const char* origin, int64_t vi, uint32_t inten,
                               float ident, float* f) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  if (ALN && inten == full) {
    IO::unpack(ld16(origin + vi * 16), f);
    return;
  }
#pragma unroll
  for (int j = 0; j < V; ++j) {
    float v = ident;
    if (inten & (1u << j)) v = IO::load1(origin + (vi * V + j) * IO::ES);
    f[j] = v;
  }
}

template <class IO, bool ALN>
__device__ inline void lb_store(char* origin, int64_t vi, uint32_t valid,
                                const float* f) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  if (ALN && valid == full) {
    st16(origin + vi * 16, IO::pack(f));
    return;
  }
#pragma unroll
  for (int j = 0; j < V; ++j)
    if (valid & (1u << j)) IO::store1(origin + (vi * V + j) * IO::ES, f[j]);
}

// Segmented scan over the lanes: maps (a, x) with a flag f (1 = a segment
// starts inside this lane's range, so earlier lanes do not reach past it).
template <int CTRL, int ROWMASK>
__device__ inline void seg_step(float& a, float& x, int& f) {
  const float as = dpp<CTRL, ROWMASK>(1.0f, a);
  const float xs = dpp<CTRL, ROWMASK>(0.0f, x);
  const int fs = __builtin_amdgcn_update_dpp(0, f, CTRL, ROWMASK, 0xf, false);
  if (!f) {
    x = fmaf(a, xs, x);
    a = a * as;
  }
  f |= fs;
}

__device__ inline void wave_scan_seg(float& a, float& x, int& f) {
  seg_step<kRowShr1, 0xf>(a, x, f);
  seg_step<kRowShr2, 0xf>(a, x, f);
  seg_step<kRowShr4, 0xf>(a, x, f);
  seg_step<kRowShr8, 0xf>(a, x, f);
  seg_step<kRowBcast15, 0xa>(a, x, f);
  seg_step<kRowBcast31, 0xc>(a, x, f);
}

// Result of a sub-tile's local scan: the lane's exclusive prefix (ea, ex,
// ef) and the sub-tile total (ta, tx, tf).
struct SegScan {
  float ea, ex, ta, tx;
  int ef, tf;
};

__device__ inline SegScan seg_finish(float A, float X, int F) {
  wave_scan_seg(A, X, F);
  SegScan r;
  r.ta = readlane(A, kWave - 1);
  r.tx = readlane(X, kWave - 1);
  r.tf = __builtin_amdgcn_readlane(F, kWave - 1);
  r.ea = dpp<kWaveShr1, 0xf>(1.0f, A);
  r.ex = dpp<kWaveShr1, 0xf>(0.0f, X);
  r.ef = __builtin_amdgcn_update_dpp(0, F, kWaveShr1, 0xf, 0xf, false);
  return r;
}

__device__ inline SegScan seg_from(const SubScan& s, bool head_in_subtile) {
  SegScan r;
  r.ea = s.ea;
  r.ex = s.ex;
  r.ta = s.ta;
  r.tx = s.tx;
  r.ef = 0;
  r.tf = head_in_subtile ? 1 : 0;
  return r;
}

// Carry into the lane from the carry into its sub-tile.
__device__ inline float seg_carry_in(const SegScan& s, float carry) {
  return s.ef ? s.ex : fmaf(s.ea, carry, s.ex);
}
// Carry out of a sub-tile (or tile) map.
__device__ inline float seg_apply_total(float ta, float tx, int tf,
                                        float carry) {
  return tf ? tx : fmaf(ta, carry, tx);
}

// ---- forward, segmented (slow-path) local scan and apply ----
template <class IO, bool REV>
__device__ inline SegScan fwd_local_seg(const float* g, const float* x,
                                        uint32_t valid, uint32_t head) {
  constexpr int V = IO::V;
  float A = 1.0f, X = 0.0f;
  int F = 0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, REV>(i);
    if (!(valid & (1u << j))) continue;
    if (head & (1u << j)) {
      A = 0.0f;
      X = x[j];
      F = 1;
    } else {
      X = fmaf(g[j], X, x[j]);
      A = A * g[j];
    }
  }
  return seg_finish(A, X, F);
}

template <class IO, bool REV>
__device__ inline void fwd_apply_seg(const float* g, const float* x,
                                     uint32_t valid, uint32_t head,
                                     const SegScan& s, float carry,
                                     float* hout) {
  constexpr int V = IO::V;
  float hh = seg_carry_in(s, carry);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, REV>(i);
    if (valid & (1u << j)) hh = (head & (1u << j)) ? x[j] : fmaf(g[j], hh, x[j]);
    hout[j] = hh;
  }
}

// ---- backward, segmented local scan and apply (B order = REV) ----
template <class IO, bool REV>
__device__ inline SegScan bwd_local_seg(const float* g, const float* dy,
                                        uint32_t valid, uint32_t head,
                                        float carry_g, float& gprev) {
  constexpr int V = IO::V;
  constexpr int jl = mem_idx<V, REV>(V - 1);
  gprev = dpp<kWaveShr1, 0xf>(carry_g, g[jl]);
  float A = 1.0f, X = 0.0f;
  int F = 0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, REV>(i);
    const float gs = (i == 0) ? gprev : g[mem_idx<V, REV>(i - 1)];
    if (!(valid & (1u << j))) continue;
    if (head & (1u << j)) {
      A = 0.0f;
      X = dy[j];
      F = 1;
    } else {
      X = fmaf(gs, X, dy[j]);
      A = A * gs;
    }
  }
  return seg_finish(A, X, F);
}

template <class IO, bool REV>
__device__ inline void bwd_apply_seg(const float* g, const float* dy,
                                     const float* h, uint32_t valid,
                                     uint32_t head, uint32_t tail, float gprev,
                                     float hnext_in, const SegScan& s,
                                     float carry, float* dxo, float* dgo) {
  constexpr int V = IO::V;
  constexpr int jf = mem_idx<V, REV>(0);
  const float hnx = dpp<kWaveShl1, 0xf>(hnext_in, h[jf]);
  float d = seg_carry_in(s, carry);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, REV>(i);
    const float gs = (i == 0) ? gprev : g[mem_idx<V, REV>(i - 1)];
    if (valid & (1u << j)) d = (head & (1u << j)) ? dy[j] : fmaf(gs, d, dy[j]);
    float hn = (i == V - 1) ? hnx : h[mem_idx<V, REV>(i + 1)];
    if (tail & (1u << j)) hn = 0.0f;
    dxo[j] = d;
    dgo[j] = hn * d;
  }
}

// Tile map composition: cur then sub-tile total (ta, tx, tf).
__device__ inline void lb_compose(float& A, float& X, int& F, float ta,
                                  float tx, int tf) {
  if (tf) {
    A = ta;
    X = tx;
    F = 1;
  } else {
    X = fmaf(ta, X, tx);
    A = A * ta;
  }
}

// Elements of vector vi inside the tensor (bit j = memory index j).
template <class IO>
__device__ inline uint32_t lb_inten(const LbGeo& g, int64_t vi) {
  constexpr int V = IO::V;
  const int64_t e0 = vi * V - g.phase;
  if (e0 >= 0 && e0 + V <= g.n) return (1u << V) - 1;
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < V; ++j)
    if (e0 + j >= 0 && e0 + j < g.n) m |= 1u << j;
  return m;
}


}  // namespace
}  // namespace asc

#endif  // ASC_SEG_COMMON_H
