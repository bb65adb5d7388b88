// Backward that recomputes the forward states (asc_scan_bwd_recompute).
//
// The autograd functions normally keep the forward's output h alive until
// the backward, one [C, T] tensor per call.  In the opt-in recompute mode
// they keep the forward's inputs (gates, tokens) and one checkpoint per
// chunk of each row instead: the forward state just before the chunk in
// forward-scan order (asc_scan_checkpoints samples it from h right after the
// forward; 4 bytes per 4096 fp32 / 8192 fp16-bf16 elements).  The backward
// here reads dy, g and x (not h), recomputes h chunk by chunk in registers
// from the chunk's checkpoint, rounds it to the storage type (the states the
// plain backward would have read) and runs the fused backward on it: still
// 5 tensors of traffic (20 bytes per fp32 element), no h in memory.
//
// A chunk is the chained walk's (kChainWaves x kChainU sub-tiles: 4096 fp32
// / 8192 fp16-bf16 elements of one row), lanes in B order (the adjoint's
// scan order, as in scan_chain.hip).  Per chunk:
//   1. each wave loads its two sub-tiles of dy, g, x; computes the forward
//      recurrence's per-lane maps in forward order (the reverse of B order:
//      lanes are mirrored with ds_bpermute for that DPP scan) and the
//      adjoint's maps in B order; the wave maps meet in LDS;
//   2. each wave composes its forward carry (checkpoint, then the maps of
//      the waves before it in forward order) and recomputes its states; the
//      state of its first element in B order goes to LDS (the neighbouring
//      wave's shifted state);
//   3. each wave composes its backward carry and writes dx, dg.
// Two walks use it:
//   * chained (k_scan_bwd_rc_chain): one workgroup per chunk with the
//     chained walk's slots, for segments aligned to the chunk grid (tested
//     on the device, as in scan_chain.hip);
//   * per item (k_scan_bwd_rc_item): one workgroup per (segment, channel)
//     item looping over the chunks the segment touches in B order (edges
//     masked per element), the carry in registers; it runs for every other
//     geometry, and before the chained walk for the unaligned segments
//     (clearing the chained walk's slots first).
//
// Reference semantics: the same fused backward as _kernels.py:171-287 (the
// states the reference saves in scan_eager.py:42-47 are recomputed instead
// of read).

#include "chain_common.h"

namespace asc {
namespace {

struct RcPtrs {
  const char* dy;  // dense gradient, or one value per row (DYC)
  const char* g;
  const char* x;   // the forward's tokens (its input)
  char* dx;
  char* dg;
  const float* ckpt;  // C * kr forward carries (asc_scan_checkpoints)
};

struct RcParams {
  ChainGeo geo;          // kr = chunks per row (rounded up)
  RcPtrs t;
  int64_t dy_rs;         // DYC: element stride between rows of dy
  LbSlot* slots;         // chained walk
  // per-item walk before the chained walk: Geometry::chain_*
  int64_t chain_ch;
  unsigned long long* chain_slots;
  int64_t chain_words;
  uint32_t* chain_flag;
};

__device__ inline float lane_mirror(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(
      (kWave - 1 - lane) << 2, __float_as_int(v)));
}

// Scan of affine maps over the lanes in descending lane order (lane 63
// first): the exclusive prefix of the lane and the total of all 64.
__device__ inline SubScan wave_scan_affine_desc(float a, float x, int lane) {
  a = lane_mirror(a, lane);
  x = lane_mirror(x, lane);
  wave_scan_affine(a, x);
  SubScan r;
  r.ta = readlane(a, kWave - 1);
  r.tx = readlane(x, kWave - 1);
  r.ea = lane_mirror(dpp<kWaveShr1, 0xf>(1.0f, a), lane);
  r.ex = lane_mirror(dpp<kWaveShr1, 0xf>(0.0f, x), lane);
  return r;
}

// Loads vector vi of `base`; EDGE: elements outside [P0, P1) read `ident`
// (a vector that lies wholly outside is not read: the last chunk of the
// last row may reach past the tensor).
template <class IO, bool EDGE>
__device__ inline uint4 rc_load(const char* base, int64_t vi, int64_t P0,
                                int64_t P1, float ident) {
  constexpr int V = IO::V;
  const int64_t pv = vi * V;
  if (!EDGE || (pv >= P0 && pv + V <= P1)) return ld16(base + vi * 16);
  float f[V];
  if (pv + V <= P0 || pv >= P1) {
#pragma unroll
    for (int j = 0; j < V; ++j) f[j] = ident;
  } else {
    IO::unpack(ld16(base + vi * 16), f);
#pragma unroll
    for (int j = 0; j < V; ++j)
      if (pv + j < P0 || pv + j >= P1) f[j] = ident;
  }
  return IO::pack(f);
}

// Per-chunk registers of one wave (kChainU sub-tiles).
template <class IO>
struct RcWave {
  uint4 yq[kChainU], gq[kChainU], xq[kChainU], hq[kChainU];
  int64_t vi[kChainU];
  SubScan sf[kChainU];  // forward: lane prefix (forward lane order), total
  SubScan sb[kChainU];  // adjoint (B order)
  float gprv[kChainU];
  float fa, fx;         // the wave's forward map (forward order)
  float ba, bx;         // the wave's adjoint map (B order)
};

// Vector of (wave wv, sub-tile u, lane) in a chunk that starts at element
// e0 (memory order), B order.
template <int V, bool RB>
__device__ inline int64_t rc_vec(int64_t e0, int64_t CH, int wv, int u,
                                 int lane) {
  const int64_t i = static_cast<int64_t>(wv * kChainU + u) * kWave + lane;
  return RB ? (e0 + CH) / V - 1 - i : e0 / V + i;
}

// Phase 1a: the wave's loads (EDGE: masked to [P0, P1), else whole
// vectors, which need no segment lookup and are issued before it).
template <class IO, bool RB, bool DYC, bool EDGE>
__device__ inline void rc_load_chunk(const RcPtrs& t, int64_t e0, int64_t P0,
                                     int64_t P1, int wv, int lane,
                                     RcWave<IO>& s) {
  constexpr int V = IO::V;
  constexpr int64_t CH = chain_elems(V);
#pragma unroll
  for (int u = 0; u < kChainU; ++u) {
    s.vi[u] = rc_vec<V, RB>(e0, CH, wv, u, lane);
    if (!DYC) s.yq[u] = rc_load<IO, EDGE>(t.dy, s.vi[u], P0, P1, 0.0f);
    s.gq[u] = rc_load<IO, EDGE>(t.g, s.vi[u], P0, P1, 1.0f);
    s.xq[u] = rc_load<IO, EDGE>(t.x, s.vi[u], P0, P1, 0.0f);
  }
}

// Phase 1b: both local scans.  [P0, P1): the segment's elements; bhead /
// btail: its first / last element in B order (the forward's head is btail);
// mk(u): whether sub-tile u may hold either (per-element tests).
template <class IO, bool RB, bool DYC, bool EDGE, class Mk>
__device__ inline void rc_phase1(const RcPtrs& t, int64_t P0, int64_t P1,
                                 int64_t bhead, int64_t btail, float dyv,
                                 int lane, Mk mk, RcWave<IO>& s) {
  constexpr int V = IO::V;
  constexpr int U = kChainU;
  constexpr int jl = mem_idx<V, RB>(V - 1);
  constexpr int jf = mem_idx<V, RB>(0);
  // the gate just before the wave's first element in B order (the pad 1
  // outside the segment)
  const int64_t pf = s.vi[0] * V + jf;
  const int64_t pg = RB ? pf + 1 : pf - 1;
  float cg = (pg >= P0 && pg < P1) ? IO::load1(t.g + pg * IO::ES) : 1.0f;
  s.ba = 1.0f;
  s.bx = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float g[V], x[V], y[V];
    IO::unpack(s.gq[u], g);
    IO::unpack(s.xq[u], x);
    const int64_t pv = s.vi[u] * V;
    if (DYC) {
#pragma unroll
      for (int j = 0; j < V; ++j)
        y[j] = (!EDGE || (pv + j >= P0 && pv + j < P1)) ? dyv : 0.0f;
    } else {
      IO::unpack(s.yq[u], y);
    }
    // forward recurrence, forward order inside the lane
    const bool m = EDGE || mk(u);
    float A = 1.0f, X = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int j = mem_idx<V, !RB>(i);
      if (m && pv + j == btail) {
        A = 0.0f;
        X = x[j];
      } else {
        X = fmaf(g[j], X, x[j]);
        A = A * g[j];
      }
    }
    s.sf[u] = wave_scan_affine_desc(A, X, lane);
    // adjoint, B order
    if (m)
      s.sb[u] = bwd_local<IO, RB, true>(g, y, pv, bhead, cg, s.gprv[u]);
    else
      s.sb[u] = bwd_local<IO, RB, false>(g, y, pv, 0, cg, s.gprv[u]);
    cg = readlane(g[jl], kWave - 1);
    s.bx = fmaf(s.sb[u].ta, s.bx, s.sb[u].tx);
    s.ba = s.ba * s.sb[u].ta;
  }
  s.fa = 1.0f;
  s.fx = 0.0f;
#pragma unroll
  for (int u = U - 1; u >= 0; --u) {
    s.fx = fmaf(s.sf[u].ta, s.fx, s.sf[u].tx);
    s.fa = s.fa * s.sf[u].ta;
  }
}

// Phase 2: the states from the wave's forward carry cf (rounded to the
// storage type, kept packed); returns the state of the wave's first element
// in B order.
template <class IO, bool RB, bool EDGE, class Mk>
__device__ inline float rc_phase2(int64_t btail, float cf, Mk mk,
                                  RcWave<IO>& s) {
  constexpr int V = IO::V;
  constexpr int U = kChainU;
  constexpr int jf = mem_idx<V, RB>(0);
#pragma unroll
  for (int u = U - 1; u >= 0; --u) {
    float g[V], x[V], h[V];
    repack_point<IO>(s.gq[u]);
    repack_point<IO>(s.xq[u]);
    IO::unpack(s.gq[u], g);
    IO::unpack(s.xq[u], x);
    const int64_t pv = s.vi[u] * V;
    if (EDGE || mk(u))
      fwd_apply<IO, !RB, true>(g, x, pv, btail, s.sf[u], cf, h);
    else
      fwd_apply<IO, !RB, false>(g, x, pv, 0, s.sf[u], cf, h);
    s.hq[u] = IO::pack(h);
    cf = fmaf(s.sf[u].ta, cf, s.sf[u].tx);
  }
  float h0[V];
  IO::unpack(s.hq[0], h0);
  return readlane(h0[jf], 0);
}

// Phase 3: dx, dg from the wave's backward carry c and the state just past
// its last element in B order (hlast).
template <class IO, bool RB, bool DYC, bool EDGE, class Mk>
__device__ inline void rc_phase3(const RcPtrs& t, int64_t P0, int64_t P1,
                                 int64_t bhead, int64_t btail, float dyv,
                                 float c, float hlast, Mk mk, RcWave<IO>& s) {
  constexpr int V = IO::V;
  constexpr int U = kChainU;
  constexpr int jf = mem_idx<V, RB>(0);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float g[V], y[V], h[V], dx[V], dg[V];
    repack_point<IO>(s.gq[u]);
    IO::unpack(s.gq[u], g);
    IO::unpack(s.hq[u], h);
    const int64_t pv = s.vi[u] * V;
    if (DYC) {
#pragma unroll
      for (int j = 0; j < V; ++j)
        y[j] = (!EDGE || (pv + j >= P0 && pv + j < P1)) ? dyv : 0.0f;
    } else {
      repack_point<IO>(s.yq[u]);
      IO::unpack(s.yq[u], y);
    }
    float hin = hlast;
    if (u + 1 < U) {
      float hn[V];
      IO::unpack(s.hq[u + 1 < U ? u + 1 : u], hn);
      hin = readlane(hn[jf], 0);
    }
    if (EDGE || mk(u))
      bwd_apply<IO, RB, true>(g, y, h, pv, bhead, btail, s.gprv[u], hin,
                              s.sb[u], c, dx, dg);
    else
      bwd_apply<IO, RB, false>(g, y, h, pv, 0, 0, s.gprv[u], hin, s.sb[u], c,
                               dx, dg);
    if (EDGE) {
      store_vec<IO, true, true>(t.dx, s.vi[u], true, P0, P1, dx);
      store_vec<IO, true, true>(t.dg, s.vi[u], true, P0, P1, dg);
    } else {
      st16(t.dx + s.vi[u] * 16, IO::pack(dx));
      st16(t.dg + s.vi[u] * 16, IO::pack(dg));
    }
    c = fmaf(s.sb[u].ta, c, s.sb[u].tx);
  }
}

struct RcLds {
  float2 fagg[kChainWaves];  // wave forward maps
  float2 bagg[kChainWaves];  // wave adjoint maps
  float hb[kChainWaves];     // state of each wave's first element (B order)
  float carry;               // chained walk: the chunk's backward carry
};

// ---- chained walk: one chunk per workgroup ----
template <class IO, bool RB, bool DYC>
__device__ inline void rc_chain_chunk(const RcParams& p, int64_t b, int lane,
                                      int wv, RcLds& L) {
  constexpr int V = IO::V;
  constexpr int64_t CH = chain_elems(V);
  ChainChunk k;
  // read the chunk before its segment is looked up when every segment is
  // chunk-aligned (chain_survey_of)
  const uint32_t sv = chain_survey_of(p.geo);
  if (sv == kChainNone) return;
  const bool all = sv == kChainAll;
  if (!all && !chain_chunk<CH>(p.geo, b, RB, k)) return;
  k.row = b / p.geo.kr;
  {
    const int64_t rr = b - k.row * p.geo.kr;
    k.e0 = k.row * p.geo.T + (RB ? p.geo.kr - 1 - rr : rr) * CH;
  }
  const float dyv =
      DYC ? IO::load1(p.t.dy + k.row * p.dy_rs * IO::ES) : 0.0f;
  RcWave<IO> s;
  rc_load_chunk<IO, RB, DYC, false>(p.t, k.e0, 0, 0, wv, lane, s);
  if (all && !chain_chunk<CH>(p.geo, b, RB, k)) return;  // outside all
  const int64_t bhead = RB ? k.P1 - 1 : k.P0;
  const int64_t btail = RB ? k.P0 : k.P1 - 1;
  const bool tail_chunk = RB ? k.first_mem : k.last_mem;
  auto mk = [&](int u) {
    return (u == 0 && wv == 0 && k.j == 0) ||
           (tail_chunk && u == kChainU - 1 && wv == kChainWaves - 1);
  };
  rc_phase1<IO, RB, DYC, false>(p.t, k.P0, k.P1, bhead, btail, dyv, lane, mk,
                                s);
  if (lane == 0) {
    L.fagg[wv] = make_float2(s.fa, s.fx);
    L.bagg[wv] = make_float2(s.ba, s.bx);
  }
  __syncthreads();
  // the forward carry into the chunk: its checkpoint (0 when the chunk holds
  // the segment's head)
  const float cfk = tail_chunk ? 0.0f : p.t.ckpt[k.row * p.geo.kr + k.t0 / CH];
  float A = 1.0f, X = 0.0f;
  if (wv == 0) {
#pragma unroll
    for (int w = 0; w < kChainWaves; ++w) {
      X = fmaf(L.bagg[w].x, X, L.bagg[w].y);
      A = A * L.bagg[w].x;
    }
    if (lane == 0) chain_publish(p.slots + b, k.j, A, X);
  }
  float cf = cfk;
  for (int w = kChainWaves - 1; w > wv; --w) cf = fmaf(L.fagg[w].x, cf, L.fagg[w].y);
  const float hf0 = rc_phase2<IO, RB, false>(btail, cf, mk, s);
  if (lane == 0) L.hb[wv] = hf0;
  if (wv == 0) {
    float carry = 0.0f;
    if (k.j > 0) {
      BwdPtrs q{};
      q.dy = p.t.dy;
      q.g = p.t.g;
      carry = chain_carry(p.slots, b, k.j, lane, p.geo.spin, [&]() {
        return chain_prefix_bwd<IO, RB, DYC>(q, k, lane, dyv);
      });
    }
    if (lane == 0) {
      L.carry = carry;
      if (k.j % kChainBlock == kChainBlock - 1)
        lb_put(&p.slots[b].x, kLbIncl, fmaf(A, carry, X));
    }
  }
  __syncthreads();
  float c = L.carry;
  for (int w = 0; w < wv; ++w) c = fmaf(L.bagg[w].x, c, L.bagg[w].y);
  const float hlast = wv + 1 < kChainWaves ? L.hb[wv + 1] : cfk;
  rc_phase3<IO, RB, DYC, false>(p.t, k.P0, k.P1, bhead, btail, dyv, c, hlast,
                                mk, s);
}

// DIRS: 1 = backward of a causal forward scan, 2 = of a reverse one.
template <class IO, int DIRS, bool DYC>
__global__ void __launch_bounds__(kChainWaves* kWave)
    k_scan_bwd_rc_chain(RcParams p) {
  __shared__ RcLds L;
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  rc_chain_chunk<IO, DIRS == 1, DYC>(p, blockIdx.x, lane, wv, L);
}

// ---- per-item walk: one workgroup per (segment, channel) item ----
template <class IO, bool RB, bool DYC>
__device__ inline void rc_item(const RcParams& p, int64_t P0, int64_t P1,
                               int64_t row, int lane, int wv, RcLds& L) {
  constexpr int V = IO::V;
  constexpr int64_t CH = chain_elems(V);
  const int64_t base = row * p.geo.T;  // phase 0: element index = position
  const float dyv = DYC ? IO::load1(p.t.dy + row * p.dy_rs * IO::ES) : 0.0f;
  const int64_t bhead = RB ? P1 - 1 : P0;
  const int64_t btail = RB ? P0 : P1 - 1;
  const int64_t k_lo = (P0 - base) / CH, k_hi = (P1 - 1 - base) / CH;
  const int64_t nk = k_hi - k_lo + 1;
  auto none = [](int) { return false; };
  float carry = 0.0f;  // backward carry into the chunk (B order)
  for (int64_t n = 0; n < nk; ++n) {
    const int64_t kc = RB ? k_hi - n : k_lo + n;
    const int64_t e0 = base + kc * CH;
    const bool edge = e0 < P0 || e0 + CH > P1;
    const bool has_fhead = RB ? kc == k_lo : kc == k_hi;
    const float cfk = has_fhead ? 0.0f : p.t.ckpt[row * p.geo.kr + kc];
    RcWave<IO> s;
    if (edge) {
      rc_load_chunk<IO, RB, DYC, true>(p.t, e0, P0, P1, wv, lane, s);
      rc_phase1<IO, RB, DYC, true>(p.t, P0, P1, bhead, btail, dyv, lane, none,
                                   s);
    } else {
      rc_load_chunk<IO, RB, DYC, false>(p.t, e0, P0, P1, wv, lane, s);
      rc_phase1<IO, RB, DYC, false>(p.t, P0, P1, bhead, btail, dyv, lane,
                                    none, s);
    }
    if (lane == 0) {
      L.fagg[wv] = make_float2(s.fa, s.fx);
      L.bagg[wv] = make_float2(s.ba, s.bx);
    }
    __syncthreads();
    float cf = cfk;
    for (int w = kChainWaves - 1; w > wv; --w)
      cf = fmaf(L.fagg[w].x, cf, L.fagg[w].y);
    const float hf0 = edge ? rc_phase2<IO, RB, true>(btail, cf, none, s)
                           : rc_phase2<IO, RB, false>(btail, cf, none, s);
    if (lane == 0) L.hb[wv] = hf0;
    // every wave composes the same carries in the same order
    float c = carry;
    for (int w = 0; w < wv; ++w) c = fmaf(L.bagg[w].x, c, L.bagg[w].y);
#pragma unroll
    for (int w = 0; w < kChainWaves; ++w)
      carry = fmaf(L.bagg[w].x, carry, L.bagg[w].y);
    __syncthreads();
    const float hlast = wv + 1 < kChainWaves ? L.hb[wv + 1] : cfk;
    if (edge)
      rc_phase3<IO, RB, DYC, true>(p.t, P0, P1, bhead, btail, dyv, c, hlast,
                                   none, s);
    else
      rc_phase3<IO, RB, DYC, false>(p.t, P0, P1, bhead, btail, dyv, c, hlast,
                                    none, s);
  }
}

template <class IO, int DIRS, bool DYC>
__global__ void __launch_bounds__(kChainWaves* kWave)
    k_scan_bwd_rc_item(RcParams p) {
  __shared__ RcLds L;
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  Geometry geo{p.geo.cu,    p.geo.cu64,    p.geo.S,       p.geo.C,
               p.geo.T,     p.geo.S * p.geo.C, 1,         0,
               p.chain_ch,  p.chain_slots, p.chain_words, p.chain_flag};
  // the same value in every wave of the workgroup: all return together
  if (geo.chain_ch > 0 &&
      chain_prologue(geo, static_cast<int64_t>(blockIdx.x) * kChainWaves + wv,
                     static_cast<int64_t>(gridDim.x) * kChainWaves, lane))
    return;
  for (int64_t w = blockIdx.x; w < geo.items; w += gridDim.x) {
    int br;
    int64_t P0, P1, row;
    if (!item_range<true>(geo, w, br, P0, P1, row, true)) continue;
    rc_item<IO, DIRS == 1, DYC>(p, P0, P1, row, lane, wv, L);
  }
}

// ---- checkpoints: the forward state before each chunk ----
// ckpt[c * kr + k] = the state adjacent to chunk k of row c on the side the
// forward scan comes from (causal: element k*CH - 1; reverse: the element
// after the chunk), if that element lies in the same segment as the chunk's
// first element in forward order; 0 otherwise.
template <class IO>
__global__ void __launch_bounds__(256)
    k_scan_ckpt(const char* h, float* ckpt, const void* cu, int cu64,
                int64_t S, int64_t C, int64_t T, int64_t kr, int64_t CH,
                int rev) {
  const int64_t n = C * kr;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  auto cu_at = [&](int64_t i) -> int64_t {
    int64_t v = cu64 ? reinterpret_cast<const int64_t*>(cu)[i]
                     : static_cast<int64_t>(reinterpret_cast<const int32_t*>(cu)[i]);
    return v < 0 ? 0 : (v > T ? T : v);
  };
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += stride) {
    const int64_t c = i / kr, k = i - c * kr;
    const int64_t tf = rev ? ((k + 1) * CH < T ? (k + 1) * CH : T) - 1 : k * CH;
    const int64_t tp = rev ? tf + 1 : tf - 1;
    float v = 0.0f;
    if (tp >= 0 && tp < T) {
      // segment of tf: the last s with cu[s] <= tf
      int64_t lo = 0, hi = S + 1;
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (cu_at(mid) <= tf) lo = mid + 1;
        else hi = mid;
      }
      const int64_t s = lo - 1;
      if (s >= 0 && s < S) {
        const int64_t s0 = cu_at(s), s1 = cu_at(s + 1);
        if (tf < s1 && tp >= s0 && tp < s1)
          v = IO::load1(h + (c * T + tp) * IO::ES);
      }
    }
    ckpt[i] = v;
  }
}

template <class IO, bool DYC>
const void* pick_rc_chain(bool causal) {
  return causal ? reinterpret_cast<const void*>(&k_scan_bwd_rc_chain<IO, 1, DYC>)
                : reinterpret_cast<const void*>(&k_scan_bwd_rc_chain<IO, 2, DYC>);
}
template <class IO, bool DYC>
const void* pick_rc_item(bool causal) {
  return causal ? reinterpret_cast<const void*>(&k_scan_bwd_rc_item<IO, 1, DYC>)
                : reinterpret_cast<const void*>(&k_scan_bwd_rc_item<IO, 2, DYC>);
}
template <bool DYC>
const void* pick_rc(int dtype, bool causal, bool chain) {
  switch (dtype) {
    case ASC_F32:
      return chain ? pick_rc_chain<IoF32, DYC>(causal) : pick_rc_item<IoF32, DYC>(causal);
    case ASC_F16:
      return chain ? pick_rc_chain<IoF16, DYC>(causal) : pick_rc_item<IoF16, DYC>(causal);
    default:
      return chain ? pick_rc_chain<IoBF16, DYC>(causal) : pick_rc_item<IoBF16, DYC>(causal);
  }
}

}  // namespace

int64_t rc_chunks_per_row(int64_t T, int v) {
  const int64_t CH = chain_elems(v);
  return (T + CH - 1) / CH;
}

int rc_checkpoints(const void* h, float* ckpt, const void* cu, int cu_dtype,
                   int64_t S, int64_t C, int64_t T, int dtype, int reverse,
                   void* stream) {
  const int v = 16 / elem_size(dtype);
  int64_t kr = rc_chunks_per_row(T, v);
  const int64_t n = C * kr;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  const char* hp = static_cast<const char*>(h);
  int cu64 = cu_dtype == ASC_CU_I64;
  int64_t CH = chain_elems(v);
  int rev = reverse ? 1 : 0;
  const void* cup = cu;
  void* args[] = {&hp, &ckpt, &cup, &cu64, &S, &C, &T, &kr, &CH, &rev};
  const void* fn = dtype == ASC_F32 ? reinterpret_cast<const void*>(&k_scan_ckpt<IoF32>)
                   : dtype == ASC_F16 ? reinterpret_cast<const void*>(&k_scan_ckpt<IoF16>)
                                      : reinterpret_cast<const void*>(&k_scan_ckpt<IoBF16>);
  const hipError_t e = hipLaunchKernel(fn, dim3(static_cast<unsigned>(blocks)),
                                       dim3(256), args, 0,
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ASC_OK : static_cast<int>(e);
}

int rc_bwd(const RcArgs& a, void* stream) {
  const int v = 16 / elem_size(a.dtype);
  RcParams p{};
  Geometry g{a.cu, a.cu64, a.S, a.C, a.T, a.S * a.C, 1, 0};
  p.t = RcPtrs{static_cast<const char*>(a.dy), static_cast<const char*>(a.g),
               static_cast<const char*>(a.x), static_cast<char*>(a.dx),
               static_cast<char*>(a.dg), a.ckpt};
  p.dy_rs = a.dy_rs;
  const bool dyc = a.dy_rs >= 0;
  // the per-item walk first (for chained calls it clears the slots and
  // takes the unaligned segments), then the chained walk for chunk-aligned
  // long segments
  const bool chained =
      !a.inplace && chain_share(g, true, v, a.ws, a.ws_bytes, true);
  p.geo = chain_geo(g, v);
  p.slots = reinterpret_cast<LbSlot*>(g.chain_slots);
  p.chain_ch = g.chain_ch;
  p.chain_slots = g.chain_slots;
  p.chain_words = g.chain_words;
  p.chain_flag = g.chain_flag;
  RcParams pi = p;
  pi.geo.kr = rc_chunks_per_row(a.T, v);
  pi.geo.nchunks = a.C * pi.geo.kr;
  // before the chained walk the grid is capped at 8 workgroups per CU
  // (grid-stride loops take the rest): where every segment is aligned each
  // workgroup looks at cu_seqlens once and returns, 2-3 resident at a time
  // per CU (an uncapped grid of 12288 cost 30-50 us at cfg5)
  constexpr int64_t kRcPartnerBlocks = 2048;
  int64_t blocks = a.S * a.C;
  if (chained && blocks > kRcPartnerBlocks) blocks = kRcPartnerBlocks;
  const void* fn = dyc ? pick_rc<true>(a.dtype, a.causal, false)
                       : pick_rc<false>(a.dtype, a.causal, false);
  int st = launch(fn, blocks, kChainWaves, pi, stream);
  if (st || !chained) return st;
  fn = dyc ? pick_rc<true>(a.dtype, a.causal, true)
           : pick_rc<false>(a.dtype, a.causal, true);
  return launch(fn, p.geo.nchunks, kChainWaves, p, stream);
}

}  // namespace asc
