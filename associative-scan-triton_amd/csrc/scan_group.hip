// Several items per wave for short segments: each group of G lanes of a
// wave (G = 32: two items per wave, G = 16: four) walks one (segment,
// channel) item, G * L vectors per step (L consecutive vectors per lane).
// A launch of short items is bound by how fast waves start (about 2000 per
// us on MI355X, 12288 one-wave items of 128 fp32 elements: the last of them
// starts after 6 us, each lives 2-3 us); grouping divides the waves by 64/G
// for the same instructions per item, since the groups scan in one pass:
// the DPP scan stops before the first step that crosses a group
// (row_bcast:31 for halves, row_bcast:15 for rows of 16), and the three
// lane shifts that cross a group edge (the exclusive prefix, the shifted
// gate, the shifted state) take the group's own value there instead.
// Every element is tested against its item's edges (both edges of a short
// item usually fall in one step).

#include "asc_common.h"

namespace asc {
namespace {

// Inclusive affine scan within each row of 16 lanes.
__device__ inline void row_scan_affine(float& a, float& x) {
  if (ASC_DPP_ASM) {
    asm("s_nop 1\n\t" ASC_AFFINE(ASC_DPP_SHR(1)) "s_nop 0\n\t"
            ASC_AFFINE(ASC_DPP_SHR(2)) "s_nop 0\n\t" ASC_AFFINE(ASC_DPP_SHR(4))
                "s_nop 0\n\t" ASC_AFFINE(ASC_DPP_SHR(8)) "s_nop 1"
        : "+v"(a), "+v"(x));
    return;
  }
  affine_step<kRowShr1, 0xf>(a, x);
  affine_step<kRowShr2, 0xf>(a, x);
  affine_step<kRowShr4, 0xf>(a, x);
  affine_step<kRowShr8, 0xf>(a, x);
}

template <int G>
__device__ inline void group_scan_affine(float& a, float& x) {
  if (G == 32)
    half_scan_affine(a, x);
  else
    row_scan_affine(a, x);
}

// The group's value at its last lane (lane q*G + G-1 for group q).
template <int G>
__device__ inline float group_last(float v, int q) {
  if (G == 32) {
    const float lo = readlane(v, 31), hi = readlane(v, 63);
    return q ? hi : lo;
  }
  const float v0 = readlane(v, 15), v1 = readlane(v, 31),
              v2 = readlane(v, 47), v3 = readlane(v, 63);
  return q < 2 ? (q ? v1 : v0) : (q == 3 ? v3 : v2);
}

// The lane's start value from its group's carry (carried_start within each
// group: lane 0 of a group takes the carry, not the previous group's last
// lane) and the group's carry out.
template <int G>
__device__ inline float group_carried_start(float A, float X, int hl, int q,
                                            float& carry) {
  group_scan_affine<G>(A, X);
  const float y = fmaf(A, carry, X);
  float start = dpp<kWaveShr1, 0xf>(carry, y);
  if (hl == 0) start = carry;
  carry = group_last<G>(y, q);
  return start;
}

// Vectors of a group's item in scan order: vector i is v0 + i (forward) or
// v1 - i (reverse).
struct GroupItem {
  int64_t P0, P1;  // element range (empty: P0 = P1 = 0)
  int64_t v0, v1, nv;
  __device__ inline GroupItem(int64_t p0, int64_t p1, int V) : P0(p0), P1(p1) {
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

// Steps of the longest item of the wave's groups (uniform).
template <int G>
__device__ inline int64_t group_steps(const GroupItem& it, int per_step) {
  const int n = static_cast<int>((it.nv + per_step - 1) / per_step);
  int m = __builtin_amdgcn_readlane(n, 0);
#pragma unroll
  for (int q = 1; q < kWave / G; ++q) {
    const int nq = __builtin_amdgcn_readlane(n, q * G);
    m = nq > m ? nq : m;
  }
  return m;
}

// L: vectors per lane and step, consecutive in scan order; the lane's
// elements in scan order are those of its vectors m = 0 .. L-1 in turn.
// The launches use L = 1 (rows of 16 lanes with two vectors each lost to
// halves with one; see group_lanes).  Written for any L, the loops over m
// also gave the fastest code for L = 1 (ragged 1-250-element fp32 segments,
// backward: 58 us against 68 for the same steps written without them).
template <class IO, bool REV, int G, int L>
__device__ inline void group_fwd(const FwdPtrs& t, const GroupItem& it, int hl,
                                 int q) {
  constexpr int V = IO::V;
  const int64_t nmax = group_steps<G>(it, G * L);
  const int64_t head = REV ? it.P1 - 1 : it.P0;
  float carry = 0.0f;
  for (int64_t k = 0; k < nmax; ++k) {
    float g[L][V], x[L][V];
    int64_t vi[L];
    bool ok[L];
#pragma unroll
    for (int m = 0; m < L; ++m) {
      const int64_t i = (k * G + hl) * L + m;
      ok[m] = i < it.nv;
      vi[m] = REV ? it.v1 - i : it.v0 + i;
      const char* const src[2] = {t.g, t.x};
      const float ident[2] = {1.0f, 0.0f};
      float gx[2][V];
      load_vecs<IO, 2>(src, vi[m], ok[m], it.P0, it.P1, ident, gx, t.pend);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        g[m][e] = gx[0][e];
        x[m][e] = gx[1][e];
      }
    }
    float A = 1.0f, X = 0.0f;
#pragma unroll
    for (int m = 0; m < L; ++m) {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const int j = mem_idx<V, REV>(e);
        if (vi[m] * V + j == head) {
          A = 0.0f;
          X = x[m][j];
        } else {
          X = fmaf(g[m][j], X, x[m][j]);
          A = A * g[m][j];
        }
      }
    }
    float hh = group_carried_start<G>(A, X, hl, q, carry);
#pragma unroll
    for (int m = 0; m < L; ++m) {
      float h[V];
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const int j = mem_idx<V, REV>(e);
        hh = vi[m] * V + j == head ? x[m][j] : fmaf(g[m][j], hh, x[m][j]);
        h[j] = hh;
      }
      store_vec<IO, true, true>(t.h, vi[m], ok[m], it.P0, it.P1, h);
    }
  }
}

// RB: B order (the adjoint's scan order) is reverse memory order.
template <class IO, bool RB, bool DYC, int G, int L>
__device__ inline void group_bwd(const BwdPtrs& t, const GroupItem& it, int hl,
                                 int q, float dyv) {
  constexpr int V = IO::V;
  constexpr int jl = mem_idx<V, RB>(V - 1);  // last element in B order
  constexpr int jf = mem_idx<V, RB>(0);      // first element in B order
  const int64_t nmax = group_steps<G>(it, G * L);
  const int64_t head = RB ? it.P1 - 1 : it.P0;
  const int64_t tail = RB ? it.P0 : it.P1 - 1;
  float carry = 0.0f, carry_g = 1.0f;
  for (int64_t k = 0; k < nmax; ++k) {
    float g[L][V], dy[L][V], h[L][V];
    int64_t vi[L];
    bool ok[L];
#pragma unroll
    for (int m = 0; m < L; ++m) {
      const int64_t i = (k * G + hl) * L + m;
      ok[m] = i < it.nv;
      vi[m] = RB ? it.v1 - i : it.v0 + i;
      if (DYC) {
        const char* const src[2] = {t.g, t.h};
        const float ident[2] = {1.0f, 0.0f};
        float gh[2][V];
        load_vecs<IO, 2>(src, vi[m], ok[m], it.P0, it.P1, ident, gh, t.pend);
#pragma unroll
        for (int e = 0; e < V; ++e) {
          g[m][e] = gh[0][e];
          h[m][e] = gh[1][e];
        }
      } else {
        const char* const src[3] = {t.dy, t.g, t.h};
        const float ident[3] = {0.0f, 1.0f, 0.0f};
        float ygh[3][V];
        load_vecs<IO, 3>(src, vi[m], ok[m], it.P0, it.P1, ident, ygh, t.pend);
#pragma unroll
        for (int e = 0; e < V; ++e) {
          dy[m][e] = ygh[0][e];
          g[m][e] = ygh[1][e];
          h[m][e] = ygh[2][e];
        }
      }
    }
    // (DYC: the row value fills dy after the loads are issued, so that its
    // own load does not hold them back)
    if (DYC) {
#pragma unroll
      for (int m = 0; m < L; ++m)
        dyc_vec<IO, true>(dyv, vi[m], ok[m], it.P0, it.P1, dy[m]);
    }
    // the state just past this step in B order (0 past the item)
    const int64_t il = (k * G + G) * L - 1;
    const int64_t vl = RB ? it.v1 - il : it.v0 + il;
    const int64_t pn = RB ? vl * V - 1 : vl * V + V;
    const float halo =
        (pn >= it.P0 && pn < it.P1) ? IO::load1(t.h + pn * IO::ES) : 0.0f;
    // first phase: shifted gates (lane 0 of each group takes its group's
    // carry_g), the adjoint's maps
    float gprev = dpp<kWaveShr1, 0xf>(carry_g, g[L - 1][jl]);
    if (hl == 0) gprev = carry_g;
    auto gate_before = [&](int m, int e) -> float {
      if (e > 0) return g[m][mem_idx<V, RB>(e - 1)];
      return m > 0 ? g[m > 0 ? m - 1 : 0][jl] : gprev;
    };
    float A = 1.0f, X = 0.0f;
#pragma unroll
    for (int m = 0; m < L; ++m) {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const int j = mem_idx<V, RB>(e);
        const float gs = gate_before(m, e);
        if (vi[m] * V + j == head) {
          A = 0.0f;
          X = dy[m][j];
        } else {
          X = fmaf(gs, X, dy[m][j]);
          A = A * gs;
        }
      }
    }
    float d = group_carried_start<G>(A, X, hl, q, carry);
    // second phase: dx, and dg from the shifted state (the last lane of
    // each group takes its group's halo)
    float hnx = dpp<kWaveShl1, 0xf>(halo, h[0][jf]);
    if (hl == G - 1) hnx = halo;
#pragma unroll
    for (int m = 0; m < L; ++m) {
      float dx[V], dg[V];
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const int j = mem_idx<V, RB>(e);
        const float gs = gate_before(m, e);
        d = vi[m] * V + j == head ? dy[m][j] : fmaf(gs, d, dy[m][j]);
        float hn = e + 1 < V ? h[m][mem_idx<V, RB>(e + 1)]
                             : (m + 1 < L ? h[m + 1 < L ? m + 1 : m][jf] : hnx);
        if (vi[m] * V + j == tail) hn = 0.0f;
        dx[j] = d;
        dg[j] = hn * d;
      }
      store_vec<IO, true, true>(t.dx, vi[m], ok[m], it.P0, it.P1, dx);
      store_vec<IO, true, true>(t.dg, vi[m], ok[m], it.P0, it.P1, dg);
    }
    carry_g = group_last<G>(g[L - 1][jl], q);
  }
}

// Group w of a branch: items K*w .. K*w + K-1 of that branch (K = 64/G;
// the last ones may not exist).  All are decoded before any cu_seqlens
// value is read, and an item of the same segment as the one before reuses
// its values (the item order puts neighbouring channels of one segment
// side by side), so the wave usually waits on one round of scalar loads.
// Returns the lane's group's item range (empty: P0 = P1 = 0) and row.
template <int G>
__device__ inline void group_items(const Geometry& geo, int64_t w, int& br,
                                   int q, int64_t& P0, int64_t& P1,
                                   int64_t& row) {
  constexpr int K = kWave / G;
  const int64_t gpb = (geo.items + K - 1) / K;  // groups per branch
  br = w >= gpb ? 1 : 0;
  const int64_t loc = w - br * gpb;
  int64_t s[K], c[K];
  bool has[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    has[j] = K * loc + j < geo.items;
    s[j] = 0;
    c[j] = 0;
    if (has[j]) item_seg_chan(geo, K * loc + j, true, s[j], c[j]);
  }
  int64_t t0[K], t1[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    if (j > 0 && s[j] == s[j - 1]) {
      t0[j] = t0[j > 0 ? j - 1 : 0];
      t1[j] = t1[j > 0 ? j - 1 : 0];
    } else {
      cu_edges(geo, s[j], t0[j], t1[j]);
    }
  }
  P0 = 0;
  P1 = 0;
  row = 0;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const int64_t a = t0[j] < 0 ? 0 : (t0[j] > geo.T ? geo.T : t0[j]);
    const int64_t b = t1[j] < a ? a : (t1[j] > geo.T ? geo.T : t1[j]);
    const int64_t base = c[j] * geo.T + geo.phase;
    const bool live = has[j] && b > a;
    if (q == j) {
      P0 = live ? base + a : 0;
      P1 = live ? base + b : 0;
      row = c[j];
    }
  }
}

template <class IO, int DIRS, int G, int L>
__global__ void __launch_bounds__(kWave) k_scan_fwd_group(FwdParams p) {
  if (skipped(p)) return;
  constexpr int K = kWave / G;
  const int lane = threadIdx.x;
  const int hl = lane & (G - 1);
  const int q = lane / G;
  const int64_t W = (p.geo.items + K - 1) / K * p.geo.nbranch;
  for (int64_t w = blockIdx.x; w < W; w += gridDim.x) {
    int br;
    int64_t P0, P1, row;
    group_items<G>(p.geo, w, br, q, P0, P1, row);
    const GroupItem it(P0, P1, IO::V);
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      group_fwd<IO, false, G, L>(p.br[br], it, hl, q);
    else
      group_fwd<IO, true, G, L>(p.br[br], it, hl, q);
  }
}

// DIRS: the forward scan's direction, as for the other backward kernels.
template <class IO, int DIRS, bool DYC, int G, int L>
__global__ void __launch_bounds__(kWave) k_scan_bwd_group(BwdParams p) {
  if (skipped(p)) return;
  constexpr int K = kWave / G;
  const int lane = threadIdx.x;
  const int hl = lane & (G - 1);
  const int q = lane / G;
  const int64_t W = (p.geo.items + K - 1) / K * p.geo.nbranch;
  for (int64_t w = blockIdx.x; w < W; w += gridDim.x) {
    int br;
    int64_t P0, P1, row;
    group_items<G>(p.geo, w, br, q, P0, P1, row);
    const GroupItem it(P0, P1, IO::V);
    // DYC: each group's row value (read by every lane of the group)
    float dyv = 0.0f;
    if (DYC && P1 > P0) dyv = IO::load1(p.br[br].dy + row * p.dy_rs[br] * IO::ES);
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      group_bwd<IO, true, DYC, G, L>(p.br[br], it, hl, q, dyv);
    else
      group_bwd<IO, false, DYC, G, L>(p.br[br], it, hl, q, dyv);
  }
}

template <class IO, int G>
const void* pick_fwd_group(int dirs) {
  if (dirs == 1) return reinterpret_cast<const void*>(&k_scan_fwd_group<IO, 1, G, 1>);
  if (dirs == 2) return reinterpret_cast<const void*>(&k_scan_fwd_group<IO, 2, G, 1>);
  return reinterpret_cast<const void*>(&k_scan_fwd_group<IO, 3, G, 1>);
}

template <class IO, bool DYC, int G>
const void* pick_bwd_group(int dirs) {
  if (dirs == 1) return reinterpret_cast<const void*>(&k_scan_bwd_group<IO, 1, DYC, G, 1>);
  if (dirs == 2) return reinterpret_cast<const void*>(&k_scan_bwd_group<IO, 2, DYC, G, 1>);
  return reinterpret_cast<const void*>(&k_scan_bwd_group<IO, 3, DYC, G, 1>);
}

template <class IO, int G>
const void* pick_bwd_group(int dirs, bool dyc) {
  return dyc ? pick_bwd_group<IO, true, G>(dirs) : pick_bwd_group<IO, false, G>(dirs);
}

// Lanes per item for the geometry's mean segment (V elements per vector):
// rows of 16 for a mean within one vector per lane of 16 lanes, else
// halves.  Measured with caches flushed, forward / backward us, against
// halves: 16 x 64 fp32 elements x 1536 rows 13.4 / 15.8 -> 11.4 / 13.0,
// 8 x 128 bf16 10.8 / 12.5 -> 9.9 / 11.3, fp16 10.6 / 15.2 -> 10.2 / 10.8,
// ragged 1-120 fp32 elements 30.8 / 43.8 -> 28.8 / 41.4.  Rows of 16 with
// two vectors per lane lost to halves at 128 fp32 elements (11.6 / 15.9
// against 9.9 / 12.3) and on ragged 1-250 (49.8 / 90.3 against 40.3 /
// 58.5).
int group_lanes(const Geometry& geo, int v) {
  const int64_t den = geo.S > 0 ? geo.S : 1;
  return geo.T <= den * 16 * v ? 16 : 32;
}

}  // namespace

// A mean segment of at most one step of a half.  Up to two or four steps
// (T = 256 / 512 fp32, 512 / 1024 bf16 and ragged segments of those means)
// ran at best even with one wave per item and lost up to 25% in the
// backward (the halves of a pair wait for the longer item).
bool group_walk_use(const Geometry& geo, int v) {
  return geo.T <= (geo.S > 0 ? geo.S : 1) * static_cast<int64_t>(32) * v;
}

int group_walk_fwd(const FwdParams& p, int dtype, int dirs, void* stream) {
  const int G = group_lanes(p.geo, 16 / elem_size(dtype));
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = G == 16 ? pick_fwd_group<IoF32, 16>(dirs) : pick_fwd_group<IoF32, 32>(dirs); break;
    case ASC_F16: fn = G == 16 ? pick_fwd_group<IoF16, 16>(dirs) : pick_fwd_group<IoF16, 32>(dirs); break;
    default: fn = G == 16 ? pick_fwd_group<IoBF16, 16>(dirs) : pick_fwd_group<IoBF16, 32>(dirs); break;
  }
  const int64_t K = kWave / G;
  const int64_t groups = (p.geo.items + K - 1) / K * p.geo.nbranch;
  return launch(fn, walk_grid(p, groups, 1), 1, p, stream);
}

int group_walk_bwd(const BwdParams& p, int dtype, int dirs, bool dyc,
                   void* stream) {
  const int G = group_lanes(p.geo, 16 / elem_size(dtype));
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = G == 16 ? pick_bwd_group<IoF32, 16>(dirs, dyc) : pick_bwd_group<IoF32, 32>(dirs, dyc); break;
    case ASC_F16: fn = G == 16 ? pick_bwd_group<IoF16, 16>(dirs, dyc) : pick_bwd_group<IoF16, 32>(dirs, dyc); break;
    default: fn = G == 16 ? pick_bwd_group<IoBF16, 16>(dirs, dyc) : pick_bwd_group<IoBF16, 32>(dirs, dyc); break;
  }
  const int64_t K = kWave / G;
  const int64_t groups = (p.geo.items + K - 1) / K * p.geo.nbranch;
  return launch(fn, walk_grid(p, groups, 1), 1, p, stream);
}

}  // namespace asc
