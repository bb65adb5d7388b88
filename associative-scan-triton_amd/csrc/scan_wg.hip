#include "asc_common.h"

namespace asc {
namespace {

// ---------------------------------------------------------------------------
// Workgroup-cooperative walk for long segments.  NW waves of one workgroup
// sweep one item together: in iteration `it`, wave `wv` owns sub-tiles
// it*NW*kUW + wv*kUW + u (u < kUW), so an iteration streams NW*kUW KiB of
// every tensor contiguously and far fewer rows are in flight at once than
// with one wave per item (HBM rewards the fewer, wider streams).  After
// its wave scans, each wave publishes its aggregate map in LDS; after one
// barrier every wave folds the aggregates of the waves before it into the
// iteration carry.  All waves fold the same values in the same order, so
// they agree bit for bit on the next carry.  The aggregate array is
// double-buffered by iteration parity: one barrier per iteration suffices.
// The next iteration's loads are issued before the current one is scanned.
// ---------------------------------------------------------------------------
template <class IO, bool REV>
__device__ inline bool interior(const Walk<IO, REV>& w, int64_t kk) {
  return kk >= 1 && kk < w.kfast;
}

template <class IO, bool REV, bool ALN>
__device__ inline void load_sub(const char* origin, const Walk<IO, REV>& w,
                                int64_t kk, int lane, float ident, float* f) {
  const int64_t vi = w.vec(kk, lane);
  if (interior(w, kk))
    load_vec<IO, ALN, false>(origin, vi, true, w.P0, w.P1, ident, f);
  else
    load_vec<IO, ALN, true>(origin, vi, w.lane_valid(kk, lane), w.P0, w.P1,
                            ident, f);
}

template <class IO, bool REV, bool ALN>
__device__ inline void store_sub(char* origin, const Walk<IO, REV>& w,
                                 int64_t kk, int lane, const float* f) {
  const int64_t vi = w.vec(kk, lane);
  if (interior(w, kk))
    store_vec<IO, ALN, false>(origin, vi, true, w.P0, w.P1, f);
  else
    store_vec<IO, ALN, true>(origin, vi, w.lane_valid(kk, lane), w.P0, w.P1, f);
}

// Folds the aggregates of waves [0, wv) into `carry` and returns the carry
// into wave wv; `carry` advances over all NW aggregates.
template <int NW>
__device__ inline float fold_aggregates(const float2* slot, int wv,
                                        float& carry) {
  float run = carry, mine = carry;
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    if (j == wv) mine = run;
    const float2 a = slot[j];
    run = fmaf(a.x, run, a.y);
  }
  carry = run;
  return mine;
}

template <class IO, bool REV, bool ALN, int NW>
__device__ void fwd_item_wg(const FwdPtrs& t, int64_t P0, int64_t P1,
                            int lane, int wv, float2* agg) {
  constexpr int V = IO::V;
  constexpr int TS = NW * kUW;
  const Walk<IO, REV> w(P0, P1, t.pend);
  const int64_t niter = (w.nsub + TS - 1) / TS;
  float gA[kUW][V], xA[kUW][V], gB[kUW][V], xB[kUW][V];
  float carry = 0.0f;
  auto load = [&](float(&g)[kUW][V], float(&x)[kUW][V], int64_t it) {
#pragma unroll
    for (int u = 0; u < kUW; ++u) {
      const int64_t kk = it * TS + wv * kUW + u;
      load_sub<IO, REV, ALN>(t.g, w, kk, lane, 1.0f, g[u]);
      load_sub<IO, REV, ALN>(t.x, w, kk, lane, 0.0f, x[u]);
    }
  };
  auto step = [&](const float(&g)[kUW][V], const float(&x)[kUW][V],
                  int64_t it) {
    SubScan sc[kUW];
    float wa = 1.0f, wx = 0.0f;
#pragma unroll
    for (int u = 0; u < kUW; ++u) {
      const int64_t kk = it * TS + wv * kUW + u;
      const int64_t pv = w.vec(kk, lane) * V;
      if (interior(w, kk))
        sc[u] = fwd_local<IO, REV, false>(g[u], x[u], pv, 0);
      else
        sc[u] = fwd_local<IO, REV, true>(g[u], x[u], pv, w.head());
      wx = fmaf(sc[u].ta, wx, sc[u].tx);
      wa = wa * sc[u].ta;
    }
    float2* slot = agg + (it & 1) * NW;
    if (lane == 0) slot[wv] = make_float2(wa, wx);
    __syncthreads();
    float c = fold_aggregates<NW>(slot, wv, carry);
#pragma unroll
    for (int u = 0; u < kUW; ++u) {
      const int64_t kk = it * TS + wv * kUW + u;
      const int64_t pv = w.vec(kk, lane) * V;
      float hf[V];
      if (interior(w, kk))
        fwd_apply<IO, REV, false>(g[u], x[u], pv, 0, sc[u], c, hf);
      else
        fwd_apply<IO, REV, true>(g[u], x[u], pv, w.head(), sc[u], c, hf);
      store_sub<IO, REV, ALN>(t.h, w, kk, lane, hf);
      c = fmaf(sc[u].ta, c, sc[u].tx);
    }
  };
  load(gA, xA, 0);
  for (int64_t it = 0;; it += 2) {
    if (it + 1 < niter) load(gB, xB, it + 1);
    step(gA, xA, it);
    if (it + 1 >= niter) break;
    if (it + 2 < niter) load(gA, xA, it + 2);
    step(gB, xB, it + 1);
    if (it + 2 >= niter) break;
  }
}

// Gate of the element just before sub-tile kk in B order (1 outside the
// segment: the pad; the head select makes its value irrelevant there).
template <class IO, bool RB>
__device__ inline float bwd_gate_before(const BwdPtrs& t,
                                        const Walk<IO, RB>& w, int64_t kk) {
  constexpr int V = IO::V;
  const int64_t pf = w.vec(kk, 0) * V + mem_idx<V, RB>(0);
  const int64_t pp = RB ? pf + 1 : pf - 1;
  return (pp >= w.P0 && pp < w.P1) ? IO::load1(t.g + pp * IO::ES) : 1.0f;
}

template <class IO, bool RB, bool ALN, int NW, bool DYC>
__device__ void bwd_item_wg(const BwdPtrs& t, int64_t P0, int64_t P1,
                            int lane, int wv, float2* agg, float dyv) {
  constexpr int V = IO::V;
  constexpr int TS = NW * kUW;
  constexpr int jl = mem_idx<V, RB>(V - 1);
  constexpr int jf = mem_idx<V, RB>(0);
  const Walk<IO, RB> w(P0, P1, t.pend);
  const int64_t niter = (w.nsub + TS - 1) / TS;
  float yA[kUW][V], gA[kUW][V], hA[kUW][V];
  float yB[kUW][V], gB[kUW][V], hB[kUW][V];
  float gpA, hnA, gpB, hnB;
  float carry = 0.0f;
  auto load = [&](float(&y)[kUW][V], float(&g)[kUW][V], float(&h)[kUW][V],
                  float& gp, float& hn, int64_t it) {
    const int64_t k0 = it * TS + wv * kUW;
#pragma unroll
    for (int u = 0; u < kUW; ++u) {
      if (!DYC) load_sub<IO, RB, ALN>(t.dy, w, k0 + u, lane, 0.0f, y[u]);
      load_sub<IO, RB, ALN>(t.g, w, k0 + u, lane, 1.0f, g[u]);
      load_sub<IO, RB, ALN>(t.h, w, k0 + u, lane, 0.0f, h[u]);
    }
    gp = bwd_gate_before(t, w, k0);
    hn = bwd_halo(t, w, k0, kUW);
  };
  auto step = [&](const float(&yl)[kUW][V], const float(&g)[kUW][V],
                  const float(&h)[kUW][V], float gp, float hn, int64_t it) {
    const int64_t k0 = it * TS + wv * kUW;
    // DYC: dy is built here from the row's value, not carried in the
    // ping-pong buffers
    float yc[kUW][V];
    if (DYC) {
#pragma unroll
      for (int u = 0; u < kUW; ++u) {
        if (interior(w, k0 + u))
          dyc_vec<IO, false>(dyv, 0, true, 0, 0, yc[u]);
        else
          dyc_vec<IO, true>(dyv, w.vec(k0 + u, lane), w.lane_valid(k0 + u, lane),
                            w.P0, w.P1, yc[u]);
      }
    }
    const float(&y)[kUW][V] = DYC ? yc : yl;
    SubScan sc[kUW];
    float gprv[kUW];
    float wa = 1.0f, wx = 0.0f, cg = gp;
#pragma unroll
    for (int u = 0; u < kUW; ++u) {
      const int64_t pv = w.vec(k0 + u, lane) * V;
      if (interior(w, k0 + u))
        sc[u] = bwd_local<IO, RB, false>(g[u], y[u], pv, 0, cg, gprv[u]);
      else
        sc[u] = bwd_local<IO, RB, true>(g[u], y[u], pv, w.head(), cg, gprv[u]);
      cg = readlane(g[u][jl], kWave - 1);
      wx = fmaf(sc[u].ta, wx, sc[u].tx);
      wa = wa * sc[u].ta;
    }
    float2* slot = agg + (it & 1) * NW;
    if (lane == 0) slot[wv] = make_float2(wa, wx);
    __syncthreads();
    float c = fold_aggregates<NW>(slot, wv, carry);
#pragma unroll
    for (int u = 0; u < kUW; ++u) {
      const int64_t kk = k0 + u;
      const int64_t pv = w.vec(kk, lane) * V;
      const float hin = (u + 1 < kUW) ? readlane(h[u + 1][jf], 0) : hn;
      float dx[V], dg[V];
      if (interior(w, kk))
        bwd_apply<IO, RB, false>(g[u], y[u], h[u], pv, 0, 0, gprv[u], hin,
                                 sc[u], c, dx, dg);
      else
        bwd_apply<IO, RB, true>(g[u], y[u], h[u], pv, w.head(), w.tail(),
                                gprv[u], hin, sc[u], c, dx, dg);
      store_sub<IO, RB, ALN>(t.dx, w, kk, lane, dx);
      store_sub<IO, RB, ALN>(t.dg, w, kk, lane, dg);
      c = fmaf(sc[u].ta, c, sc[u].tx);
    }
  };
  load(yA, gA, hA, gpA, hnA, 0);
  for (int64_t it = 0;; it += 2) {
    if (it + 1 < niter) load(yB, gB, hB, gpB, hnB, it + 1);
    step(yA, gA, hA, gpA, hnA, it);
    if (it + 1 >= niter) break;
    if (it + 2 < niter) load(yA, gA, hA, gpA, hnA, it + 2);
    step(yB, gB, hB, gpB, hnB, it + 1);
    if (it + 2 >= niter) break;
  }
}


// Workgroup-cooperative kernels: one item per workgroup of NW waves.
// BLK: item order in channel blocks (item_range).
template <class IO, int DIRS, bool ALN, int NW, bool BLK>
__global__ void __launch_bounds__(NW* kWave) k_scan_fwd_wg(FwdParams p) {
  if (skipped(p)) return;
  __shared__ float2 agg[2 * NW];
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  const int64_t W = p.geo.items * p.geo.nbranch;
  for (int64_t item = blockIdx.x; item < W; item += gridDim.x) {
    int br;
    int64_t P0, P1, row;
    if (!item_range(p.geo, item, br, P0, P1, row, BLK)) continue;
    const FwdPtrs& t = p.br[br];
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      fwd_item_wg<IO, false, ALN, NW>(t, P0, P1, lane, wv, agg);
    else
      fwd_item_wg<IO, true, ALN, NW>(t, P0, P1, lane, wv, agg);
    __syncthreads();  // agg is reused by the next item
  }
}

template <class IO, int DIRS, bool ALN, int NW, bool DYC, bool BLK>
__global__ void __launch_bounds__(NW* kWave) k_scan_bwd_wg(BwdParams p) {
  if (skipped(p)) return;
  __shared__ float2 agg[2 * NW];
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  const int64_t W = p.geo.items * p.geo.nbranch;
  for (int64_t item = blockIdx.x; item < W; item += gridDim.x) {
    int br;
    int64_t P0, P1, row;
    if (!item_range(p.geo, item, br, P0, P1, row, BLK)) continue;
    const BwdPtrs& t = p.br[br];
    const float dyv = dyc_value<IO, DYC>(p, br, row);
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      bwd_item_wg<IO, true, ALN, NW, DYC>(t, P0, P1, lane, wv, agg, dyv);
    else
      bwd_item_wg<IO, false, ALN, NW, DYC>(t, P0, P1, lane, wv, agg, dyv);
    __syncthreads();
  }
}

template <class IO, int NW, bool BLK>
const void* pick_fwd_wg(int dirs, bool aln) {
#define ASC_F(D, A) reinterpret_cast<const void*>(&k_scan_fwd_wg<IO, D, A, NW, BLK>)
  if (dirs == 1) return aln ? ASC_F(1, true) : ASC_F(1, false);
  if (dirs == 2) return aln ? ASC_F(2, true) : ASC_F(2, false);
  return aln ? ASC_F(3, true) : ASC_F(3, false);
#undef ASC_F
}

template <class IO, int NW, bool BLK>
const void* pick_bwd_wg(int dirs, bool aln, bool dyc) {
#define ASC_B(D, A, Y) reinterpret_cast<const void*>(&k_scan_bwd_wg<IO, D, A, NW, Y, BLK>)
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

template <class IO>
const void* pick_fwd_wg(int nw, int dirs, bool aln, bool blk) {
  if (blk)
    return nw == 16 ? pick_fwd_wg<IO, 16, true>(dirs, aln) : pick_fwd_wg<IO, 8, true>(dirs, aln);
  return nw == 16 ? pick_fwd_wg<IO, 16, false>(dirs, aln) : pick_fwd_wg<IO, 8, false>(dirs, aln);
}

template <class IO>
const void* pick_bwd_wg(int nw, int dirs, bool aln, bool dyc, bool blk) {
  if (blk)
    return nw == 16 ? pick_bwd_wg<IO, 16, true>(dirs, aln, dyc)
                    : pick_bwd_wg<IO, 8, true>(dirs, aln, dyc);
  return nw == 16 ? pick_bwd_wg<IO, 16, false>(dirs, aln, dyc)
                  : pick_bwd_wg<IO, 8, false>(dirs, aln, dyc);
}

// Item order of the workgroup walks: channel blocks up to a mean segment
// of 32K elements, channel-major beyond (measured, fp32, see item_range).
bool wg_chan_blocks(const Geometry& geo) {
  return geo.T / (geo.S > 0 ? geo.S : 1) <= 32768;
}

}  // namespace

int wg_fwd(FwdParams p, int nw, int dtype, int dirs, bool aln, void* stream) {
  const bool blk = wg_chan_blocks(p.geo);
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = pick_fwd_wg<IoF32>(nw, dirs, aln, blk); break;
    case ASC_F16: fn = pick_fwd_wg<IoF16>(nw, dirs, aln, blk); break;
    default: fn = pick_fwd_wg<IoBF16>(nw, dirs, aln, blk); break;
  }
  return launch(fn, walk_grid(p, p.geo.items * p.geo.nbranch, nw), nw, p, stream);
}

int wg_bwd(BwdParams p, int nw, int dtype, int dirs, bool aln, bool dyc,
           void* stream) {
  const bool blk = wg_chan_blocks(p.geo);
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = pick_bwd_wg<IoF32>(nw, dirs, aln, dyc, blk); break;
    case ASC_F16: fn = pick_bwd_wg<IoF16>(nw, dirs, aln, dyc, blk); break;
    default: fn = pick_bwd_wg<IoBF16>(nw, dirs, aln, dyc, blk); break;
  }
  return launch(fn, walk_grid(p, p.geo.items * p.geo.nbranch, nw), nw, p, stream);
}

}  // namespace asc
