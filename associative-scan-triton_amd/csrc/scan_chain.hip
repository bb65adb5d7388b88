// Chained-chunk walk: long segments whose edges fall on chunk boundaries.
//
// The workgroup walk streams each (segment, channel) item from end to end in
// one workgroup, so at any moment the chip reads a few hundred separate
// streams, one per row; on MI355X that pattern tops out near 5.5 (backward)
// and 5.8 TB/s (forward).  Here each workgroup owns one chunk of
// kChainWaves x kChainU sub-tiles of one row (4096 fp32 / 8192 fp16-bf16
// elements), workgroups are numbered in scan order along each row, and the
// workgroups that run together stream one contiguous window of memory
// (measured at cfg5's size, forward / backward: 6.15 / 6.23 TB/s against
// 5.84 / 5.55 for the workgroup walk).  Carries
// between the chunks of a segment go through tagged workspace slots, like
// the look-back walk, but with a fixed composition so that results are
// bitwise reproducible from run to run:
//   * chunk j of a segment (in scan order) scans its data, then publishes
//     its aggregate map, or, for j == 0 (which holds the segment head), its
//     inclusive value, or nothing yet for a checkpoint (j % 64 == 63);
//   * its carry-in is composed, with one DPP scan over at most 64 lanes,
//     from the inclusive value of the last checkpoint before it (or of
//     chunk 0) and the aggregates of the chunks in between;
//   * a checkpoint publishes its inclusive value once it has its carry.
// A wait is bounded: after the spin limit the waiting wave scans the
// segment's prefix before its chunk itself (one sub-tile at a time), so
// progress never depends on workgroup scheduling (that carry is composed in
// another order, so only such a pathological wait changes the last bits).
//
// The host cannot see cu_seqlens, so the call first launches the
// workgroup / one-wave walk, which clears the slots and walks the items of
// every segment whose edges are not both on the chunk grid; the chained
// walk then takes the chunks of the other segments (both kernels apply the
// same test to the same cu_seqlens values).  Where every edge is aligned
// the first launch only clears the slots.

#include "chain_common.h"

namespace asc {
namespace {

struct ChainFwdParams {
  ChainGeo geo;
  FwdPtrs br[2];
  LbSlot* slots;  // nbranch * nchunks
};

struct ChainBwdParams {
  ChainGeo geo;
  BwdPtrs br[2];
  int64_t dy_rs[2];  // DYC: element stride between rows of each gradient
  LbSlot* slots;
};

// ---- forward ----
// Carry into the chunk from the segment's elements before it (scan order),
// one sub-tile at a time (the bounded-wait fallback).
template <class IO, bool REV>
__device__ float chain_prefix_fwd(const FwdPtrs& t, const ChainChunk& k,
                                  int lane) {
  constexpr int V = IO::V;
  const int64_t head = REV ? k.P1 - 1 : k.P0;
  const int64_t nsub = k.j * (chain_elems(V) / (kWave * V));
  const int64_t v0 = REV ? k.P1 / V - 1 : k.P0 / V;  // first vector, scan order
  float carry = 0.0f;
  for (int64_t s = 0; s < nsub; ++s) {
    const int64_t i = s * kWave + lane;
    const int64_t vi = REV ? v0 - i : v0 + i;
    float g[V], x[V];
    IO::unpack(ld16(t.g + vi * 16), g);
    IO::unpack(ld16(t.x + vi * 16), x);
    const SubScan ss = s == 0 ? fwd_local<IO, REV, true>(g, x, vi * V, head)
                              : fwd_local<IO, REV, false>(g, x, vi * V, 0);
    carry = fmaf(ss.ta, carry, ss.tx);
  }
  return carry;
}

template <class IO, bool REV>
__device__ inline void chain_fwd_chunk(const ChainFwdParams& p, int br,
                                       int64_t b, int lane, int wv,
                                       float2* agg, float* carry_s) {
  constexpr int V = IO::V;
  constexpr int U = kChainU;
  constexpr int64_t CH = chain_elems(V);
  ChainChunk k;
  const FwdPtrs& t = p.br[br];
  // read the chunk before its segment is looked up when every segment is
  // chunk-aligned (chain_survey_of)
  const uint32_t sv = chain_survey_of(p.geo);
  if (sv == kChainNone) return;
  const bool all = sv == kChainAll;
  if (!all && !chain_chunk<CH>(p.geo, b, REV, k)) return;
  k.row = b / p.geo.kr;
  {
    const int64_t rr = b - k.row * p.geo.kr;
    k.e0 = k.row * p.geo.T + (REV ? p.geo.kr - 1 - rr : rr) * CH;
  }
  uint4 gq[U], xq[U];
  int64_t vi[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = static_cast<int64_t>(wv * U + u) * kWave + lane;
    vi[u] = REV ? (k.e0 + CH) / V - 1 - i : k.e0 / V + i;
    gq[u] = ld16(t.g + vi[u] * 16);
    xq[u] = ld16(t.x + vi[u] * 16);
  }
  if (all && !chain_chunk<CH>(p.geo, b, REV, k)) return;  // outside all
  const int64_t head = REV ? k.P1 - 1 : k.P0;
  const bool hsub = k.j == 0 && wv == 0;  // sub-tile 0 of wave 0 holds the head
  SubScan sc[U];
  float wa = 1.0f, wx = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float g[V], x[V];
    IO::unpack(gq[u], g);
    IO::unpack(xq[u], x);
    if (u == 0 && hsub)
      sc[u] = fwd_local<IO, REV, true>(g, x, vi[u] * V, head);
    else
      sc[u] = fwd_local<IO, REV, false>(g, x, vi[u] * V, 0);
    wx = fmaf(sc[u].ta, wx, sc[u].tx);
    wa = wa * sc[u].ta;
  }
  if (lane == 0) agg[wv] = make_float2(wa, wx);
  __syncthreads();
  if (wv == 0) {
    float A = 1.0f, X = 0.0f;
#pragma unroll
    for (int w = 0; w < kChainWaves; ++w) {
      X = fmaf(agg[w].x, X, agg[w].y);
      A = A * agg[w].x;
    }
    LbSlot* slots = p.slots + br * p.geo.nchunks;
    if (lane == 0) chain_publish(slots + b, k.j, A, X);
    float carry = 0.0f;
    if (k.j > 0)
      carry = chain_carry(slots, b, k.j, lane, p.geo.spin, [&]() {
        return chain_prefix_fwd<IO, REV>(t, k, lane);
      });
    if (lane == 0) {
      *carry_s = carry;
      if (k.j % kChainBlock == kChainBlock - 1)
        lb_put(&slots[b].x, kLbIncl, fmaf(A, carry, X));
    }
  }
  __syncthreads();
  float c = *carry_s;
  for (int w = 0; w < wv; ++w) c = fmaf(agg[w].x, c, agg[w].y);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float g[V], x[V], hf[V];
    repack_point<IO>(gq[u]);
    repack_point<IO>(xq[u]);
    IO::unpack(gq[u], g);
    IO::unpack(xq[u], x);
    if (u == 0 && hsub)
      fwd_apply<IO, REV, true>(g, x, vi[u] * V, head, sc[u], c, hf);
    else
      fwd_apply<IO, REV, false>(g, x, vi[u] * V, 0, sc[u], c, hf);
    st16(t.h + vi[u] * 16, IO::pack(hf));
    c = fmaf(sc[u].ta, c, sc[u].tx);
  }
}

// fp16/bf16: asked for 8 waves per SIMD, the forward fits 55-62 VGPRs
// without spilling (77-85 unasked, 5-6 waves): 8 x 64K segments bf16 5.90 ->
// 6.05 TB/s, fp16 5.43 -> 6.1.  The backward spills 28-76 bytes per lane at
// 8 waves and is slower so (bf16 5.55 against 5.7 TB/s), so it is not asked.
template <class IO, int DIRS>
__global__ void __launch_bounds__(kChainWaves* kWave, IO::V == 4 ? 1 : 8)
    k_scan_fwd_chain(ChainFwdParams p) {
  __shared__ float2 agg[kChainWaves];
  __shared__ float carry_s;
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  const int64_t gb = blockIdx.x;
  const int br = gb >= p.geo.nchunks ? 1 : 0;
  const int64_t b = gb - br * p.geo.nchunks;
  if (DIRS == 1 || (DIRS == 3 && br == 0))
    chain_fwd_chunk<IO, false>(p, br, b, lane, wv, agg, &carry_s);
  else
    chain_fwd_chunk<IO, true>(p, br, b, lane, wv, agg, &carry_s);
}

// ---- backward ----
template <class IO, bool RB, bool DYC>
__device__ inline void chain_bwd_chunk(const ChainBwdParams& p, int br,
                                       int64_t b, int lane, int wv,
                                       float2* agg, float* carry_s) {
  constexpr int V = IO::V;
  constexpr int U = kChainU;
  constexpr int64_t CH = chain_elems(V);
  constexpr int jl = mem_idx<V, RB>(V - 1);  // last element in B order
  constexpr int jf = mem_idx<V, RB>(0);      // first element in B order
  ChainChunk k;
  const BwdPtrs& t = p.br[br];
  // as in chain_fwd_chunk
  const uint32_t sv = chain_survey_of(p.geo);
  if (sv == kChainNone) return;
  const bool all = sv == kChainAll;
  if (!all && !chain_chunk<CH>(p.geo, b, RB, k)) return;
  k.row = b / p.geo.kr;
  {
    const int64_t rr = b - k.row * p.geo.kr;
    k.e0 = k.row * p.geo.T + (RB ? p.geo.kr - 1 - rr : rr) * CH;
  }
  uint4 yq[U], gq[U], hq[U];
  int64_t vi[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = static_cast<int64_t>(wv * U + u) * kWave + lane;
    vi[u] = RB ? (k.e0 + CH) / V - 1 - i : k.e0 / V + i;
    yq[u] = DYC ? make_uint4(0, 0, 0, 0) : ld16(t.dy + vi[u] * 16);
    gq[u] = ld16(t.g + vi[u] * 16);
    hq[u] = ld16(t.h + vi[u] * 16);
  }
  // DYC: the gradient is the row's one value (every element of the chunk
  // lies in the segment)
  const float dyv =
      DYC ? IO::load1(t.dy + k.row * p.dy_rs[br] * IO::ES) : 0.0f;
  auto unpack_y = [&](int u, float* y) {
    if (DYC) {
#pragma unroll
      for (int e = 0; e < V; ++e) y[e] = dyv;
    } else {
      IO::unpack(yq[u], y);
    }
  };
  if (all && !chain_chunk<CH>(p.geo, b, RB, k)) return;
  const int64_t head = RB ? k.P1 - 1 : k.P0;  // B-order head and tail
  const int64_t tail = RB ? k.P0 : k.P1 - 1;
  const bool tail_chunk = RB ? k.first_mem : k.last_mem;
  // the gate just before this wave's first element in B order (1 outside
  // the segment: the pad), the state just past its last one (0 outside)
  const int64_t w0 = static_cast<int64_t>(wv * U) * kWave;
  const int64_t vfirst = RB ? (k.e0 + CH) / V - 1 - w0 : k.e0 / V + w0;
  const int64_t pg = vfirst * V + jf + (RB ? 1 : -1);
  const float gp = (pg >= k.P0 && pg < k.P1) ? IO::load1(t.g + pg * IO::ES) : 1.0f;
  const int64_t wl = w0 + U * kWave - 1;
  const int64_t vlast = RB ? (k.e0 + CH) / V - 1 - wl : k.e0 / V + wl;
  const int64_t ph = RB ? vlast * V - 1 : vlast * V + V;
  const float hn = (ph >= k.P0 && ph < k.P1) ? IO::load1(t.h + ph * IO::ES) : 0.0f;
  auto masked = [&](int u) {
    return (u == 0 && wv == 0 && k.j == 0) ||
           (tail_chunk && u == U - 1 && wv == kChainWaves - 1);
  };
  SubScan sc[U];
  float gprv[U];
  float wa = 1.0f, wx = 0.0f, cg = gp;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float g[V], y[V];
    IO::unpack(gq[u], g);
    unpack_y(u, y);
    if (masked(u))
      sc[u] = bwd_local<IO, RB, true>(g, y, vi[u] * V, head, cg, gprv[u]);
    else
      sc[u] = bwd_local<IO, RB, false>(g, y, vi[u] * V, 0, cg, gprv[u]);
    cg = readlane(g[jl], kWave - 1);
    wx = fmaf(sc[u].ta, wx, sc[u].tx);
    wa = wa * sc[u].ta;
  }
  if (lane == 0) agg[wv] = make_float2(wa, wx);
  __syncthreads();
  if (wv == 0) {
    float A = 1.0f, X = 0.0f;
#pragma unroll
    for (int w = 0; w < kChainWaves; ++w) {
      X = fmaf(agg[w].x, X, agg[w].y);
      A = A * agg[w].x;
    }
    LbSlot* slots = p.slots + br * p.geo.nchunks;
    if (lane == 0) chain_publish(slots + b, k.j, A, X);
    float carry = 0.0f;
    if (k.j > 0)
      carry = chain_carry(slots, b, k.j, lane, p.geo.spin, [&]() {
        return chain_prefix_bwd<IO, RB, DYC>(t, k, lane, dyv);
      });
    if (lane == 0) {
      *carry_s = carry;
      if (k.j % kChainBlock == kChainBlock - 1)
        lb_put(&slots[b].x, kLbIncl, fmaf(A, carry, X));
    }
  }
  __syncthreads();
  float c = *carry_s;
  for (int w = 0; w < wv; ++w) c = fmaf(agg[w].x, c, agg[w].y);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float g[V], y[V], h[V], hnext[V];
    repack_point<IO>(gq[u]);
    repack_point<IO>(yq[u]);
    repack_point<IO>(hq[u]);
    IO::unpack(gq[u], g);
    unpack_y(u, y);
    IO::unpack(hq[u], h);
    float hin = hn;
    if (u + 1 < U) {
      IO::unpack(hq[u + 1 < U ? u + 1 : u], hnext);
      hin = readlane(hnext[jf], 0);
    }
    float dx[V], dg[V];
    if (masked(u))
      bwd_apply<IO, RB, true>(g, y, h, vi[u] * V, head, tail, gprv[u], hin,
                              sc[u], c, dx, dg);
    else
      bwd_apply<IO, RB, false>(g, y, h, vi[u] * V, 0, 0, gprv[u], hin, sc[u],
                               c, dx, dg);
    st16(t.dx + vi[u] * 16, IO::pack(dx));
    st16(t.dg + vi[u] * 16, IO::pack(dg));
    c = fmaf(sc[u].ta, c, sc[u].tx);
  }
}

// DIRS as for the other backward kernels: the forward scan's direction.
template <class IO, int DIRS, bool DYC>
__global__ void __launch_bounds__(kChainWaves* kWave)
    k_scan_bwd_chain(ChainBwdParams p) {
  __shared__ float2 agg[kChainWaves];
  __shared__ float carry_s;
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  const int64_t gb = blockIdx.x;
  const int br = gb >= p.geo.nchunks ? 1 : 0;
  const int64_t b = gb - br * p.geo.nchunks;
  if (DIRS == 1 || (DIRS == 3 && br == 0))
    chain_bwd_chunk<IO, true, DYC>(p, br, b, lane, wv, agg, &carry_s);
  else
    chain_bwd_chunk<IO, false, DYC>(p, br, b, lane, wv, agg, &carry_s);
}

// dirs 1 or 2: a two-branch call launches each branch on its own
template <class IO>
const void* pick_fwd_chain(int dirs) {
  if (dirs == 1) return reinterpret_cast<const void*>(&k_scan_fwd_chain<IO, 1>);
  return reinterpret_cast<const void*>(&k_scan_fwd_chain<IO, 2>);
}

template <class IO, bool DYC>
const void* pick_bwd_chain(int dirs) {
  if (dirs == 1) return reinterpret_cast<const void*>(&k_scan_bwd_chain<IO, 1, DYC>);
  return reinterpret_cast<const void*>(&k_scan_bwd_chain<IO, 2, DYC>);
}

template <class IO>
const void* pick_bwd_chain(int dirs, bool dyc) {
  return dyc ? pick_bwd_chain<IO, true>(dirs) : pick_bwd_chain<IO, false>(dirs);
}

}  // namespace

int64_t chain_bytes(int64_t S, int64_t C, int64_t T, int v, int nbranch) {
  // the larger of the forward's and the backward's needs (one size serves
  // both calls)
  int64_t kr = chain_rows(S, C, T, v, nbranch, true);
  if (kr == 0) kr = chain_rows(S, C, T, v, nbranch, false);
  return kr == 0 ? 0 : chain_need(C, kr, nbranch);
}

bool chain_plan(Geometry& g, bool aln, int dtype, void* ws, int64_t ws_bytes,
                bool bwd) {
  return chain_share(g, aln, 16 / elem_size(dtype), ws, ws_bytes, bwd);
}

int chain_fwd(const FwdParams& p, int dtype, int dirs, void* stream) {
  const int v = 16 / elem_size(dtype);
  ChainFwdParams q{};
  q.geo = chain_geo(p.geo, v);
  q.slots = reinterpret_cast<LbSlot*>(p.geo.chain_slots);
  // one launch per branch (both branches in one grid measured slower)
  auto one = [&](int b, int d) {
    ChainFwdParams r = q;
    r.geo.nbranch = 1;
    r.br[0] = p.br[b];
    r.slots = q.slots + b * q.geo.nchunks;
    const void* fn = nullptr;
    switch (dtype) {
      case ASC_F32: fn = pick_fwd_chain<IoF32>(d); break;
      case ASC_F16: fn = pick_fwd_chain<IoF16>(d); break;
      default: fn = pick_fwd_chain<IoBF16>(d); break;
    }
    return launch(fn, r.geo.nchunks, kChainWaves, r, stream);
  };
  int status = dirs == 3 ? one(0, 1) : one(0, dirs);
  if (status == ASC_OK && dirs == 3) status = one(1, 2);
  return status;
}

int chain_bwd(const BwdParams& p, int dtype, bool dyc, int dirs,
              void* stream) {
  const int v = 16 / elem_size(dtype);
  ChainBwdParams q{};
  q.geo = chain_geo(p.geo, v);
  q.slots = reinterpret_cast<LbSlot*>(p.geo.chain_slots);
  auto one = [&](int b, int d) {
    ChainBwdParams r = q;
    r.geo.nbranch = 1;
    r.br[0] = p.br[b];
    r.dy_rs[0] = p.dy_rs[b];
    r.slots = q.slots + b * q.geo.nchunks;
    const void* fn = nullptr;
    switch (dtype) {
      case ASC_F32: fn = pick_bwd_chain<IoF32>(d, dyc); break;
      case ASC_F16: fn = pick_bwd_chain<IoF16>(d, dyc); break;
      default: fn = pick_bwd_chain<IoBF16>(d, dyc); break;
    }
    return launch(fn, r.geo.nchunks, kChainWaves, r, stream);
  };
  int status = dirs == 3 ? one(0, 1) : one(0, dirs);
  if (status == ASC_OK && dirs == 3) status = one(1, 2);
  return status;
}

}  // namespace asc
