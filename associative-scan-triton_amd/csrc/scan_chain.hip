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
// The host cannot see cu_seqlens, so a setup kernel checks on the device
// that every edge is chunk-aligned (and zeroes the slots); the chained walk
// runs only then, and the workgroup / one-wave walk launched after it with
// the same flag runs only otherwise.

#include "asc_common.h"
#include "lookback_slots.h"

namespace asc {
namespace {

// Chunk shape, measured on MI355X (fp32, C = 1536, 64K / 16K segments,
// forward / backward TB/s): 8 waves x 2 sub-tiles 6.18 / 6.26 and 6.09 /
// 5.97; 8 x 4 6.05 / 6.00 and 5.74 / 5.53; 16 x 2 5.96 / 6.09 and 5.68 /
// 5.56; 16 x 4 5.72 / 5.58; 4 x 2 5.06 / 5.64 (64K); one sub-tile per
// wave (8 or 16 waves) 4.2-5.2 forward.
constexpr int kChainWaves = 8;  // waves per workgroup (one chunk)
constexpr int kChainU = 2;      // sub-tiles per wave
constexpr int64_t kChainFlagBytes = 256;  // workspace: flag word, then slots
constexpr int kChainBlock = 64;           // chunks per checkpoint

// fp16/bf16 chunks keep their loaded vectors packed while the chunk waits
// for its carry and unpack them again to apply it (fp32 unpacking is a
// bitcast).  The empty asm marks the packed words as changed, so that the
// compiler cannot reuse the first unpacking and keep 8 floats per vector
// alive across the barrier instead of 4 words.
template <class IO>
__device__ inline void repack_point(uint4& q) {
  if (IO::V != 4)
    asm volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w));
}

constexpr int64_t chain_elems(int v) {
  return static_cast<int64_t>(kChainWaves) * kChainU * kWave * v;
}

struct ChainGeo {
  const void* cu;
  int cu64;
  int64_t S, C, T;
  int64_t kr;       // chunks per row
  int64_t nchunks;  // chunks per branch (C * kr)
  int nbranch;
  uint32_t spin;
  const uint32_t* ok;  // set by the setup kernel: every edge chunk-aligned
};

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

__device__ inline int64_t chain_cu(const ChainGeo& g, int64_t i) {
  return uniform(g.cu64
                     ? reinterpret_cast<const int64_t*>(g.cu)[i]
                     : static_cast<int64_t>(reinterpret_cast<const int32_t*>(g.cu)[i]));
}

// Segment holding row offset t: the last s with cu[s] <= t; -1 before
// cu[0], S at or past cu[S].
__device__ inline int64_t chain_seg(const ChainGeo& g, int64_t t) {
  if (t < chain_cu(g, 0)) return -1;
  if (t >= chain_cu(g, g.S)) return g.S;
  int64_t lo = 0, hi = g.S;  // cu[lo] <= t < cu[hi]
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (chain_cu(g, mid) <= t) lo = mid;
    else hi = mid;
  }
  return lo;
}

// Where chunk b (scan order within its branch) lies.  rev: the scan runs
// from high to low addresses, so the row's chunks are numbered from its end.
struct ChainChunk {
  int64_t row, t0;  // row and row offset of the chunk's first element
  int64_t e0;       // element index (phase 0) of that element
  int64_t P0, P1;   // the segment's element range
  int64_t j;        // index of the chunk within its segment, in scan order
  bool first_mem;   // the chunk starts at the segment start (memory order)
  bool last_mem;    // the chunk ends at the segment end
};

template <int64_t CH>
__device__ inline bool chain_chunk(const ChainGeo& g, int64_t b, bool rev,
                                   ChainChunk& k) {
  k.row = b / g.kr;
  const int64_t rr = b - k.row * g.kr;
  k.t0 = (rev ? g.kr - 1 - rr : rr) * CH;
  k.e0 = k.row * g.T + k.t0;
  const int64_t s = chain_seg(g, k.t0);
  if (s < 0 || s >= g.S) return false;
  const int64_t s0 = chain_cu(g, s), s1 = chain_cu(g, s + 1);
  k.P0 = k.row * g.T + s0;
  k.P1 = k.row * g.T + s1;
  k.j = rev ? (s1 - k.t0 - CH) / CH : (k.t0 - s0) / CH;
  k.first_mem = k.t0 == s0;
  k.last_mem = k.t0 + CH == s1;
  return true;
}

// Publishes a chunk's map right after its local scan: chunk 0 holds the
// head, so its map is its inclusive value; a checkpoint publishes later.
__device__ inline void chain_publish(LbSlot* sl, int64_t j, float A, float X) {
  if (j == 0) {
    lb_put(&sl->x, kLbIncl, X);
  } else if (j % kChainBlock != kChainBlock - 1) {
    lb_put(&sl->a, kLbAgg, A);
    lb_put(&sl->x, kLbAgg, X);
  }
}

// Carry into chunk j > 0 (slot b) from its predecessors' slots (chunk k of
// the segment sits in slot b - (j - k)); `prefix` computes it from the
// inputs if a wait runs past the spin limit.  Called by one whole wave.
template <class Prefix>
__device__ inline float chain_carry(LbSlot* slots, int64_t b, int64_t j,
                                    int lane, uint32_t spin, Prefix prefix) {
  const int64_t cp = (j / kChainBlock) * kChainBlock - 1;  // checkpoint
  const int64_t base = cp < 0 ? 0 : cp;  // its inclusive value, or chunk 0's
  const int n = static_cast<int>(j - base);  // lanes [0, n): chunks base..j-1
  const bool need = lane < n;
  LbSlot* mine = slots + (b - j + base + (need ? lane : 0));
  float ma = 1.0f, mx = 0.0f;
  bool have = !need;
  for (uint32_t polls = 0;; ++polls) {
    if (!have) {
      float a, x;
      const int kind = lb_read(mine, a, x);
      if (lane == 0 ? kind == kLbIncl : kind == kLbAgg) {
        have = true;
        ma = lane == 0 ? 0.0f : a;
        mx = x;
      }
    }
    if (__builtin_amdgcn_ballot_w64(!have) == 0) break;
    if (polls >= spin) return prefix();
    __builtin_amdgcn_s_sleep(2);
  }
  wave_scan_affine(ma, mx);
  return readlane(mx, n - 1);
}

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
  // the chunk lies inside one segment or outside all (aligned edges), so
  // its vectors are read whole before the segment is looked up
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
  if (!chain_chunk<CH>(p.geo, b, REV, k)) return;  // outside every segment
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
  if (*p.geo.ok == 0u) return;
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
// RB: B order (the adjoint's scan order) is reverse memory order, the
// backward of a causal forward scan.
template <class IO, bool RB, bool DYC>
__device__ float chain_prefix_bwd(const BwdPtrs& t, const ChainChunk& k,
                                  int lane, float dyv) {
  constexpr int V = IO::V;
  constexpr int jl = mem_idx<V, RB>(V - 1);
  const int64_t head = RB ? k.P1 - 1 : k.P0;
  const int64_t nsub = k.j * (chain_elems(V) / (kWave * V));
  const int64_t v0 = RB ? k.P1 / V - 1 : k.P0 / V;
  float carry = 0.0f, cg = 1.0f;
  for (int64_t s = 0; s < nsub; ++s) {
    const int64_t i = s * kWave + lane;
    const int64_t vi = RB ? v0 - i : v0 + i;
    float g[V], y[V], gprev;
    IO::unpack(ld16(t.g + vi * 16), g);
    if (DYC) {
#pragma unroll
      for (int e = 0; e < V; ++e) y[e] = dyv;
    } else {
      IO::unpack(ld16(t.dy + vi * 16), y);
    }
    const SubScan ss =
        s == 0 ? bwd_local<IO, RB, true>(g, y, vi * V, head, cg, gprev)
               : bwd_local<IO, RB, false>(g, y, vi * V, 0, cg, gprev);
    cg = readlane(g[jl], kWave - 1);
    carry = fmaf(ss.ta, carry, ss.tx);
  }
  return carry;
}

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
  if (!chain_chunk<CH>(p.geo, b, RB, k)) return;
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
  if (*p.geo.ok == 0u) return;
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

// Zeroes the slots; block 0 also sets *ok to 1 exactly when cu_seqlens is
// non-decreasing, inside [0, T] and a multiple of the chunk size throughout.
__global__ void __launch_bounds__(256)
    k_chain_setup(u64* slots, int64_t nwords, const void* cu, int cu64,
                  int64_t S, int64_t T, int64_t CH, uint32_t* ok) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
       i < nwords; i += stride)
    slots[i] = 0;
  if (blockIdx.x != 0) return;
  int good = 1;
  for (int64_t s = threadIdx.x; s <= S; s += 256) {
    const int64_t v = cu64 ? reinterpret_cast<const int64_t*>(cu)[s]
                           : reinterpret_cast<const int32_t*>(cu)[s];
    if (v < 0 || v > T || v % CH != 0) good = 0;
    if (s > 0) {
      const int64_t pv = cu64 ? reinterpret_cast<const int64_t*>(cu)[s - 1]
                              : reinterpret_cast<const int32_t*>(cu)[s - 1];
      if (pv > v) good = 0;
    }
  }
  good = __syncthreads_and(good);
  if (threadIdx.x == 0) *ok = good ? 1u : 0u;
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

// Chunks per row when the geometry can take the chained walk: rows a
// multiple of the chunk size, a mean segment of 1 to kChainMaxMean chunks
// (32 for the backward), one workgroup per chunk within the grid limit; 0
// otherwise.  Measured on MI355X against the per-item walks (C =
// 1536, uniform segments), fp32 forward / backward TB/s:
//   8K elements 5.9 / 5.8 against 5.8 / 5.5;  32K 6.1 / 5.9 against 5.7 / 5.6;
//   64K 6.2 / 6.3 against 5.9 / 5.5;  128K 5.5 / 5.9 against 5.9 / 5.5;
//   512K 4.4 / 5.1 against 5.8 / 5.5 (a chunk waits for every aggregate of
//   its window, so long windows suffer from stragglers; checkpoints every 8
//   or 16 chunks serialise instead and were slower still);
// bf16 6.05 / 5.7 at 64K against 5.0 / 4.9 (packed vectors held across the
// barrier and 8 forward waves per SIMD; 5.3 / 5.5 before).  Two-branch calls launch
// each branch on its own: both in one grid ran at 5.8 / 5.8 (cfg4) where
// one branch at a time runs 6.2 / 6.0 (the per-item walks: 6.1 / 5.8).
constexpr int64_t kChainMaxMeanFwd = 16, kChainMaxMeanBwd = 32;
int64_t chain_rows(int64_t S, int64_t C, int64_t T, int v, int nbranch,
                   bool bwd) {
  const int64_t CH = chain_elems(v);
  if (S <= 0 || C <= 0 || T <= 0 || T % CH != 0) return 0;
  const int64_t mean = T / S;
  if (mean < CH || mean > (bwd ? kChainMaxMeanBwd : kChainMaxMeanFwd) * CH)
    return 0;
  const int64_t kr = T / CH;
  if (kr > kMaxGrid / C) return 0;
  return kr;
}

ChainGeo chain_geo(const Geometry& g, int v, void* ws) {
  ChainGeo q{};
  q.cu = g.cu;
  q.cu64 = g.cu64;
  q.S = g.S;
  q.C = g.C;
  q.T = g.T;
  q.kr = g.T / chain_elems(v);
  q.nchunks = g.C * q.kr;
  q.nbranch = g.nbranch;
  q.spin = lb_spin_limit();
  q.ok = static_cast<const uint32_t*>(ws);
  return q;
}

int chain_setup(const ChainGeo& q, int v, void* ws, void* stream) {
  u64* slots = reinterpret_cast<u64*>(static_cast<char*>(ws) + kChainFlagBytes);
  int64_t nwords = q.nchunks * q.nbranch * static_cast<int64_t>(sizeof(LbSlot) / 8);
  int64_t blocks = (nwords + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  const void* cu = q.cu;
  int cu64 = q.cu64;
  int64_t S = q.S, T = q.T, CH = chain_elems(v);
  uint32_t* ok = static_cast<uint32_t*>(ws);
  void* args[] = {&slots, &nwords, &cu, &cu64, &S, &T, &CH, &ok};
  const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&k_chain_setup),
                                       dim3(static_cast<unsigned>(blocks)), dim3(256),
                                       args, 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ASC_OK : static_cast<int>(e);
}

int64_t chain_need(int64_t C, int64_t kr, int nbranch) {
  return kChainFlagBytes + nbranch * C * kr * static_cast<int64_t>(sizeof(LbSlot));
}

// Common conditions: a workspace, all tensors 16-byte aligned (phase 0), a
// geometry the walk takes.
bool chain_ready(const Geometry& g, bool aln, int v, void* ws,
                 int64_t ws_bytes, bool bwd) {
  if (!ws || reinterpret_cast<uintptr_t>(ws) % 32 != 0) return false;
  if (!aln || g.phase != 0) return false;
  const int64_t kr = chain_rows(g.S, g.C, g.T, v, g.nbranch, bwd);
  return kr > 0 && ws_bytes >= chain_need(g.C, kr, g.nbranch);
}

}  // namespace

int64_t chain_bytes(int64_t S, int64_t C, int64_t T, int v, int nbranch) {
  // the larger of the forward's and the backward's needs (one size serves
  // both calls)
  int64_t kr = chain_rows(S, C, T, v, nbranch, true);
  if (kr == 0) kr = chain_rows(S, C, T, v, nbranch, false);
  return kr == 0 ? 0 : chain_need(C, kr, nbranch);
}

bool chain_fwd(const FwdParams& p, int dtype, bool aln, int dirs, void* ws,
               int64_t ws_bytes, void* stream, int& status,
               const uint32_t** skip) {
  const int v = 16 / elem_size(dtype);
  if (!chain_ready(p.geo, aln, v, ws, ws_bytes, false)) return false;
  ChainFwdParams q{};
  q.geo = chain_geo(p.geo, v, ws);
  for (int b = 0; b < p.geo.nbranch; ++b) q.br[b] = p.br[b];
  q.slots = reinterpret_cast<LbSlot*>(static_cast<char*>(ws) + kChainFlagBytes);
  if ((status = chain_setup(q.geo, v, ws, stream))) return true;
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
  status = dirs == 3 ? one(0, 1) : one(0, dirs);
  if (status == ASC_OK && dirs == 3) status = one(1, 2);
  *skip = static_cast<const uint32_t*>(ws);
  return true;
}

bool chain_bwd(const BwdParams& p, int dtype, bool aln, bool dyc, int dirs,
               void* ws, int64_t ws_bytes, void* stream, int& status,
               const uint32_t** skip) {
  const int v = 16 / elem_size(dtype);
  if (!chain_ready(p.geo, aln, v, ws, ws_bytes, true)) return false;
  ChainBwdParams q{};
  q.geo = chain_geo(p.geo, v, ws);
  for (int b = 0; b < p.geo.nbranch; ++b) {
    q.br[b] = p.br[b];
    q.dy_rs[b] = p.dy_rs[b];
  }
  q.slots = reinterpret_cast<LbSlot*>(static_cast<char*>(ws) + kChainFlagBytes);
  if ((status = chain_setup(q.geo, v, ws, stream))) return true;
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
  status = dirs == 3 ? one(0, 1) : one(0, dirs);
  if (status == ASC_OK && dirs == 3) status = one(1, 2);
  *skip = static_cast<const uint32_t*>(ws);
  return true;
}

}  // namespace asc
