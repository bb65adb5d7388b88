// Shared pieces of the chained-chunk walks (scan_chain.hip: the plain
// forward and backward; scan_recompute.hip: the backward that recomputes the
// forward states): the chunk shape, the tagged carry slots and their fixed
// composition order, which segments the walk takes, and the host-side
// geometry conditions.  See scan_chain.hip for the walk itself.
#ifndef ASC_CHAIN_COMMON_H
#define ASC_CHAIN_COMMON_H

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
constexpr int kChainBlock = 64;           // chunks per checkpoint
constexpr int64_t kChainFlagBytes = 256;  // workspace: flag word, then slots

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
  // written by the per-item walk launched before (chain_survey)
  const uint32_t* survey;
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
// Returns false unless the segment holding the chunk's first element lies
// inside [0, T] with both edges on the chunk grid (then it holds the whole
// chunk); the per-item walk launched before the chained walk takes every
// other segment (chain_takes applies the same test).
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
  if (!chain_takes(CH, g.T, s0, s1)) return false;
  k.P0 = k.row * g.T + s0;
  k.P1 = k.row * g.T + s1;
  k.j = rev ? (s1 - k.t0 - CH) / CH : (k.t0 - s0) / CH;
  k.first_mem = k.t0 == s0;
  k.last_mem = k.t0 + CH == s1;
  return true;
}

// What the per-item walk launched before found (chain_survey; one scalar
// load).  kChainAll: a chunk lies inside one segment or outside all, so its
// vectors are read whole before the segment is looked up.  kChainSome: the
// chunk looks up its segment first and reads its vectors only if the
// chained walk takes it (the per-item walk took the others).  kChainNone:
// nothing to do.
__device__ inline uint32_t chain_survey_of(const ChainGeo& g) {
  return __builtin_amdgcn_readfirstlane(*g.survey);
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

ChainGeo chain_geo(const Geometry& g, int v) {
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
  q.survey = g.chain_flag;
  return q;
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

// When the chained walk takes the call: sets g.chain_* so that the
// per-item walk launched first writes the flag word at the start of ws,
// clears the slots after it and leaves the chunk-aligned segments to it.
bool chain_share(Geometry& g, bool aln, int v, void* ws, int64_t ws_bytes,
                 bool bwd) {
  if (!chain_ready(g, aln, v, ws, ws_bytes, bwd)) return false;
  const int64_t kr = g.T / chain_elems(v);
  g.chain_ch = chain_elems(v);
  g.chain_flag = static_cast<uint32_t*>(ws);
  g.chain_slots = reinterpret_cast<u64*>(static_cast<char*>(ws) + kChainFlagBytes);
  g.chain_words = (chain_need(g.C, kr, g.nbranch) - kChainFlagBytes) /
                  static_cast<int64_t>(sizeof(u64));
  return true;
}

}  // namespace
}  // namespace asc

#endif  // ASC_CHAIN_COMMON_H
