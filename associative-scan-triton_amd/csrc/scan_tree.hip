// Tree walk: the single-pass walk over chunks of the flat array for problems
// with few (segment, channel) items (one long sequence, a handful of
// channels), where one wave or workgroup per item would leave most CUs idle.
//
// The flat array of all rows is cut into chunks of kTreeWaves (16) waves x
// kTreeU (2) sub-tiles: 8192 fp32 / 16384 fp16-bf16 elements, one
// workgroup per chunk in scan order, within 64 VGPRs so that two workgroups
// share a CU.  A chunk that lies inside one segment takes the chained
// walk's scan; one that holds segment or row boundaries (or a tensor end)
// takes per-element segment flags (tree_seg_flags) and the segmented scans
// of seg_common.h.
// Carries between chunks go through a tree of published maps in the
// caller's workspace:
//   * level 0: each chunk's map (A, X, F), F = a segment head lies inside
//     (then the map is an inclusive value), published right after its local
//     scan;
//   * level L >= 1: the map of a group of 64 level-(L-1) groups, published
//     by the last chunk of the group once it has composed them.
// The carry into chunk b composes, level by level from the bottom, the maps
// of b's earlier siblings (one DPP scan over at most 64 lanes per level) and
// stops at the nearest map with F = 1.  Which maps are composed, and in which
// order, is fixed by the data, not by timing, so the results are bitwise
// reproducible (the look-back walk uses whichever predecessor it meets
// first as inclusive, and its last bits vary); and since a group's map
// depends only on its members, no serial chain of carries forms (the
// chained walk's 64-chunk checkpoints wait for one another).
//
// Chunks are numbered by blockIdx and wait only for smaller ones.  Every
// wait is bounded (the spin limit of asc_set_lookback_spin_limit): a wave
// whose wait expires raises a flag in the workspace and its chunk stops
// (all its waves together, past the barrier that hands over the carry), as
// does every chunk that sees the flag when it polls; the workspace-free
// walk launched behind the tree kernel, which returns at once when the
// flag is clear, then recomputes the whole call.  Progress therefore never depends
// on the order in which workgroups are dispatched, at no register cost in
// the tree kernel (a fallback that recomputes a missing map inside it
// doubled its registers); numbering chunks by a ticket taken from an atomic
// counter at the workgroup's start instead cost 20% (one fp32 row of 2^27
// elements: 3.56 against 4.33 TB/s forward), the atomic's round trip delays
// every chunk's loads.

#include "chain_common.h"
#include "seg_common.h"

namespace asc {
namespace {

constexpr int kTreeMaxLevels = 4;        // up to 64^4 chunks per branch
constexpr int64_t kTreeFlagBytes = 256;  // workspace: the failure flag first
constexpr int kTreeFan = 64;
// Chunk shape: kTreeWaves waves x kTreeU sub-tiles.
#ifndef ASC_TREE_WAVES
#define ASC_TREE_WAVES 16
#endif
constexpr int kTreeWaves = ASC_TREE_WAVES;
#ifndef ASC_TREE_U
#define ASC_TREE_U 2
#endif
constexpr int kTreeU = ASC_TREE_U;  // sub-tiles per wave
constexpr int64_t kTreeChunkVec =
    static_cast<int64_t>(kTreeWaves) * kTreeU * kWave;  // vectors per chunk

struct TreeGeo {
  LbGeo g;             // segments, tensor, phase (its tile fields unused)
  int64_t nchunks;     // chunks per branch
  int levels;          // slot levels in use (the top one has <= 64 groups)
  int64_t off[kTreeMaxLevels];  // first slot of each level (per branch)
  int64_t per_branch;           // slots per branch
};

struct TreeFwdParams {
  TreeGeo t;
  FwdPtrs br[2];
  LbSlot* slots;
  uint32_t* fail;  // set when a wait expired (zeroed with the slots)
};

__device__ inline bool tree_failed(uint32_t* fail) {
  return __hip_atomic_load(fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
__device__ inline void tree_fail(uint32_t* fail) {
  __hip_atomic_store(fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Vector of (wave wv, sub-tile u, lane) in chunk b (scan order).
template <class IO, bool REV>
__device__ inline int64_t tree_vec(const LbGeo& g, int64_t b, int wv, int u,
                                   int lane) {
  const int64_t i = b * kTreeChunkVec +
                    static_cast<int64_t>(wv * kTreeU + u) * kWave + lane;
  return REV ? g.nvec - 1 - i : i;
}

// Chunk classification (uniform), as lb_classify for a tile: fast when every
// element of the chunk lies in one segment of one row; then phead / ptail
// are the segment's first / last element in scan order if they are the
// chunk's first / last element, else -1.
template <class IO, bool REV>
__device__ inline LbTile tree_classify(const LbGeo& g, int64_t b) {
  constexpr int V = IO::V;
  LbTile r{false, -1, -1, 0, 0, 0};
  const int64_t v_lo = REV ? g.nvec - (b + 1) * kTreeChunkVec : b * kTreeChunkVec;
  const int64_t e_lo = uniform(v_lo * V - g.phase);
  const int64_t e_hi = e_lo + kTreeChunkVec * V;
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
  const int64_t hd = REV ? ce - 1 : cs;
  const int64_t tl_ = REV ? cs : ce - 1;
  if (hd == (REV ? th - 1 : tl)) r.phead = base + hd;
  if (tl_ == (REV ? tl : th - 1)) r.ptail = base + tl_;
  return r;
}

// Whether chunk b lies inside the tensor (uniform): its vectors are then
// loaded without per-vector bounds checks, so that every load of the chunk
// goes out at once.
template <class IO, bool REV>
__device__ inline bool tree_whole(const LbGeo& g, int64_t b) {
  const int64_t v_lo = REV ? g.nvec - (b + 1) * kTreeChunkVec : b * kTreeChunkVec;
  return v_lo >= 0 && v_lo * IO::V - g.phase >= 0 &&
         (v_lo + kTreeChunkVec) * IO::V - g.phase <= g.n;
}

// Loads vector vi packed; elements outside the tensor read `ident`.
template <class IO>
__device__ inline uint4 tree_load(const char* origin, int64_t vi,
                                  uint32_t inten, float ident) {
  constexpr uint32_t full = (1u << IO::V) - 1;
  if (inten == full) return ld16(origin + vi * 16);
  float f[IO::V];
  lb_load<IO, true>(origin, vi, inten, ident, f);
  return IO::pack(f);
}

// A map (A, X, F) of the tree and its slot encoding: F = 1 is published as
// an inclusive value (A unused).
struct TreeMap {
  float a, x;
  int f;
};
__device__ inline void tree_publish(LbSlot* s, const TreeMap& m) {
  if (m.f) {
    lb_put(&s->x, kLbIncl, m.x);
  } else {
    lb_put(&s->a, kLbAgg, m.a);
    lb_put(&s->x, kLbAgg, m.x);
  }
}
// m then n (n covers the later elements).
__device__ inline TreeMap tree_then(const TreeMap& m, const TreeMap& n) {
  if (n.f) return n;
  return TreeMap{m.a * n.a, fmaf(n.a, m.x, n.x), m.f};
}

// Composition, in order, of level-L slots [base, base + n) (n <= 64; lane i
// reads slot base + i): waits until every slot after the last inclusive one
// is published and returns their composed map (F = 1 if an inclusive one
// was met).  A wait that runs past `spin` polls, or sees the failure flag,
// raises the flag and sets ok = false.  Called by one whole wave.
__device__ inline TreeMap tree_compose(LbSlot* lv, int64_t base, int n,
                                       int lane, uint32_t spin, uint32_t* fail,
                                       bool& ok) {
  const bool mine = lane < n;
  LbSlot* sl = lv + base + (mine ? lane : 0);
  float a = 1.0f, x = 0.0f;
  int kind = mine ? kLbNone : kLbAgg;
  for (uint32_t polls = 0;; ++polls) {
    if (kind == kLbNone) kind = lb_read(sl, a, x);
    const u64 incl = __builtin_amdgcn_ballot_w64(kind == kLbIncl);
    const int r = incl ? 63 - __builtin_clzll(incl) : -1;
    const u64 above = r >= 63 ? 0ull : (~0ull << (r + 1));
    if (!(__builtin_amdgcn_ballot_w64(kind == kLbNone) & above)) break;
    if (polls >= spin || tree_failed(fail)) {
      if (lane == 0) tree_fail(fail);
      ok = false;
      return TreeMap{1.0f, 0.0f, 0};
    }
    __builtin_amdgcn_s_sleep(2);
  }
  const u64 incl = __builtin_amdgcn_ballot_w64(kind == kLbIncl);
  const int r = incl ? 63 - __builtin_clzll(incl) : -1;
  float ma = a, mx = x;
  if (!mine || lane < r) {
    ma = 1.0f;
    mx = 0.0f;
  } else if (lane == r) {
    ma = 0.0f;
  }
  wave_scan_affine(ma, mx);
  TreeMap m;
  m.a = readlane(ma, n - 1);
  m.x = readlane(mx, n - 1);
  m.f = r >= 0 ? 1 : 0;
  return m;
}

// The tree's work for chunk b, by one whole wave once the chunk's own map m
// is known: publishes m (level 0) and the map of every group whose last
// chunk b is (when later chunks exist), and returns the carry into b when
// need_carry; ok = false when a wait failed (see tree_compose).
__device__ inline float tree_step(const TreeGeo& tg, LbSlot* slots, int64_t b,
                                  TreeMap m, bool need_carry, int lane,
                                  uint32_t* fail, bool& ok) {
  if (lane == 0) tree_publish(slots + tg.off[0] + b, m);
  const bool later = b + 1 < tg.nchunks;
  TreeMap acc{1.0f, 0.0f, 0};  // the carry's map, nearest levels first
  bool carry_done = !need_carry;
  bool pub = later;            // b is the last chunk of its level-L group
  int64_t i = b;               // b's group index at level L
  for (int L = 0; L < tg.levels; ++L) {
    const bool top = L + 1 == tg.levels;
    // b completes its level-(L+1) group: it publishes that group's map
    pub = pub && !top && ((i + 1) % kTreeFan == 0);
    if (carry_done && !pub) break;
    const int64_t base = top ? 0 : (i / kTreeFan) * kTreeFan;
    const int n = static_cast<int>(i - base);
    TreeMap sib{1.0f, 0.0f, 0};
    if (n > 0) {
      sib = tree_compose(slots + tg.off[L], base, n, lane, tg.g.spin_limit,
                         fail, ok);
      if (!ok) return 0.0f;
    }
    if (!carry_done) {
      acc = tree_then(sib, acc);
      if (sib.f) carry_done = true;
    }
    if (pub) {
      m = tree_then(sib, m);
      if (lane == 0) tree_publish(slots + tg.off[L + 1] + (i + 1) / kTreeFan - 1, m);
    }
    i /= kTreeFan;
  }
  return acc.x;  // applied to the state before the first element: 0
}

// Whether a wave's sub-tiles need the carry: unless the first element (scan
// order) that lies in a segment is a segment head (as lb_needs_carry).
template <class IO, bool REV>
__device__ inline bool tree_needs_carry(const uint32_t* valid,
                                        const uint32_t* head) {
  constexpr int V = IO::V;
#pragma unroll
  for (int u = 0; u < kTreeU; ++u) {
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

// Per-element flags of a wave's sub-tiles in a chunk that holds segment or
// row edges, bit j for memory index j of the lane's vector vi[u]: valid
// (inside the tensor and inside [cu[0], cu[S]) of its row), head / tail
// (first / last element of its segment in scan order).  The wave's element
// range is searched once (a uniform binary search over cu_seqlens, scalar
// loads), then the edges inside it are walked in a uniform loop in which
// every lane marks its own elements: a few scalar loads per edge instead of
// a search per lane through vector loads (measured on 4 ragged fp32 rows
// of 9M elements: 4.49 / 4.91 against 3.38 / 4.15 TB/s forward / backward;
// 2 ragged bf16 rows 3.33 / 3.66 against 2.25 / 2.98).
template <class IO, bool REV>
__device__ inline void tree_seg_flags(const LbGeo& g, int64_t b, int wv,
                                      const int64_t* vi, uint32_t* valid,
                                      uint32_t* head, uint32_t* tail) {
  constexpr int V = IO::V;
  constexpr int U = kTreeU;
  int64_t e0[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    valid[u] = head[u] = tail[u] = 0;
    e0[u] = vi[u] * V - g.phase;
  }
  const int64_t va = tree_vec<IO, REV>(g, b, wv, 0, 0);
  const int64_t vb = tree_vec<IO, REV>(g, b, wv, U - 1, kWave - 1);
  const int64_t vmin = va < vb ? va : vb, vmax = va < vb ? vb : va;
  const int64_t lo = uniform(vmin * V - g.phase < 0 ? 0 : vmin * V - g.phase);
  const int64_t hi =
      uniform((vmax + 1) * V - g.phase > g.n ? g.n : (vmax + 1) * V - g.phase);
  if (lo >= hi) return;
  const int64_t cu0 = uniform(lb_cu(g, 0)), cuS = uniform(lb_cu(g, g.S));
  for (int64_t r = uniform(lo / g.T); r * g.T < hi; ++r) {
    const int64_t rlo = r * g.T;
    const int64_t tl = lo - rlo > 0 ? lo - rlo : 0;
    const int64_t th = hi - rlo < g.T ? hi - rlo : g.T;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int64_t t = e0[u] + j - rlo;
        if (t >= tl && t < th && t >= cu0 && t < cuS) valid[u] |= 1u << j;
      }
    // edges p = cu[k] with p in [tl, th]: p starts segment k (k < S) and
    // p - 1 ends segment k - 1 (k >= 1)
    for (int64_t k = uniform(tl > 0 ? lb_find(g, tl - 1) + 1 : 0); k <= g.S;
         ++k) {
      const int64_t p = uniform(lb_cu(g, k));
      if (p > th) break;
      const bool starts = k < g.S && p >= tl && p < th && p >= cu0 && p < cuS;
      const bool ends =
          k >= 1 && p - 1 >= tl && p - 1 < th && p - 1 >= cu0 && p - 1 < cuS;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t d = rlo + p - e0[u];
        if (starts && d >= 0 && d < V) {
          if (REV) tail[u] |= 1u << d;
          else head[u] |= 1u << d;
        }
        if (ends && d - 1 >= 0 && d - 1 < V) {
          if (REV) head[u] |= 1u << (d - 1);
          else tail[u] |= 1u << (d - 1);
        }
      }
    }
  }
}

// ---- forward ----
struct TreePart {
  float a, x;
  int f;
  int flags;  // bit 1: some element lies in a segment; bit 0: needs a carry
};

// What wave 0 hands the other waves after the tree step: each wave's carry
// and whether every wait succeeded.
struct TreeMeet {
  float carry[kTreeWaves];
  int ok;
};

// Wave 0's work between the chunk's two barriers: the waves' maps (one per
// lane) are scanned across lanes, which gives the chunk's map (published by
// the tree step, which returns the carry into the chunk) and every wave's
// exclusive prefix, applied to that carry.  The chunk needs a carry unless
// the first wave holding an element of some segment starts with a head.
__device__ inline void tree_meet(const TreeGeo& tg, LbSlot* slots, int64_t b,
                                 const TreePart* parts, int lane,
                                 uint32_t* fail, TreeMeet* out) {
  TreePart q{1.0f, 0.0f, 0, 0};
  if (lane < kTreeWaves) q = parts[lane];
  const u64 any = __builtin_amdgcn_ballot_w64((q.flags & 2) != 0);
  const bool need =
      any && (__builtin_amdgcn_readlane(q.flags, __builtin_ctzll(any)) & 1);
  const SegScan s = seg_finish(q.a, q.x, q.f);
  bool ok = true;
  const float carry =
      tree_step(tg, slots, b, TreeMap{s.ta, s.tx, s.tf}, need, lane, fail, ok);
  if (lane < kTreeWaves) out->carry[lane] = seg_carry_in(s, carry);
  if (lane == 0) out->ok = ok ? 1 : 0;
}

// The local scan of one sub-tile: the chained walk's scan when the chunk
// lies in one segment, the per-element flags otherwise.
// (slow chunks: valid / head come from tree_seg_flags)
template <class IO, bool REV>
__device__ inline SegScan tree_fwd_sub(const LbTile& ti, int64_t vi, int wv,
                                       int u, const float* gf,
                                       const float* xf, uint32_t& valid,
                                       uint32_t& head) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  if (ti.fast) {
    valid = full;
    head = 0;
    const bool h0 = wv == 0 && u == 0;
    SubScan ss;
    if (h0)
      ss = fwd_local<IO, REV, true>(gf, xf, vi * V, ti.phead);
    else
      ss = fwd_local<IO, REV, false>(gf, xf, vi * V, -1);
    return seg_from(ss, h0 && ti.phead >= 0);
  }
  return fwd_local_seg<IO, REV>(gf, xf, valid, head);
}

// One chunk of the forward: the loads (tensor bounds only) go out before
// the segment lookup; the chunk's waves scan their sub-tiles, meet in LDS,
// wave 0 runs the tree step, and every wave applies its carry and stores.
template <class IO, bool REV>
__device__ inline void tree_fwd_chunk(const TreeFwdParams& p, int br,
                                      int64_t b, int lane, int wv,
                                      TreePart* parts, TreeMeet* meet) {
  constexpr int V = IO::V;
  constexpr int U = kTreeU;
  const LbGeo& g = p.t.g;
  const FwdPtrs& q = p.br[br];
  uint4 gq[U], xq[U];
  int64_t vi[U];
#pragma unroll
  for (int u = 0; u < U; ++u) vi[u] = tree_vec<IO, REV>(g, b, wv, u, lane);
  if (tree_whole<IO, REV>(g, b)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      gq[u] = ld16(q.g + vi[u] * 16);
      xq[u] = ld16(q.x + vi[u] * 16);
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t inten = lb_inten<IO>(g, vi[u]);
      gq[u] = tree_load<IO>(q.g, vi[u], inten, 1.0f);
      xq[u] = tree_load<IO>(q.x, vi[u], inten, 0.0f);
    }
  }
  const LbTile ti = tree_classify<IO, REV>(g, b);
  SegScan sc[U];
  uint32_t valid[U], head[U];
  if (!ti.fast) {
    uint32_t tail[U];
    tree_seg_flags<IO, REV>(g, b, wv, vi, valid, head, tail);
  }
  TreeMap wm{1.0f, 0.0f, 0};
  uint32_t anyv = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float gf[V], xf[V];
    IO::unpack(gq[u], gf);
    IO::unpack(xq[u], xf);
    sc[u] = tree_fwd_sub<IO, REV>(ti, vi[u], wv, u, gf, xf, valid[u], head[u]);
    anyv |= valid[u];
    lb_compose(wm.a, wm.x, wm.f, sc[u].ta, sc[u].tx, sc[u].tf);
  }
  bool need_w;
  if (ti.fast) {
    need_w = ti.phead < 0;
  } else {
    need_w = tree_needs_carry<IO, REV>(valid, head);
  }
  const bool any_w = __builtin_amdgcn_ballot_w64(anyv != 0) != 0;
  if (lane == 0)
    parts[wv] = TreePart{wm.a, wm.x, wm.f, (any_w ? 2 : 0) | (need_w ? 1 : 0)};
  __syncthreads();
  if (wv == 0)
    tree_meet(p.t, p.slots + br * p.t.per_branch, b, parts, lane, p.fail, meet);
  __syncthreads();
  // a failed wait: the workspace-free walk behind this launch recomputes
  // the call
  if (!meet->ok) return;
  float c = meet->carry[wv];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float gf[V], xf[V], hf[V];
    repack_point<IO>(gq[u]);
    repack_point<IO>(xq[u]);
    IO::unpack(gq[u], gf);
    IO::unpack(xq[u], xf);
    if (ti.fast) {
      const SubScan ss{sc[u].ea, sc[u].ex, sc[u].ta, sc[u].tx};
      if (wv == 0 && u == 0)
        fwd_apply<IO, REV, true>(gf, xf, vi[u] * V, ti.phead, ss, c, hf);
      else
        fwd_apply<IO, REV, false>(gf, xf, vi[u] * V, -1, ss, c, hf);
      st16(q.h + vi[u] * 16, IO::pack(hf));
    } else {
      fwd_apply_seg<IO, REV>(gf, xf, valid[u], head[u], sc[u], c, hf);
      lb_store<IO, true>(q.h, vi[u], valid[u], hf);
    }
    c = seg_apply_total(sc[u].ta, sc[u].tx, sc[u].tf, c);
  }
}

// DIRS: 1 = causal, 2 = reverse (one branch per launch).
template <class IO, int DIRS>
__global__ void __launch_bounds__(kTreeWaves* kWave, 8)
    k_scan_fwd_tree(TreeFwdParams p) {
  __shared__ TreePart parts[kTreeWaves];
  __shared__ TreeMeet meet;
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  tree_fwd_chunk<IO, DIRS == 2>(p, 0, blockIdx.x, lane, wv, parts, &meet);
}

// ---- backward (B order: RB = the forward was causal) ----
struct TreeBwdParams {
  TreeGeo t;
  BwdPtrs br[2];
  int64_t dy_rs[2];  // DYC: element stride between rows of each gradient
  LbSlot* slots;
  uint32_t* fail;
};

// DYC: the gradients of vector vi's elements (one value per row, read
// through the rows' stride; 0 outside the tensor), packed like a loaded
// vector.
template <class IO>
__device__ inline uint4 tree_dyc_vec(const char* dy, int64_t rs,
                                     const LbGeo& g, const LbTile& ti,
                                     int64_t vi) {
  constexpr int V = IO::V;
  float f[V];
  const int64_t e0 = vi * V - g.phase;
  // row and row offset of element 0 (offsets from the chunk's first
  // in-tensor element stay far below 2^31)
  int64_t row = ti.c0;
  int32_t rem = ti.t0 + static_cast<int32_t>(e0 - ti.ebase);
  const int32_t T = static_cast<int32_t>(g.T);
  if (rem >= T) {
    row += rem / T;
    rem %= T;
  }
#pragma unroll
  for (int j = 0; j < V; ++j) {
    if (j > 0 && ++rem == T) {
      rem = 0;
      ++row;
    }
    const int64_t e = e0 + j;
    f[j] = (e >= 0 && e < g.n) ? IO::load1(dy + row * rs * IO::ES) : 0.0f;
  }
  return IO::pack(f);
}

// One chunk of the backward, as tree_fwd_chunk: every wave loads its
// sub-tiles and two halos (the gate just before its first element in B
// order, 1 outside the tensor, and the state just past its last one, 0
// outside), the shifted gates and states cross lanes by DPP and sub-tiles
// by readlane, and segment heads and tails reset them exactly.
// HL: the loaded states wait for the carry in LDS (hl: kTreeWaves * kTreeU
// * 64 vectors), not in registers: fp16 / bf16 chunks then fit 64 VGPRs,
// two workgroups per CU.
// DYC: the gradient is one value per row (dy_rs), constant along time.
template <class IO, bool RB, bool HL, bool DYC>
__device__ inline void tree_bwd_chunk(const TreeBwdParams& p, int br,
                                      int64_t b, int lane, int wv,
                                      TreePart* parts, TreeMeet* meet,
                                      uint4* hl) {
  constexpr int V = IO::V;
  constexpr int U = kTreeU;
  constexpr uint32_t full = (1u << V) - 1;
  constexpr int jl = mem_idx<V, RB>(V - 1);  // last element in B order
  constexpr int jf = mem_idx<V, RB>(0);      // first element in B order
  const LbGeo& g = p.t.g;
  const BwdPtrs& q = p.br[br];
  uint4 yq[U], gq[U], hq[U];
  int64_t vi[U];
#pragma unroll
  for (int u = 0; u < U; ++u) vi[u] = tree_vec<IO, RB>(g, b, wv, u, lane);
  if (tree_whole<IO, RB>(g, b)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!DYC) yq[u] = ld16(q.dy + vi[u] * 16);
      gq[u] = ld16(q.g + vi[u] * 16);
      hq[u] = ld16(q.h + vi[u] * 16);
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t inten = lb_inten<IO>(g, vi[u]);
      if (!DYC) yq[u] = tree_load<IO>(q.dy, vi[u], inten, 0.0f);
      gq[u] = tree_load<IO>(q.g, vi[u], inten, 1.0f);
      hq[u] = tree_load<IO>(q.h, vi[u], inten, 0.0f);
    }
  }
  if (HL) {
#pragma unroll
    for (int u = 0; u < U; ++u) hl[(wv * U + u) * kWave + lane] = hq[u];
  }
  float cg = 1.0f, hn = 0.0f;
  {
    const int64_t pf = tree_vec<IO, RB>(g, b, wv, 0, 0) * V + jf;
    const int64_t pp = RB ? pf + 1 : pf - 1;
    if (pp - g.phase >= 0 && pp - g.phase < g.n) cg = IO::load1(q.g + pp * IO::ES);
    const int64_t pl = tree_vec<IO, RB>(g, b, wv, U - 1, kWave - 1) * V + jl;
    const int64_t pn = RB ? pl - 1 : pl + 1;
    if (pn - g.phase >= 0 && pn - g.phase < g.n) hn = IO::load1(q.h + pn * IO::ES);
  }
  const LbTile ti = tree_classify<IO, RB>(g, b);
  // DYC: a fast chunk lies in one row and reads its one gradient value;
  // other chunks read one per element
  float dyv = 0.0f;
  if (DYC) {
    if (ti.fast) {
      dyv = IO::load1(q.dy + ti.c0 * p.dy_rs[br] * IO::ES);
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u)
        yq[u] = tree_dyc_vec<IO>(q.dy, p.dy_rs[br], g, ti, vi[u]);
    }
  }
  auto unpack_y = [&](int u, float* y) {
    if (DYC && ti.fast) {
#pragma unroll
      for (int e = 0; e < V; ++e) y[e] = dyv;
    } else {
      IO::unpack(yq[u], y);
    }
  };
  // the fast path masks the chunk's first sub-tile (segment head) and its
  // last one (segment tail)
  auto masked = [&](int u) {
    return (wv == 0 && u == 0) || (wv == kTreeWaves - 1 && u == U - 1);
  };
  SegScan sc[U];
  uint32_t valid[U], head[U], tail[U];
  if (!ti.fast) tree_seg_flags<IO, RB>(g, b, wv, vi, valid, head, tail);
  float gprv[U];
  TreeMap wm{1.0f, 0.0f, 0};
  uint32_t anyv = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float gf[V], yf[V];
    IO::unpack(gq[u], gf);
    unpack_y(u, yf);
    if (ti.fast) {
      valid[u] = full;
      head[u] = 0;
      tail[u] = 0;
      SubScan ss;
      if (masked(u))
        ss = bwd_local<IO, RB, true>(gf, yf, vi[u] * V, ti.phead, cg, gprv[u]);
      else
        ss = bwd_local<IO, RB, false>(gf, yf, vi[u] * V, -1, cg, gprv[u]);
      sc[u] = seg_from(ss, wv == 0 && u == 0 && ti.phead >= 0);
    } else {
      sc[u] = bwd_local_seg<IO, RB>(gf, yf, valid[u], head[u], cg, gprv[u]);
    }
    cg = readlane(gf[jl], kWave - 1);
    anyv |= valid[u];
    lb_compose(wm.a, wm.x, wm.f, sc[u].ta, sc[u].tx, sc[u].tf);
  }
  const bool need_w =
      ti.fast ? ti.phead < 0 : tree_needs_carry<IO, RB>(valid, head);
  const bool any_w = __builtin_amdgcn_ballot_w64(anyv != 0) != 0;
  if (lane == 0)
    parts[wv] = TreePart{wm.a, wm.x, wm.f, (any_w ? 2 : 0) | (need_w ? 1 : 0)};
  __syncthreads();
  if (wv == 0)
    tree_meet(p.t, p.slots + br * p.t.per_branch, b, parts, lane, p.fail, meet);
  __syncthreads();
  if (!meet->ok) return;
  float c = meet->carry[wv];
  // dx first, then dg = (shifted state) * dx with the states unpacked only
  // then: g, dy and h are never unpacked at once
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float gf[V], yf[V], dx[V];
    repack_point<IO>(gq[u]);
    if (!(DYC && ti.fast)) repack_point<IO>(yq[u]);
    IO::unpack(gq[u], gf);
    unpack_y(u, yf);
    uint32_t vd = valid[u], hd = head[u], tl = tail[u];
    if (ti.fast) {  // the segment's head and tail inside the chunk, if any
      vd = full;
      hd = (ti.phead >= 0 && wv == 0 && u == 0 && lane == 0) ? 1u << jf : 0u;
      tl = (ti.ptail >= 0 && wv == kTreeWaves - 1 && u == U - 1 &&
            lane == kWave - 1) ? 1u << jl : 0u;
    }
    float d = seg_carry_in(sc[u], c);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int j = mem_idx<V, RB>(i);
      const float gs = (i == 0) ? gprv[u] : gf[mem_idx<V, RB>(i - 1)];
      if (vd & (1u << j)) d = (hd & (1u << j)) ? yf[j] : fmaf(gs, d, yf[j]);
      dx[j] = d;
    }
    if (ti.fast) st16(q.dx + vi[u] * 16, IO::pack(dx));
    else lb_store<IO, true>(q.dx, vi[u], vd, dx);
    uint4 hv, hw;
    if (HL) {
      hv = hl[(wv * U + u) * kWave + lane];
      if (u + 1 < U) hw = hl[(wv * U + u + 1) * kWave];
    } else {
      repack_point<IO>(hq[u]);
      hv = hq[u];
      if (u + 1 < U) hw = hq[u + 1 < U ? u + 1 : u];
    }
    float hf[V], dg[V];
    IO::unpack(hv, hf);
    float hin = hn;
    if (u + 1 < U) {
      float hnext[V];
      IO::unpack(hw, hnext);
      hin = HL ? hnext[jf] : readlane(hnext[jf], 0);
    }
    const float hnx = dpp<kWaveShl1, 0xf>(hin, hf[jf]);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int j = mem_idx<V, RB>(i);
      float hs = (i == V - 1) ? hnx : hf[mem_idx<V, RB>(i + 1)];
      if (tl & (1u << j)) hs = 0.0f;
      dg[j] = hs * dx[j];
    }
    if (ti.fast) st16(q.dg + vi[u] * 16, IO::pack(dg));
    else lb_store<IO, true>(q.dg, vi[u], vd, dg);
    c = seg_apply_total(sc[u].ta, sc[u].tx, sc[u].tf, c);
  }
}

// DIRS: the forward scan's direction (1 = causal: B order reverse).
#ifndef ASC_TREE_BWD_HL
#define ASC_TREE_BWD_HL 1
#endif
template <class IO>
constexpr bool TreeHl = ASC_TREE_BWD_HL && IO::V != 4;
template <class IO, int DIRS, bool DYC>
__global__ void __launch_bounds__(kTreeWaves* kWave, TreeHl<IO> || IO::V == 4 ? 8 : 6)
    k_scan_bwd_tree(TreeBwdParams p) {
  __shared__ TreePart parts[kTreeWaves];
  __shared__ TreeMeet meet;
  __shared__ uint4 hl[TreeHl<IO> ? kTreeWaves * kTreeU * kWave : 1];
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  tree_bwd_chunk<IO, DIRS == 1, TreeHl<IO>, DYC>(p, 0, blockIdx.x, lane, wv,
                                                 parts, &meet, hl);
}

template <class IO>
const void* pick_bwd_tree(int dirs, bool dyc) {
  if (dyc)
    return dirs == 1 ? reinterpret_cast<const void*>(&k_scan_bwd_tree<IO, 1, true>)
                     : reinterpret_cast<const void*>(&k_scan_bwd_tree<IO, 2, true>);
  return dirs == 1 ? reinterpret_cast<const void*>(&k_scan_bwd_tree<IO, 1, false>)
                   : reinterpret_cast<const void*>(&k_scan_bwd_tree<IO, 2, false>);
}

template <class IO>
const void* pick_fwd_tree(int dirs) {
  return dirs == 1 ? reinterpret_cast<const void*>(&k_scan_fwd_tree<IO, 1>)
                   : reinterpret_cast<const void*>(&k_scan_fwd_tree<IO, 2>);
}

// Slot levels of the tree for nchunks chunks: level L holds
// ceil(nchunks / 64^L) maps; the top level is the first with at most 64.
TreeGeo tree_geo(const Geometry& geo, int v, uint32_t spin) {
  TreeGeo t{};
  t.g = LbGeo{geo.cu, geo.cu64, geo.S, geo.C, geo.T, geo.C * geo.T, geo.phase,
              0, 0, 1, spin};
  t.g.nvec = (t.g.phase + t.g.n + v - 1) / v;
  t.nchunks = (t.g.nvec + kTreeChunkVec - 1) / kTreeChunkVec;
  int64_t cnt = t.nchunks, off = 0;
  t.levels = 0;
  while (true) {
    t.off[t.levels++] = off;
    off += cnt;
    if (cnt <= kTreeFan || t.levels == kTreeMaxLevels) break;
    cnt = (cnt + kTreeFan - 1) / kTreeFan;
  }
  t.per_branch = off;
  return t;
}

}  // namespace

// The tree walk's workspace for n elements per branch (the worst-case
// phase), 0 when it cannot run (more chunks than its levels or one grid
// hold).
int64_t tree_bytes(int64_t n, int v, int nbranch) {
  Geometry geo{};
  geo.C = 1;
  geo.T = n;
  geo.phase = v - 1;
  const TreeGeo t = tree_geo(geo, v, 0);
  if (t.nchunks > kMaxGrid) return 0;
  int64_t top = t.nchunks;
  for (int L = 1; L < t.levels; ++L) top = (top + kTreeFan - 1) / kTreeFan;
  if (top > kTreeFan) return 0;
  return kTreeFlagBytes +
         t.per_branch * nbranch * static_cast<int64_t>(sizeof(LbSlot));
}

namespace {

// Host side of both directions: checks that the tree can run with this
// workspace, zeroes the flag and the slots, and launches one grid per
// branch (the branches share the failure flag).
// dy_rs: the backward's row strides (DYC), else nullptr.
template <class TP, class BP, class Pick>
bool tree_launch(const Geometry& geo, const BP* br, const int64_t* dy_rs,
                 int dtype, int dirs, bool aln, void* ws, int64_t ws_bytes,
                 void* stream, int& status, const uint32_t** fail, Pick pick) {
  if (!aln || !ws || reinterpret_cast<uintptr_t>(ws) % 32 != 0) return false;
  const int v = 16 / elem_size(dtype);
  TP q{};
  q.t = tree_geo(geo, v, lb_spin_limit());
  int64_t top = q.t.nchunks;
  for (int L = 1; L < q.t.levels; ++L) top = (top + kTreeFan - 1) / kTreeFan;
  if (q.t.nchunks > kMaxGrid || top > kTreeFan) return false;
  const int64_t need =
      kTreeFlagBytes +
      q.t.per_branch * geo.nbranch * static_cast<int64_t>(sizeof(LbSlot));
  if (ws_bytes < need) return false;
  q.slots = reinterpret_cast<LbSlot*>(static_cast<char*>(ws) + kTreeFlagBytes);
  q.fail = static_cast<uint32_t*>(ws);
  if ((status = fill_zero(ws, need, stream))) return true;
  *fail = q.fail;
  for (int b = 0; b < geo.nbranch; ++b) {
    TP r = q;
    r.br[0] = br[b];
    if constexpr (std::is_same_v<TP, TreeBwdParams>) r.dy_rs[0] = dy_rs[b];
    r.slots = q.slots + b * q.t.per_branch;
    const int d = dirs == 3 ? (b == 0 ? 1 : 2) : dirs;
    if ((status = launch(pick(dtype, d), r.t.nchunks, kTreeWaves, r, stream)))
      return true;
  }
  return true;
}

}  // namespace

bool tree_fwd(const FwdParams& p, int dtype, int dirs, bool aln, void* ws,
              int64_t ws_bytes, void* stream, int& status,
              const uint32_t** fail) {
  return tree_launch<TreeFwdParams>(
      p.geo, p.br, nullptr, dtype, dirs, aln, ws, ws_bytes, stream, status, fail,
      [](int dt, int d) {
        switch (dt) {
          case ASC_F32: return pick_fwd_tree<IoF32>(d);
          case ASC_F16: return pick_fwd_tree<IoF16>(d);
          default: return pick_fwd_tree<IoBF16>(d);
        }
      });
}

bool tree_bwd(const BwdParams& p, int dtype, int dirs, bool aln, bool dyc,
              void* ws, int64_t ws_bytes, void* stream, int& status,
              const uint32_t** fail) {
  return tree_launch<TreeBwdParams>(
      p.geo, p.br, p.dy_rs, dtype, dirs, aln, ws, ws_bytes, stream, status,
      fail, [dyc](int dt, int d) {
        switch (dt) {
          case ASC_F32: return pick_bwd_tree<IoF32>(d, dyc);
          case ASC_F16: return pick_bwd_tree<IoF16>(d, dyc);
          default: return pick_bwd_tree<IoBF16>(d, dyc);
        }
      });
}

}  // namespace asc
