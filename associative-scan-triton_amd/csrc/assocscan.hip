// libassocscan: gfx950 kernels and C ABI for the first-order linear
// recurrence h[t] = g[t]*h[t-1] + x[t] over packed segments.
//
// Design (one wavefront per (segment, channel) pair, no LDS, no barriers):
//   * A segment of one row is walked in "sub-tiles" of 64 x 16 bytes: lane l
//     owns one 16-byte vector (4 fp32 or 8 fp16/bf16 elements), so every
//     global load/store instruction of the wave covers 1 KiB contiguously
//     (global_load_dwordx4).  Vectors are aligned in memory; a segment start
//     or end that falls inside a vector is handled by per-element masking on
//     the first and last sub-tile only.
//   * Inside a sub-tile: each lane scans its own elements serially, the 64
//     lane aggregates are combined by an inclusive DPP scan (row_shr 1/2/4/8,
//     row_bcast 15/31), the exclusive prefix is taken with wave_shr:1, and the
//     lane re-walks its elements from its prefix.  The carry between
//     sub-tiles is a wave-uniform register, so each element is read once and
//     written once.
//   * Scan elements are affine maps m = (A, X): h -> A*h + X.  Composition
//     "left then right" is (Al, Xl) then (Ar, Xr) = (Ar*Al, Ar*Xl + Xr); this
//     is the reference combine op (_kernels.py:6-16).  Identity is (1, 0).
//   * Accumulation is fp32 for every storage type; fp16/bf16 are converted
//     on load and rounded to nearest-even on store.
//   * Segment heads are exact: h[start] = x[start] and dx[end-1] = dy[end-1]
//     bit for bit (a select, never a multiply of the carry by zero).
//
// Reference semantics followed: _kernels.py:19-81 and :84-168 (forward,
// reverse indexing :55-58, gate product :74-76, in-place :77-81) and
// _kernels.py:171-287 / :290-374 (fused backward with shifted gates and
// states, pads 1.0 / 0.0 at segment edges :232-247, :266-283).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "assocscan.h"

#ifndef ASC_WAVES_PER_BLOCK
#define ASC_WAVES_PER_BLOCK 1
#endif
#ifndef ASC_FWD_UNROLL
#define ASC_FWD_UNROLL 4
#endif
#ifndef ASC_BWD_UNROLL
#define ASC_BWD_UNROLL 2
#endif

namespace {

constexpr int kWave = 64;
constexpr int kWPB = ASC_WAVES_PER_BLOCK;

// ---------------------------------------------------------------------------
// Storage types.  V elements per 16-byte vector; ES bytes per element.
// ---------------------------------------------------------------------------
struct IoF32 {
  static constexpr int V = 4;
  static constexpr int ES = 4;
  __device__ static inline void unpack(const uint4& q, float* f) {
    f[0] = __uint_as_float(q.x);
    f[1] = __uint_as_float(q.y);
    f[2] = __uint_as_float(q.z);
    f[3] = __uint_as_float(q.w);
  }
  __device__ static inline uint4 pack(const float* f) {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]),
                      __float_as_uint(f[2]), __float_as_uint(f[3]));
  }
  __device__ static inline float load1(const char* p) {
    return *reinterpret_cast<const float*>(p);
  }
  __device__ static inline void store1(char* p, float v) {
    *reinterpret_cast<float*>(p) = v;
  }
};

__device__ inline float h2f(uint32_t bits16) {
  return static_cast<float>(
      __builtin_bit_cast(_Float16, static_cast<unsigned short>(bits16)));
}
__device__ inline uint32_t f2h(float f) {
  return __builtin_bit_cast(unsigned short, static_cast<_Float16>(f));
}
__device__ inline float b2f(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ inline uint32_t f2b(float f) {
  // gfx950 converts with round-to-nearest-even (v_cvt_pk_bf16_f32).
  return __builtin_bit_cast(unsigned short, static_cast<__bf16>(f));
}

template <float (*CVT)(uint32_t), uint32_t (*RND)(float)>
struct IoHalf {
  static constexpr int V = 8;
  static constexpr int ES = 2;
  __device__ static inline void unpack(const uint4& q, float* f) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = CVT(w[i] & 0xffffu);
      f[2 * i + 1] = CVT(w[i] >> 16);
    }
  }
  __device__ static inline uint4 pack(const float* f) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = RND(f[2 * i]) | (RND(f[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ static inline float load1(const char* p) {
    return CVT(*reinterpret_cast<const unsigned short*>(p));
  }
  __device__ static inline void store1(char* p, float v) {
    *reinterpret_cast<unsigned short*>(p) = static_cast<unsigned short>(RND(v));
  }
};
using IoF16 = IoHalf<h2f, f2h>;
using IoBF16 = IoHalf<b2f, f2b>;

// ---------------------------------------------------------------------------
// Cross-lane primitives (DPP).  update_dpp leaves `old` in lanes whose source
// lane is out of range or whose row is masked off, so passing the identity
// as `old` makes those lanes combine with the identity.
// ---------------------------------------------------------------------------
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114,
              kRowShr8 = 0x118, kWaveShl1 = 0x130, kWaveShr1 = 0x138,
              kRowBcast15 = 0x142, kRowBcast31 = 0x143;

template <int CTRL, int ROWMASK>
__device__ inline float dpp(float old, float src) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      __float_as_int(old), __float_as_int(src), CTRL, ROWMASK, 0xf, false));
}

__device__ inline float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

template <int CTRL, int ROWMASK>
__device__ inline void affine_step(float& a, float& x) {
  const float as = dpp<CTRL, ROWMASK>(1.0f, a);
  const float xs = dpp<CTRL, ROWMASK>(0.0f, x);
  x = fmaf(a, xs, x);
  a = a * as;
}

// Inclusive scan of affine maps over the 64 lanes (lane 0 first).
__device__ inline void wave_scan_affine(float& a, float& x) {
  affine_step<kRowShr1, 0xf>(a, x);
  affine_step<kRowShr2, 0xf>(a, x);
  affine_step<kRowShr4, 0xf>(a, x);
  affine_step<kRowShr8, 0xf>(a, x);
  affine_step<kRowBcast15, 0xa>(a, x);
  affine_step<kRowBcast31, 0xc>(a, x);
}

template <int CTRL, int ROWMASK>
__device__ inline void mul_step(float& p) {
  p = p * dpp<CTRL, ROWMASK>(1.0f, p);
}

// Inclusive product scan over the 64 lanes.
__device__ inline void wave_scan_mul(float& p) {
  mul_step<kRowShr1, 0xf>(p);
  mul_step<kRowShr2, 0xf>(p);
  mul_step<kRowShr4, 0xf>(p);
  mul_step<kRowShr8, 0xf>(p);
  mul_step<kRowBcast15, 0xa>(p);
  mul_step<kRowBcast31, 0xc>(p);
}

// ---------------------------------------------------------------------------
// Geometry of one (segment, channel) work item.
//
// Positions P live in a per-call "phase" frame: P = c*T + t + phase, where
// phase = (address / ES) mod V is shared by all tensors of the call, so that
// vector vi = P / V starts at the 16-byte aligned address origin + 16*vi
// (origin = tensor base - phase*ES).  With ALN == false (tensors with
// different phases) phase is 0 and every access is a scalar access.
// ---------------------------------------------------------------------------
template <class IO, bool REV>
struct Walk {
  int64_t P0, P1;  // element range [P0, P1), P1 > P0
  int64_t v0, v1;  // first / last vector (inclusive)
  int64_t nv;      // number of vectors
  int64_t nsub;    // number of 64-vector sub-tiles
  int64_t kfast;   // sub-tiles [1, kfast) are interior (no masking)

  __device__ inline Walk(int64_t p0, int64_t p1) : P0(p0), P1(p1) {
    constexpr int V = IO::V;
    v0 = P0 / V;
    v1 = (P1 - 1) / V;
    nv = v1 - v0 + 1;
    nsub = (nv + kWave - 1) / kWave;
    const bool tail_partial = REV ? (P0 % V) != 0 : (P1 % V) != 0;
    const bool last_edge = (nv % kWave) != 0 || tail_partial;
    kfast = nsub - (last_edge ? 1 : 0);
    if (kfast < 1) kfast = 1;
  }
  // Vector owned by `lane` in sub-tile k (scan order: lane 0 first).
  __device__ inline int64_t vec(int64_t k, int lane) const {
    const int64_t i = k * kWave + lane;
    return REV ? v1 - i : v0 + i;
  }
  __device__ inline bool lane_valid(int64_t k, int lane) const {
    return k * kWave + lane < nv;
  }
  // First / last element in scan order.
  __device__ inline int64_t head() const { return REV ? P1 - 1 : P0; }
  __device__ inline int64_t tail() const { return REV ? P0 : P1 - 1; }
};

// Memory index (0..V-1) of the i-th element of a vector in scan order.
template <int V, bool REV>
__device__ constexpr int mem_idx(int i) {
  return REV ? V - 1 - i : i;
}

// Loads one vector of `origin` for the given lane into f[] (memory order).
// MASKED: elements outside [P0, P1) (or an invalid lane) read `ident`.
template <class IO, bool ALN, bool MASKED>
__device__ inline void load_vec(const char* origin, int64_t vi, bool lane_ok,
                                int64_t P0, int64_t P1, float ident,
                                float* f) {
  constexpr int V = IO::V;
  const int64_t pv = vi * V;
  if (!MASKED) {
    if (ALN) {
      IO::unpack(*reinterpret_cast<const uint4*>(origin + vi * 16), f);
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) f[j] = IO::load1(origin + (pv + j) * IO::ES);
    }
    return;
  }
  const bool full = lane_ok && pv >= P0 && pv + V <= P1;
  if (ALN && full) {
    IO::unpack(*reinterpret_cast<const uint4*>(origin + vi * 16), f);
    return;
  }
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int64_t p = pv + j;
    float v = ident;
    if (lane_ok && p >= P0 && p < P1) v = IO::load1(origin + p * IO::ES);
    f[j] = v;
  }
}

// Stores one vector (memory order); MASKED skips elements outside [P0, P1).
template <class IO, bool ALN, bool MASKED>
__device__ inline void store_vec(char* origin, int64_t vi, bool lane_ok,
                                 int64_t P0, int64_t P1, const float* f) {
  constexpr int V = IO::V;
  const int64_t pv = vi * V;
  if (!MASKED) {
    if (ALN) {
      *reinterpret_cast<uint4*>(origin + vi * 16) = IO::pack(f);
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) IO::store1(origin + (pv + j) * IO::ES, f[j]);
    }
    return;
  }
  const bool full = lane_ok && pv >= P0 && pv + V <= P1;
  if (ALN && full) {
    *reinterpret_cast<uint4*>(origin + vi * 16) = IO::pack(f);
    return;
  }
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int64_t p = pv + j;
    if (lane_ok && p >= P0 && p < P1) IO::store1(origin + p * IO::ES, f[j]);
  }
}

// ---------------------------------------------------------------------------
// Forward scan of one (segment, channel) item.
// ---------------------------------------------------------------------------
struct FwdPtrs {
  const char* g;  // origins (see Walk)
  const char* x;
  char* h;
  char* a;        // gate-product output origin, or nullptr
};

// One sub-tile: g, x in memory order (already masked to the identity when
// MASKED); writes h (and the gate product when WA) in memory order.
template <class IO, bool REV, bool MASKED, bool WA>
__device__ inline void fwd_subtile(const float* g, const float* x, int64_t pv,
                                   int64_t phead, float& carry, float& carry_a,
                                   float* hout, float* aout) {
  constexpr int V = IO::V;
  // 1. serial scan of the lane's own elements -> lane map (A, X)
  float A = 1.0f, X = 0.0f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, REV>(i);
    if (MASKED && pv + j == phead) {
      A = 0.0f;
      X = x[j];
    } else if (i == 0 && !MASKED) {
      A = g[j];
      X = x[j];
    } else {
      X = fmaf(g[j], X, x[j]);
      A = A * g[j];
    }
  }
  // 2. wave scan of lane maps; 3. exclusive prefix applied to the carry
  wave_scan_affine(A, X);
  const float ta = readlane(A, kWave - 1);
  const float tx = readlane(X, kWave - 1);
  const float ea = dpp<kWaveShr1, 0xf>(1.0f, A);
  const float ex = dpp<kWaveShr1, 0xf>(0.0f, X);
  float hh = fmaf(ea, carry, ex);
  // 4. re-walk
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, REV>(i);
    if (MASKED && pv + j == phead)
      hh = x[j];
    else
      hh = fmaf(g[j], hh, x[j]);
    hout[j] = hh;
  }
  carry = fmaf(ta, carry, tx);
  if (WA) {
    float p = 1.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) p = p * g[j];
    wave_scan_mul(p);
    const float tp = readlane(p, kWave - 1);
    float ap = carry_a * dpp<kWaveShr1, 0xf>(1.0f, p);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int j = mem_idx<V, REV>(i);
      ap = ap * g[j];
      aout[j] = ap;
    }
    carry_a = carry_a * tp;
  }
}

template <class IO, bool REV, bool ALN, bool WA, bool MASKED, int NS>
__device__ inline void fwd_block(const FwdPtrs& t, const Walk<IO, REV>& w,
                                 int64_t k0, int lane, float& carry,
                                 float& carry_a) {
  constexpr int V = IO::V;
  float g[NS][V], x[NS][V];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int64_t vi = w.vec(k0 + u, lane);
    const bool ok = !MASKED || w.lane_valid(k0 + u, lane);
    load_vec<IO, ALN, MASKED>(t.g, vi, ok, w.P0, w.P1, 1.0f, g[u]);
    load_vec<IO, ALN, MASKED>(t.x, vi, ok, w.P0, w.P1, 0.0f, x[u]);
  }
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int64_t vi = w.vec(k0 + u, lane);
    const bool ok = !MASKED || w.lane_valid(k0 + u, lane);
    float h[V], a[V];
    fwd_subtile<IO, REV, MASKED, WA>(g[u], x[u], vi * V, w.head(), carry,
                                     carry_a, h, a);
    store_vec<IO, ALN, MASKED>(t.h, vi, ok, w.P0, w.P1, h);
    if (WA) store_vec<IO, ALN, MASKED>(t.a, vi, ok, w.P0, w.P1, a);
  }
}

template <class IO, bool REV, bool ALN, bool WA>
__device__ void fwd_item(const FwdPtrs& t, int64_t P0, int64_t P1, int lane) {
  constexpr int U = ASC_FWD_UNROLL;
  const Walk<IO, REV> w(P0, P1);
  float carry = 0.0f, carry_a = 1.0f;
  fwd_block<IO, REV, ALN, WA, true, 1>(t, w, 0, lane, carry, carry_a);
  int64_t k = 1;
  for (; k + U <= w.kfast; k += U)
    fwd_block<IO, REV, ALN, WA, false, U>(t, w, k, lane, carry, carry_a);
  for (; k < w.kfast; ++k)
    fwd_block<IO, REV, ALN, WA, false, 1>(t, w, k, lane, carry, carry_a);
  for (; k < w.nsub; ++k)
    fwd_block<IO, REV, ALN, WA, true, 1>(t, w, k, lane, carry, carry_a);
}

// ---------------------------------------------------------------------------
// Fused backward of one item.  The adjoint recurrence runs in the opposite
// direction of the forward scan ("B order"); element i of B order uses the
// gate of element i-1 (the shifted gate) and the state of element i+1 (the
// shifted state).  RB = true is the causal case (B order = reverse memory
// order).
// ---------------------------------------------------------------------------
struct BwdPtrs {
  const char* dy;
  const char* g;
  const char* h;
  char* dx;
  char* dg;
};

template <class IO, bool RB, bool MASKED>
__device__ inline void bwd_subtile(const float* g, const float* dy,
                                   const float* h, int64_t pv, int64_t phead,
                                   int64_t ptail, float& carry,
                                   float& carry_g, float hnext_in,
                                   float* dxo, float* dgo) {
  constexpr int V = IO::V;
  constexpr int jl = mem_idx<V, RB>(V - 1);  // last element in B order
  constexpr int jf = mem_idx<V, RB>(0);      // first element in B order
  // shifted gate for the lane's first element: previous lane's last gate
  const float gprev = dpp<kWaveShr1, 0xf>(carry_g, g[jl]);
  // shifted state for the lane's last element: next lane's first state
  const float hnx = dpp<kWaveShl1, 0xf>(hnext_in, h[jf]);
  float gs[V];
#pragma unroll
  for (int i = 0; i < V; ++i)
    gs[i] = (i == 0) ? gprev : g[mem_idx<V, RB>(i - 1)];
  float A = 1.0f, X = 0.0f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, RB>(i);
    if (MASKED && pv + j == phead) {
      A = 0.0f;
      X = dy[j];
    } else if (i == 0 && !MASKED) {
      A = gs[0];
      X = dy[j];
    } else {
      X = fmaf(gs[i], X, dy[j]);
      A = A * gs[i];
    }
  }
  wave_scan_affine(A, X);
  const float ta = readlane(A, kWave - 1);
  const float tx = readlane(X, kWave - 1);
  const float ea = dpp<kWaveShr1, 0xf>(1.0f, A);
  const float ex = dpp<kWaveShr1, 0xf>(0.0f, X);
  float d = fmaf(ea, carry, ex);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, RB>(i);
    if (MASKED && pv + j == phead)
      d = dy[j];
    else
      d = fmaf(gs[i], d, dy[j]);
    float hn = (i == V - 1) ? hnx : h[mem_idx<V, RB>(i + 1)];
    if (MASKED && pv + j == ptail) hn = 0.0f;
    dxo[j] = d;
    dgo[j] = hn * d;
  }
  carry = fmaf(ta, carry, tx);
  carry_g = readlane(g[jl], kWave - 1);
}

template <class IO, bool RB, bool ALN, bool MASKED, int NS>
__device__ inline void bwd_block(const BwdPtrs& t, const Walk<IO, RB>& w,
                                 int64_t k0, int lane, float& carry,
                                 float& carry_g) {
  constexpr int V = IO::V;
  float g[NS][V], dy[NS][V], h[NS][V];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int64_t vi = w.vec(k0 + u, lane);
    const bool ok = !MASKED || w.lane_valid(k0 + u, lane);
    load_vec<IO, ALN, MASKED>(t.dy, vi, ok, w.P0, w.P1, 0.0f, dy[u]);
    load_vec<IO, ALN, MASKED>(t.g, vi, ok, w.P0, w.P1, 1.0f, g[u]);
    load_vec<IO, ALN, MASKED>(t.h, vi, ok, w.P0, w.P1, 0.0f, h[u]);
  }
  // state just past this block in B order (pad 0 outside the segment)
  float halo = 0.0f;
  if (k0 + NS < w.nsub) {
    const int64_t vlast = w.vec(k0 + NS - 1, kWave - 1);
    const int64_t pn = RB ? vlast * V - 1 : vlast * V + V;
    if (pn >= w.P0 && pn < w.P1) halo = IO::load1(t.h + pn * IO::ES);
  }
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int64_t vi = w.vec(k0 + u, lane);
    const bool ok = !MASKED || w.lane_valid(k0 + u, lane);
    const float hin =
        (u + 1 < NS) ? readlane(h[u + 1][mem_idx<V, RB>(0)], 0) : halo;
    float dx[V], dg[V];
    bwd_subtile<IO, RB, MASKED>(g[u], dy[u], h[u], vi * V, w.head(), w.tail(),
                                carry, carry_g, hin, dx, dg);
    store_vec<IO, ALN, MASKED>(t.dx, vi, ok, w.P0, w.P1, dx);
    store_vec<IO, ALN, MASKED>(t.dg, vi, ok, w.P0, w.P1, dg);
  }
}

template <class IO, bool RB, bool ALN>
__device__ void bwd_item(const BwdPtrs& t, int64_t P0, int64_t P1, int lane) {
  constexpr int U = ASC_BWD_UNROLL;
  const Walk<IO, RB> w(P0, P1);
  float carry = 0.0f, carry_g = 1.0f;
  bwd_block<IO, RB, ALN, true, 1>(t, w, 0, lane, carry, carry_g);
  int64_t k = 1;
  for (; k + U <= w.kfast; k += U)
    bwd_block<IO, RB, ALN, false, U>(t, w, k, lane, carry, carry_g);
  for (; k < w.kfast; ++k)
    bwd_block<IO, RB, ALN, false, 1>(t, w, k, lane, carry, carry_g);
  for (; k < w.nsub; ++k)
    bwd_block<IO, RB, ALN, true, 1>(t, w, k, lane, carry, carry_g);
}

// ---------------------------------------------------------------------------
// Kernels.  Work item w (wave-uniform) -> branch, segment s, channel c.
// Channels vary fastest so that neighbouring waves stream rows of equal
// length.  DIRS: 1 = all items forward-direction, 2 = all reverse,
// 3 = branch 0 forward / branch 1 reverse (fused bidirectional launch).
// ---------------------------------------------------------------------------
struct Geometry {
  const void* cu;
  int cu64;
  int64_t S, C, T;
  int64_t items;  // S*C items per branch
  int nbranch;
  int phase;
};

__device__ inline int64_t cu_at(const Geometry& geo, int64_t i) {
  return geo.cu64 ? reinterpret_cast<const int64_t*>(geo.cu)[i]
                  : static_cast<int64_t>(reinterpret_cast<const int32_t*>(geo.cu)[i]);
}

// Decodes item w; returns false for an empty segment.
__device__ inline bool item_range(const Geometry& geo, int64_t w, int& br,
                                  int64_t& P0, int64_t& P1) {
  br = w >= geo.items ? 1 : 0;
  const int64_t r = w - br * geo.items;
  const int64_t s = r / geo.C;
  const int64_t c = r - s * geo.C;
  int64_t t0 = cu_at(geo, s), t1 = cu_at(geo, s + 1);
  t0 = t0 < 0 ? 0 : (t0 > geo.T ? geo.T : t0);
  t1 = t1 < t0 ? t0 : (t1 > geo.T ? geo.T : t1);
  const int64_t base = c * geo.T + geo.phase;
  P0 = base + t0;
  P1 = base + t1;
  return P1 > P0;
}

__device__ inline int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
}

struct FwdParams {
  Geometry geo;
  FwdPtrs br[2];
};

template <class IO, int DIRS, bool ALN, bool WA>
__global__ void __launch_bounds__(kWPB* kWave) k_scan_fwd(FwdParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t W = p.geo.items * p.geo.nbranch;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWPB;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * kWPB + wave_id(); w < W;
       w += stride) {
    int br;
    int64_t P0, P1;
    if (!item_range(p.geo, w, br, P0, P1)) continue;
    const FwdPtrs& t = p.br[br];
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      fwd_item<IO, false, ALN, WA>(t, P0, P1, lane);
    else
      fwd_item<IO, true, ALN, WA>(t, P0, P1, lane);
  }
}

struct BwdParams {
  Geometry geo;
  BwdPtrs br[2];
};

// DIRS refers to the forward scan being differentiated: 1 = causal forward
// (adjoint runs in reverse), 2 = reverse forward (adjoint runs forward),
// 3 = branch 0 causal / branch 1 reverse.
template <class IO, int DIRS, bool ALN>
__global__ void __launch_bounds__(kWPB* kWave) k_scan_bwd(BwdParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t W = p.geo.items * p.geo.nbranch;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWPB;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * kWPB + wave_id(); w < W;
       w += stride) {
    int br;
    int64_t P0, P1;
    if (!item_range(p.geo, w, br, P0, P1)) continue;
    const BwdPtrs& t = p.br[br];
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      bwd_item<IO, true, ALN>(t, P0, P1, lane);
    else
      bwd_item<IO, false, ALN>(t, P0, P1, lane);
  }
}

// ---------------------------------------------------------------------------
// shift_pad: elementwise, lanes interleaved (element t0 + 64*j + lane) so
// every load/store instruction is one contiguous run.  Boundaries of the
// wave's range are found by a binary search over cu_seqlens.
// ---------------------------------------------------------------------------
constexpr int kShiftPerLane = 8;
constexpr int64_t kShiftChunk = kWave * kShiftPerLane;

struct ShiftParams {
  const char* data;
  char* out;
  const void* cu;
  int cu64;
  int64_t S, C, L;
  int64_t chunks;  // chunks per row
  float pad;
  int backward;
  int wrap;
};

__device__ inline int64_t shift_boundary(const ShiftParams& p, int64_t k) {
  // k-th boundary position (k in [0, S)), ascending for a monotone cu.
  const int64_t i = p.backward ? k : k + 1;
  const int64_t v = p.cu64 ? reinterpret_cast<const int64_t*>(p.cu)[i]
                           : static_cast<int64_t>(reinterpret_cast<const int32_t*>(p.cu)[i]);
  return p.backward ? v : v - 1;
}

template <class IO>
__global__ void __launch_bounds__(4 * kWave) k_shift_pad(ShiftParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t W = p.C * p.chunks;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 4;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * 4 +
                   __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
       w < W; w += stride) {
    const int64_t c = w / p.chunks;
    const int64_t t0 = (w - c * p.chunks) * kShiftChunk;
    const int64_t t1 = t0 + kShiftChunk < p.L ? t0 + kShiftChunk : p.L;
    const char* row = p.data + c * p.L * IO::ES;
    char* orow = p.out + c * p.L * IO::ES;
    float v[kShiftPerLane];
#pragma unroll
    for (int j = 0; j < kShiftPerLane; ++j) {
      const int64_t t = t0 + j * kWave + lane;
      v[j] = 0.0f;
      if (t < t1) {
        int64_t src = p.backward ? t - 1 : t + 1;
        if (src < 0) src = p.wrap ? p.L - 1 : 0;
        if (src >= p.L) src = p.wrap ? 0 : p.L - 1;
        v[j] = IO::load1(row + src * IO::ES);
      }
    }
    // first boundary >= t0
    int64_t lo = 0, hi = p.S;
    while (lo < hi) {
      const int64_t mid = (lo + hi) / 2;
      if (shift_boundary(p, mid) < t0)
        lo = mid + 1;
      else
        hi = mid;
    }
    auto mark = [&](int64_t q) {
      if (q < t0 || q >= t1) return;
      const int64_t off = q - t0;
      const int j = static_cast<int>(off / kWave);
      if (lane == static_cast<int>(off % kWave)) {
#pragma unroll
        for (int jj = 0; jj < kShiftPerLane; ++jj)
          if (jj == j) v[jj] = p.pad;
      }
    };
    for (int64_t k = lo; k < p.S; ++k) {
      const int64_t q = shift_boundary(p, k);
      if (q >= t1) break;
      mark(q);
    }
    // A negative boundary position (end of a zero-length first segment)
    // counts from the row end, as torch indexing does in the reference.
    for (int64_t k = 0; k < p.S; ++k) {
      const int64_t q = shift_boundary(p, k);
      if (q >= 0) break;
      mark(q + p.L);
    }
#pragma unroll
    for (int j = 0; j < kShiftPerLane; ++j) {
      const int64_t t = t0 + j * kWave + lane;
      if (t < t1) IO::store1(orow + t * IO::ES, v[j]);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
int elem_size(int dtype) {
  switch (dtype) {
    case ASC_F32: return 4;
    case ASC_F16: return 2;
    case ASC_BF16: return 2;
    default: return 0;
  }
}

// Largest number of resident work-groups worth launching before the
// grid-stride loop takes over.
constexpr int64_t kMaxGrid = int64_t(1) << 24;

int check_geometry(const void* cu, int cu_dtype, int64_t S, int64_t C,
                   int64_t T, int dtype) {
  if (!cu) return ASC_E_NULL;
  if (elem_size(dtype) == 0) return ASC_E_DTYPE;
  if (cu_dtype != ASC_CU_I32 && cu_dtype != ASC_CU_I64) return ASC_E_DTYPE;
  if (S < 0 || C < 0 || T < 0) return ASC_E_SIZE;
  if (C > 0 && T > (INT64_MAX / 64) / C) return ASC_E_SIZE;
  if (S > (INT64_MAX / 64) / (C > 0 ? C : 1)) return ASC_E_SIZE;
  const uintptr_t cua = reinterpret_cast<uintptr_t>(cu);
  if (cua % (cu_dtype == ASC_CU_I64 ? 8 : 4)) return ASC_E_ALIGN;
  return ASC_OK;
}

// Shared phase of a set of tensor pointers, or -1 when they differ.
int common_phase(const void* const* ptrs, int n, int es, int v) {
  int ph = -1;
  for (int i = 0; i < n; ++i) {
    if (!ptrs[i]) continue;
    const int q = static_cast<int>((reinterpret_cast<uintptr_t>(ptrs[i]) / es) % v);
    if (ph < 0) ph = q;
    else if (ph != q) return -1;
  }
  return ph < 0 ? 0 : ph;
}

int check_ptrs(const void* const* ptrs, int n, int es) {
  for (int i = 0; i < n; ++i)
    if (ptrs[i] && reinterpret_cast<uintptr_t>(ptrs[i]) % es) return ASC_E_ALIGN;
  return ASC_OK;
}

template <class Params>
int launch(const void* fn, int64_t items, int waves_per_block, Params& p,
           void* stream) {
  int64_t blocks = (items + waves_per_block - 1) / waves_per_block;
  if (blocks > kMaxGrid) blocks = kMaxGrid;
  void* args[] = {&p};
  const hipError_t e = hipLaunchKernel(fn, dim3(static_cast<unsigned>(blocks)),
                                       dim3(waves_per_block * kWave), args, 0,
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ASC_OK : static_cast<int>(e);
}

template <class IO>
const void* pick_fwd(int dirs, bool aln, bool wa) {
#define ASC_F(D, A, W) reinterpret_cast<const void*>(&k_scan_fwd<IO, D, A, W>)
  if (dirs == 1) {
    if (aln) return wa ? ASC_F(1, true, true) : ASC_F(1, true, false);
    return wa ? ASC_F(1, false, true) : ASC_F(1, false, false);
  }
  if (dirs == 2) {
    if (aln) return wa ? ASC_F(2, true, true) : ASC_F(2, true, false);
    return wa ? ASC_F(2, false, true) : ASC_F(2, false, false);
  }
  return aln ? ASC_F(3, true, false) : ASC_F(3, false, false);
#undef ASC_F
}

template <class IO>
const void* pick_bwd(int dirs, bool aln) {
#define ASC_B(D, A) reinterpret_cast<const void*>(&k_scan_bwd<IO, D, A>)
  if (dirs == 1) return aln ? ASC_B(1, true) : ASC_B(1, false);
  if (dirs == 2) return aln ? ASC_B(2, true) : ASC_B(2, false);
  return aln ? ASC_B(3, true) : ASC_B(3, false);
#undef ASC_B
}

int run_fwd(const void* const* g, const void* const* x, void* const* h,
            void* a, int nbranch, int dirs, const void* cu, int cu_dtype,
            int64_t S, int64_t C, int64_t T, int dtype, void* stream) {
  int st = check_geometry(cu, cu_dtype, S, C, T, dtype);
  if (st) return st;
  for (int b = 0; b < nbranch; ++b)
    if (!g[b] || !x[b] || !h[b]) return ASC_E_NULL;
  const int es = elem_size(dtype);
  const int v = 16 / es;
  const void* all[7];
  int n = 0;
  for (int b = 0; b < nbranch; ++b) {
    all[n++] = g[b];
    all[n++] = x[b];
    all[n++] = h[b];
  }
  all[n++] = a;
  if ((st = check_ptrs(all, n, es))) return st;
  if (S == 0 || C == 0 || T == 0) return ASC_OK;
  const int ph = common_phase(all, n, es, v);
  const bool aln = ph >= 0;
  FwdParams p{};
  p.geo = Geometry{cu, cu_dtype == ASC_CU_I64, S, C, T, S * C, nbranch,
                   aln ? ph : 0};
  const int64_t shift = static_cast<int64_t>(p.geo.phase) * es;
  for (int b = 0; b < nbranch; ++b) {
    p.br[b].g = static_cast<const char*>(g[b]) - shift;
    p.br[b].x = static_cast<const char*>(x[b]) - shift;
    p.br[b].h = static_cast<char*>(h[b]) - shift;
    p.br[b].a = (b == 0 && a) ? static_cast<char*>(a) - shift : nullptr;
  }
  const bool wa = a != nullptr;
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = pick_fwd<IoF32>(dirs, aln, wa); break;
    case ASC_F16: fn = pick_fwd<IoF16>(dirs, aln, wa); break;
    default: fn = pick_fwd<IoBF16>(dirs, aln, wa); break;
  }
  return launch(fn, p.geo.items * nbranch, kWPB, p, stream);
}

int run_bwd(const void* const* dy, const void* const* g, const void* const* h,
            void* const* dx, void* const* dg, int nbranch, int dirs,
            const void* cu, int cu_dtype, int64_t S, int64_t C, int64_t T,
            int dtype, void* stream) {
  int st = check_geometry(cu, cu_dtype, S, C, T, dtype);
  if (st) return st;
  for (int b = 0; b < nbranch; ++b)
    if (!dy[b] || !g[b] || !h[b] || !dx[b] || !dg[b]) return ASC_E_NULL;
  const int es = elem_size(dtype);
  const int v = 16 / es;
  const void* all[10];
  int n = 0;
  for (int b = 0; b < nbranch; ++b) {
    all[n++] = dy[b];
    all[n++] = g[b];
    all[n++] = h[b];
    all[n++] = dx[b];
    all[n++] = dg[b];
  }
  if ((st = check_ptrs(all, n, es))) return st;
  if (S == 0 || C == 0 || T == 0) return ASC_OK;
  const int ph = common_phase(all, n, es, v);
  const bool aln = ph >= 0;
  BwdParams p{};
  p.geo = Geometry{cu, cu_dtype == ASC_CU_I64, S, C, T, S * C, nbranch,
                   aln ? ph : 0};
  const int64_t shift = static_cast<int64_t>(p.geo.phase) * es;
  for (int b = 0; b < nbranch; ++b) {
    p.br[b].dy = static_cast<const char*>(dy[b]) - shift;
    p.br[b].g = static_cast<const char*>(g[b]) - shift;
    p.br[b].h = static_cast<const char*>(h[b]) - shift;
    p.br[b].dx = static_cast<char*>(dx[b]) - shift;
    p.br[b].dg = static_cast<char*>(dg[b]) - shift;
  }
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = pick_bwd<IoF32>(dirs, aln); break;
    case ASC_F16: fn = pick_bwd<IoF16>(dirs, aln); break;
    default: fn = pick_bwd<IoBF16>(dirs, aln); break;
  }
  return launch(fn, p.geo.items * nbranch, kWPB, p, stream);
}

}  // namespace

extern "C" {

int asc_abi_version(void) { return ASC_ABI_VERSION; }

const char* asc_strerror(int status) {
  switch (status) {
    case ASC_OK: return "success";
    case ASC_E_NULL: return "a required pointer argument is NULL";
    case ASC_E_DTYPE: return "unsupported dtype or cu_seqlens dtype";
    case ASC_E_SIZE: return "invalid (negative or overflowing) size argument";
    case ASC_E_ALIGN: return "pointer not aligned to its element size";
    case ASC_E_ARG: return "invalid argument";
    default:
      if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
      return "unknown error";
  }
}

int asc_scan_fwd(const void* gates, const void* tokens, void* h_out,
                 void* gate_prod_out, const void* cu_seqlens, int cu_dtype,
                 int64_t num_seq, int64_t num_channels, int64_t seq_stride,
                 int dtype, int reverse, void* stream) {
  const void* g[1] = {gates};
  const void* x[1] = {tokens};
  void* h[1] = {h_out};
  return run_fwd(g, x, h, gate_prod_out, 1, reverse ? 2 : 1, cu_seqlens,
                 cu_dtype, num_seq, num_channels, seq_stride, dtype, stream);
}

int asc_scan_bwd(const void* grad, const void* gates, const void* states,
                 void* d_tokens, void* d_gates, const void* cu_seqlens,
                 int cu_dtype, int64_t num_seq, int64_t num_channels,
                 int64_t seq_stride, int dtype, int causal, void* stream) {
  const void* dy[1] = {grad};
  const void* g[1] = {gates};
  const void* h[1] = {states};
  void* dx[1] = {d_tokens};
  void* dg[1] = {d_gates};
  return run_bwd(dy, g, h, dx, dg, 1, causal ? 1 : 2, cu_seqlens, cu_dtype,
                 num_seq, num_channels, seq_stride, dtype, stream);
}

int asc_scan_bidi_fwd(const void* gates_fwd, const void* tokens_fwd,
                      const void* gates_bwd, const void* tokens_bwd,
                      void* h_fwd, void* h_bwd, const void* cu_seqlens,
                      int cu_dtype, int64_t num_seq, int64_t num_channels,
                      int64_t seq_stride, int dtype, void* stream) {
  const void* g[2] = {gates_fwd, gates_bwd};
  const void* x[2] = {tokens_fwd, tokens_bwd};
  void* h[2] = {h_fwd, h_bwd};
  return run_fwd(g, x, h, nullptr, 2, 3, cu_seqlens, cu_dtype, num_seq,
                 num_channels, seq_stride, dtype, stream);
}

int asc_scan_bidi_bwd(const void* grad_fwd, const void* grad_bwd,
                      const void* gates_fwd, const void* gates_bwd,
                      const void* states_fwd, const void* states_bwd,
                      void* d_tokens_fwd, void* d_gates_fwd,
                      void* d_tokens_bwd, void* d_gates_bwd,
                      const void* cu_seqlens, int cu_dtype, int64_t num_seq,
                      int64_t num_channels, int64_t seq_stride, int dtype,
                      void* stream) {
  const void* dy[2] = {grad_fwd, grad_bwd};
  const void* g[2] = {gates_fwd, gates_bwd};
  const void* h[2] = {states_fwd, states_bwd};
  void* dx[2] = {d_tokens_fwd, d_tokens_bwd};
  void* dg[2] = {d_gates_fwd, d_gates_bwd};
  return run_bwd(dy, g, h, dx, dg, 2, 3, cu_seqlens, cu_dtype, num_seq,
                 num_channels, seq_stride, dtype, stream);
}

int asc_shift_pad(const void* data, void* out, const void* cu_seqlens,
                  int cu_dtype, int64_t num_seq, int64_t num_channels,
                  int64_t seq_len, int dtype, double pad_value, int backward,
                  int wrap, void* stream) {
  int st = check_geometry(cu_seqlens, cu_dtype, num_seq, num_channels,
                          seq_len, dtype);
  if (st) return st;
  if (!data || !out) return ASC_E_NULL;
  const int es = elem_size(dtype);
  const void* all[2] = {data, out};
  if ((st = check_ptrs(all, 2, es))) return st;
  if (num_channels == 0 || seq_len == 0) return ASC_OK;
  ShiftParams p{};
  p.data = static_cast<const char*>(data);
  p.out = static_cast<char*>(out);
  p.cu = cu_seqlens;
  p.cu64 = cu_dtype == ASC_CU_I64;
  p.S = num_seq;
  p.C = num_channels;
  p.L = seq_len;
  p.chunks = (seq_len + kShiftChunk - 1) / kShiftChunk;
  p.pad = static_cast<float>(pad_value);
  p.backward = backward ? 1 : 0;
  p.wrap = wrap ? 1 : 0;
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = reinterpret_cast<const void*>(&k_shift_pad<IoF32>); break;
    case ASC_F16: fn = reinterpret_cast<const void*>(&k_shift_pad<IoF16>); break;
    default: fn = reinterpret_cast<const void*>(&k_shift_pad<IoBF16>); break;
  }
  return launch(fn, p.C * p.chunks, 4, p, stream);
}

}  // extern "C"
