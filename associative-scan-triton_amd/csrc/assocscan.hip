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
// Sub-tiles per wave and iteration of the workgroup-cooperative kernels.
#ifndef ASC_WG_UNROLL
#define ASC_WG_UNROLL 1
#endif
// Non-temporal (streaming) hints on the 16-byte loads / stores.
#ifndef ASC_NT_LOAD
#define ASC_NT_LOAD 1
#endif
#ifndef ASC_NT_STORE
#define ASC_NT_STORE 1
#endif

namespace {

constexpr int kWave = 64;
constexpr int kWPB = ASC_WAVES_PER_BLOCK;
constexpr int kUW = ASC_WG_UNROLL;

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

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ inline uint4 ld16(const char* p) {
  const u32x4* q = reinterpret_cast<const u32x4*>(p);
  const u32x4 v = ASC_NT_LOAD ? __builtin_nontemporal_load(q) : *q;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ inline void st16(char* p, uint4 v) {
  u32x4* q = reinterpret_cast<u32x4*>(p);
  const u32x4 w = {v.x, v.y, v.z, v.w};
  if (ASC_NT_STORE)
    __builtin_nontemporal_store(w, q);
  else
    *q = w;
}

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

// Byte offset of the lane's vector from the lowest-addressed vector of its
// sub-tile (lane 0 comes first in scan order).
template <bool REV>
__device__ inline uint32_t lane_off(int lane) {
  return static_cast<uint32_t>(REV ? (kWave - 1 - lane) : lane) * 16u;
}

// Lowest-addressed vector of sub-tile k.
template <class IO, bool REV>
__device__ inline int64_t sub_lo(const Walk<IO, REV>& w, int64_t k) {
  return REV ? w.v1 - k * kWave - (kWave - 1) : w.v0 + k * kWave;
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
      IO::unpack(ld16(origin + vi * 16), f);
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) f[j] = IO::load1(origin + (pv + j) * IO::ES);
    }
    return;
  }
  const bool full = lane_ok && pv >= P0 && pv + V <= P1;
  if (ALN && full) {
    IO::unpack(ld16(origin + vi * 16), f);
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
      st16(origin + vi * 16, IO::pack(f));
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) IO::store1(origin + (pv + j) * IO::ES, f[j]);
    }
    return;
  }
  const bool full = lane_ok && pv >= P0 && pv + V <= P1;
  if (ALN && full) {
    st16(origin + vi * 16, IO::pack(f));
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

// First phase of a sub-tile: the lane's exclusive prefix map (ea, ex) and
// the sub-tile's total map (ta, tx, uniform across the wave).
struct SubScan {
  float ea, ex, ta, tx;
};

// Lane-serial scan of the lane's elements, then the 64-lane DPP scan.
// g, x in memory order (masked to the identity when MASKED); phead is the
// segment's first element in scan order (reset exactly there).
template <class IO, bool REV, bool MASKED>
__device__ inline SubScan fwd_local(const float* g, const float* x, int64_t pv,
                                    int64_t phead) {
  constexpr int V = IO::V;
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
  wave_scan_affine(A, X);
  SubScan r;
  r.ta = readlane(A, kWave - 1);
  r.tx = readlane(X, kWave - 1);
  r.ea = dpp<kWaveShr1, 0xf>(1.0f, A);
  r.ex = dpp<kWaveShr1, 0xf>(0.0f, X);
  return r;
}

// Second phase: the lane re-walks its elements from its prefix applied to
// the carry into the sub-tile; h in memory order.
template <class IO, bool REV, bool MASKED>
__device__ inline void fwd_apply(const float* g, const float* x, int64_t pv,
                                 int64_t phead, const SubScan& s, float carry,
                                 float* hout) {
  constexpr int V = IO::V;
  float hh = fmaf(s.ea, carry, s.ex);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, REV>(i);
    if (MASKED && pv + j == phead)
      hh = x[j];
    else
      hh = fmaf(g[j], hh, x[j]);
    hout[j] = hh;
  }
}

// One sub-tile with a carry in a register; writes h (and the gate product
// when WA) in memory order.
template <class IO, bool REV, bool MASKED, bool WA>
__device__ inline void fwd_subtile(const float* g, const float* x, int64_t pv,
                                   int64_t phead, float& carry, float& carry_a,
                                   float* hout, float* aout) {
  constexpr int V = IO::V;
  const SubScan s = fwd_local<IO, REV, MASKED>(g, x, pv, phead);
  fwd_apply<IO, REV, MASKED>(g, x, pv, phead, s, carry, hout);
  carry = fmaf(s.ta, carry, s.tx);
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

// Interior sub-tiles [k, kend) ((kend - k) a positive multiple of U), all
// full and aligned.  Software-pipelined: the loads of the next block of U
// sub-tiles are issued before the current block is scanned, so each wave
// keeps 2*U*16 bytes per lane and tensor in flight while it computes.
template <class IO, bool REV, bool WA, int U>
__device__ inline void fwd_fast(const FwdPtrs& t, const Walk<IO, REV>& w,
                                int64_t k, int64_t kend, int lane,
                                float& carry, float& carry_a) {
  constexpr int V = IO::V;
  constexpr int STEP = REV ? -kWave * 16 : kWave * 16;  // bytes per sub-tile
  const uint32_t lo = lane_off<REV>(lane);
  uint4 ga[U], xa[U], gb[U], xb[U];
  auto load = [&](uint4(&g)[U], uint4(&x)[U], int64_t kk) {
    const int64_t b = sub_lo(w, kk) * 16;
    const char* gp = t.g + b + lo;
    const char* xp = t.x + b + lo;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      g[u] = ld16(gp + u * STEP);
      x[u] = ld16(xp + u * STEP);
    }
  };
  auto run = [&](const uint4(&g)[U], const uint4(&x)[U], int64_t kk) {
    const int64_t b = sub_lo(w, kk) * 16;
    char* hp = t.h + b + lo;
    char* ap = WA ? t.a + b + lo : nullptr;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float gf[V], xf[V], hf[V], af[V];
      IO::unpack(g[u], gf);
      IO::unpack(x[u], xf);
      fwd_subtile<IO, REV, false, WA>(gf, xf, 0, 0, carry, carry_a, hf, af);
      st16(hp + u * STEP, IO::pack(hf));
      if (WA) st16(ap + u * STEP, IO::pack(af));
    }
  };
  load(ga, xa, k);
  while (true) {
    const bool more = k + U < kend;
    if (more) load(gb, xb, k + U);
    run(ga, xa, k);
    k += U;
    if (!more) break;
    const bool more2 = k + U < kend;
    if (more2) load(ga, xa, k + U);
    run(gb, xb, k);
    k += U;
    if (!more2) break;
  }
}

template <class IO, bool REV, bool ALN, bool WA>
__device__ void fwd_item(const FwdPtrs& t, int64_t P0, int64_t P1, int lane) {
  constexpr int U = ASC_FWD_UNROLL;
  const Walk<IO, REV> w(P0, P1);
  float carry = 0.0f, carry_a = 1.0f;
  fwd_block<IO, REV, ALN, WA, true, 1>(t, w, 0, lane, carry, carry_a);
  int64_t k = 1;
  if (ALN) {
    const int64_t nfull = (w.kfast - 1) / U * U;
    if (nfull > 0) {
      fwd_fast<IO, REV, WA, U>(t, w, 1, 1 + nfull, lane, carry, carry_a);
      k = 1 + nfull;
    }
  } else {
    for (; k + U <= w.kfast; k += U)
      fwd_block<IO, REV, ALN, WA, false, U>(t, w, k, lane, carry, carry_a);
  }
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

// First phase of a backward sub-tile.  carry_g is the gate of the element
// just before the sub-tile in B order (it shifts into lane 0); returns the
// lane's shifted gate for its first element in gprev.
template <class IO, bool RB, bool MASKED>
__device__ inline SubScan bwd_local(const float* g, const float* dy, int64_t pv,
                                    int64_t phead, float carry_g,
                                    float& gprev) {
  constexpr int V = IO::V;
  constexpr int jl = mem_idx<V, RB>(V - 1);  // last element in B order
  gprev = dpp<kWaveShr1, 0xf>(carry_g, g[jl]);
  float A = 1.0f, X = 0.0f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, RB>(i);
    const float gs = (i == 0) ? gprev : g[mem_idx<V, RB>(i - 1)];
    if (MASKED && pv + j == phead) {
      A = 0.0f;
      X = dy[j];
    } else if (i == 0 && !MASKED) {
      A = gs;
      X = dy[j];
    } else {
      X = fmaf(gs, X, dy[j]);
      A = A * gs;
    }
  }
  wave_scan_affine(A, X);
  SubScan r;
  r.ta = readlane(A, kWave - 1);
  r.tx = readlane(X, kWave - 1);
  r.ea = dpp<kWaveShr1, 0xf>(1.0f, A);
  r.ex = dpp<kWaveShr1, 0xf>(0.0f, X);
  return r;
}

// Second phase: dx by re-walking from the prefix, dg = shifted state * dx.
// hnext_in is the state of the element just after the sub-tile in B order
// (it shifts into lane 63); ptail is the segment's last element in B order,
// whose shifted state is the pad 0.
template <class IO, bool RB, bool MASKED>
__device__ inline void bwd_apply(const float* g, const float* dy,
                                 const float* h, int64_t pv, int64_t phead,
                                 int64_t ptail, float gprev, float hnext_in,
                                 const SubScan& s, float carry, float* dxo,
                                 float* dgo) {
  constexpr int V = IO::V;
  constexpr int jf = mem_idx<V, RB>(0);  // first element in B order
  const float hnx = dpp<kWaveShl1, 0xf>(hnext_in, h[jf]);
  float d = fmaf(s.ea, carry, s.ex);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = mem_idx<V, RB>(i);
    const float gs = (i == 0) ? gprev : g[mem_idx<V, RB>(i - 1)];
    if (MASKED && pv + j == phead)
      d = dy[j];
    else
      d = fmaf(gs, d, dy[j]);
    float hn = (i == V - 1) ? hnx : h[mem_idx<V, RB>(i + 1)];
    if (MASKED && pv + j == ptail) hn = 0.0f;
    dxo[j] = d;
    dgo[j] = hn * d;
  }
}

template <class IO, bool RB, bool MASKED>
__device__ inline void bwd_subtile(const float* g, const float* dy,
                                   const float* h, int64_t pv, int64_t phead,
                                   int64_t ptail, float& carry,
                                   float& carry_g, float hnext_in,
                                   float* dxo, float* dgo) {
  constexpr int V = IO::V;
  float gprev;
  const SubScan s = bwd_local<IO, RB, MASKED>(g, dy, pv, phead, carry_g, gprev);
  bwd_apply<IO, RB, MASKED>(g, dy, h, pv, phead, ptail, gprev, hnext_in, s,
                            carry, dxo, dgo);
  carry = fmaf(s.ta, carry, s.tx);
  carry_g = readlane(g[mem_idx<V, RB>(V - 1)], kWave - 1);
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

// State just past sub-tiles [kk, kk + n) in B order, 0 past the segment.
template <class IO, bool RB>
__device__ inline float bwd_halo(const BwdPtrs& t, const Walk<IO, RB>& w,
                                 int64_t kk, int n) {
  constexpr int V = IO::V;
  if (kk + n >= w.nsub) return 0.0f;
  const int64_t vlast = w.vec(kk + n - 1, kWave - 1);
  const int64_t pn = RB ? vlast * V - 1 : vlast * V + V;
  return (pn >= w.P0 && pn < w.P1) ? IO::load1(t.h + pn * IO::ES) : 0.0f;
}

// Interior sub-tiles of the backward, software-pipelined like fwd_fast.
template <class IO, bool RB, int U>
__device__ inline void bwd_fast(const BwdPtrs& t, const Walk<IO, RB>& w,
                                int64_t k, int64_t kend, int lane,
                                float& carry, float& carry_g) {
  constexpr int V = IO::V;
  constexpr int STEP = RB ? -kWave * 16 : kWave * 16;
  const uint32_t lo = lane_off<RB>(lane);
  uint4 ya[U], ga[U], ha[U], yb[U], gb[U], hb[U];
  float halo_a, halo_b;
  auto load = [&](uint4(&y)[U], uint4(&g)[U], uint4(&h)[U], float& halo,
                  int64_t kk) {
    const int64_t b = sub_lo(w, kk) * 16;
    const char* yp = t.dy + b + lo;
    const char* gp = t.g + b + lo;
    const char* hp = t.h + b + lo;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      y[u] = ld16(yp + u * STEP);
      g[u] = ld16(gp + u * STEP);
      h[u] = ld16(hp + u * STEP);
    }
    halo = bwd_halo(t, w, kk, U);
  };
  auto run = [&](const uint4(&y)[U], const uint4(&g)[U], const uint4(&h)[U],
                 float halo, int64_t kk) {
    const int64_t b = sub_lo(w, kk) * 16;
    char* xp = t.dx + b + lo;
    char* dp = t.dg + b + lo;
    float hf[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u) IO::unpack(h[u], hf[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float yf[V], gf[V], dx[V], dg[V];
      IO::unpack(y[u], yf);
      IO::unpack(g[u], gf);
      const float hin =
          (u + 1 < U) ? readlane(hf[u + 1][mem_idx<V, RB>(0)], 0) : halo;
      bwd_subtile<IO, RB, false>(gf, yf, hf[u], 0, 0, 0, carry, carry_g, hin,
                                 dx, dg);
      st16(xp + u * STEP, IO::pack(dx));
      st16(dp + u * STEP, IO::pack(dg));
    }
  };
  load(ya, ga, ha, halo_a, k);
  while (true) {
    const bool more = k + U < kend;
    if (more) load(yb, gb, hb, halo_b, k + U);
    run(ya, ga, ha, halo_a, k);
    k += U;
    if (!more) break;
    const bool more2 = k + U < kend;
    if (more2) load(ya, ga, ha, halo_a, k + U);
    run(yb, gb, hb, halo_b, k);
    k += U;
    if (!more2) break;
  }
}

template <class IO, bool RB, bool ALN>
__device__ void bwd_item(const BwdPtrs& t, int64_t P0, int64_t P1, int lane) {
  constexpr int U = ASC_BWD_UNROLL;
  const Walk<IO, RB> w(P0, P1);
  float carry = 0.0f, carry_g = 1.0f;
  bwd_block<IO, RB, ALN, true, 1>(t, w, 0, lane, carry, carry_g);
  int64_t k = 1;
  if (ALN) {
    const int64_t nfull = (w.kfast - 1) / U * U;
    if (nfull > 0) {
      bwd_fast<IO, RB, U>(t, w, 1, 1 + nfull, lane, carry, carry_g);
      k = 1 + nfull;
    }
  } else {
    for (; k + U <= w.kfast; k += U)
      bwd_block<IO, RB, ALN, false, U>(t, w, k, lane, carry, carry_g);
  }
  for (; k < w.kfast; ++k)
    bwd_block<IO, RB, ALN, false, 1>(t, w, k, lane, carry, carry_g);
  for (; k < w.nsub; ++k)
    bwd_block<IO, RB, ALN, true, 1>(t, w, k, lane, carry, carry_g);
}

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
  const Walk<IO, REV> w(P0, P1);
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

template <class IO, bool RB, bool ALN, int NW>
__device__ void bwd_item_wg(const BwdPtrs& t, int64_t P0, int64_t P1,
                            int lane, int wv, float2* agg) {
  constexpr int V = IO::V;
  constexpr int TS = NW * kUW;
  constexpr int jl = mem_idx<V, RB>(V - 1);
  constexpr int jf = mem_idx<V, RB>(0);
  const Walk<IO, RB> w(P0, P1);
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
      load_sub<IO, RB, ALN>(t.dy, w, k0 + u, lane, 0.0f, y[u]);
      load_sub<IO, RB, ALN>(t.g, w, k0 + u, lane, 1.0f, g[u]);
      load_sub<IO, RB, ALN>(t.h, w, k0 + u, lane, 0.0f, h[u]);
    }
    gp = bwd_gate_before(t, w, k0);
    hn = bwd_halo(t, w, k0, kUW);
  };
  auto step = [&](const float(&y)[kUW][V], const float(&g)[kUW][V],
                  const float(&h)[kUW][V], float gp, float hn, int64_t it) {
    const int64_t k0 = it * TS + wv * kUW;
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

// ---------------------------------------------------------------------------
// Kernels.  Work item w (wave-uniform) -> branch, segment s, channel c.
// DIRS: 1 = all items forward-direction, 2 = all reverse,
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

// Tells the compiler a value is the same in every lane (it is: all lanes
// of a wave work on the same item), so that item geometry and base
// addresses live in scalar registers.
__device__ inline int64_t uniform(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ inline int64_t cu_at(const Geometry& geo, int64_t i) {
  return uniform(geo.cu64
                     ? reinterpret_cast<const int64_t*>(geo.cu)[i]
                     : static_cast<int64_t>(reinterpret_cast<const int32_t*>(geo.cu)[i]));
}

// Decodes item w; returns false for an empty segment.  SEG_MAJOR: items
// w, w+1 are neighbouring segments of one row, so waves that run at the
// same time stream neighbouring memory (the order used for short items);
// otherwise they are the same segment of neighbouring channels.
template <bool SEG_MAJOR>
__device__ inline bool item_range(const Geometry& geo, int64_t w, int& br,
                                  int64_t& P0, int64_t& P1) {
  br = w >= geo.items ? 1 : 0;
  const int64_t r = w - br * geo.items;
  int64_t s, c;
  if (SEG_MAJOR) {
    c = r / geo.S;
    s = r - c * geo.S;
  } else {
    s = r / geo.C;
    c = r - s * geo.C;
  }
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
    if (!item_range<true>(p.geo, w, br, P0, P1)) continue;
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
    if (!item_range<true>(p.geo, w, br, P0, P1)) continue;
    const BwdPtrs& t = p.br[br];
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      bwd_item<IO, true, ALN>(t, P0, P1, lane);
    else
      bwd_item<IO, false, ALN>(t, P0, P1, lane);
  }
}

// Workgroup-cooperative kernels: one item per workgroup of NW waves.
template <class IO, int DIRS, bool ALN, int NW>
__global__ void __launch_bounds__(NW* kWave) k_scan_fwd_wg(FwdParams p) {
  __shared__ float2 agg[2 * NW];
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  const int64_t W = p.geo.items * p.geo.nbranch;
  for (int64_t item = blockIdx.x; item < W; item += gridDim.x) {
    int br;
    int64_t P0, P1;
    if (!item_range<false>(p.geo, item, br, P0, P1)) continue;
    const FwdPtrs& t = p.br[br];
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      fwd_item_wg<IO, false, ALN, NW>(t, P0, P1, lane, wv, agg);
    else
      fwd_item_wg<IO, true, ALN, NW>(t, P0, P1, lane, wv, agg);
    __syncthreads();  // agg is reused by the next item
  }
}

template <class IO, int DIRS, bool ALN, int NW>
__global__ void __launch_bounds__(NW* kWave) k_scan_bwd_wg(BwdParams p) {
  __shared__ float2 agg[2 * NW];
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  const int64_t W = p.geo.items * p.geo.nbranch;
  for (int64_t item = blockIdx.x; item < W; item += gridDim.x) {
    int br;
    int64_t P0, P1;
    if (!item_range<false>(p.geo, item, br, P0, P1)) continue;
    const BwdPtrs& t = p.br[br];
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      bwd_item_wg<IO, true, ALN, NW>(t, P0, P1, lane, wv, agg);
    else
      bwd_item_wg<IO, false, ALN, NW>(t, P0, P1, lane, wv, agg);
    __syncthreads();
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
int launch(const void* fn, int64_t blocks, int waves_per_block, Params& p,
           void* stream) {
  if (blocks > kMaxGrid) blocks = kMaxGrid;
  void* args[] = {&p};
  const hipError_t e = hipLaunchKernel(fn, dim3(static_cast<unsigned>(blocks)),
                                       dim3(waves_per_block * kWave), args, 0,
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ASC_OK : static_cast<int>(e);
}

// Walk selection from the mean segment length (host-side, no sync).  The
// workgroup-cooperative walk pays one barrier per iteration and an
// unoverlapped first load per item, so it needs several iterations per item
// to beat one wave per item; the thresholds below are in iterations of the
// 16-wave and 8-wave tiles and were set by measurement on MI355X.
// Returns the waves per workgroup, or 0 for one wave per item.
#ifndef ASC_FWD_WG16_MIN_ITERS
#define ASC_FWD_WG16_MIN_ITERS 8
#endif
#ifndef ASC_BWD_WG16_MIN_ITERS
#define ASC_BWD_WG16_MIN_ITERS 4
#endif
#ifndef ASC_WG8_MIN_ITERS
#define ASC_WG8_MIN_ITERS 4
#endif
int pick_walk(int64_t S, int64_t T, int v, bool bwd) {
  const int64_t mean = T / (S > 0 ? S : 1);
  const int64_t tile1 = static_cast<int64_t>(kUW) * kWave * v;  // per wave
  const int64_t it16 = bwd ? ASC_BWD_WG16_MIN_ITERS : ASC_FWD_WG16_MIN_ITERS;
  if (mean >= it16 * 16 * tile1) return 16;
  if (mean >= static_cast<int64_t>(ASC_WG8_MIN_ITERS) * 8 * tile1) return 8;
  return 0;
}

template <class IO, int NW>
const void* pick_fwd_wg(int dirs, bool aln) {
#define ASC_F(D, A) reinterpret_cast<const void*>(&k_scan_fwd_wg<IO, D, A, NW>)
  if (dirs == 1) return aln ? ASC_F(1, true) : ASC_F(1, false);
  if (dirs == 2) return aln ? ASC_F(2, true) : ASC_F(2, false);
  return aln ? ASC_F(3, true) : ASC_F(3, false);
#undef ASC_F
}

template <class IO, int NW>
const void* pick_bwd_wg(int dirs, bool aln) {
#define ASC_B(D, A) reinterpret_cast<const void*>(&k_scan_bwd_wg<IO, D, A, NW>)
  if (dirs == 1) return aln ? ASC_B(1, true) : ASC_B(1, false);
  if (dirs == 2) return aln ? ASC_B(2, true) : ASC_B(2, false);
  return aln ? ASC_B(3, true) : ASC_B(3, false);
#undef ASC_B
}

template <class IO>
const void* pick_fwd_wg(int nw, int dirs, bool aln) {
  return nw == 16 ? pick_fwd_wg<IO, 16>(dirs, aln) : pick_fwd_wg<IO, 8>(dirs, aln);
}

template <class IO>
const void* pick_bwd_wg(int nw, int dirs, bool aln) {
  return nw == 16 ? pick_bwd_wg<IO, 16>(dirs, aln) : pick_bwd_wg<IO, 8>(dirs, aln);
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
  const int64_t items = p.geo.items * nbranch;
  const int nw = wa ? 0 : pick_walk(S, T, v, false);
  if (nw) {
    const void* fn = nullptr;
    switch (dtype) {
      case ASC_F32: fn = pick_fwd_wg<IoF32>(nw, dirs, aln); break;
      case ASC_F16: fn = pick_fwd_wg<IoF16>(nw, dirs, aln); break;
      default: fn = pick_fwd_wg<IoBF16>(nw, dirs, aln); break;
    }
    return launch(fn, items, nw, p, stream);
  }
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = pick_fwd<IoF32>(dirs, aln, wa); break;
    case ASC_F16: fn = pick_fwd<IoF16>(dirs, aln, wa); break;
    default: fn = pick_fwd<IoBF16>(dirs, aln, wa); break;
  }
  return launch(fn, (items + kWPB - 1) / kWPB, kWPB, p, stream);
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
  const int64_t items = p.geo.items * nbranch;
  const int nw = pick_walk(S, T, v, true);
  if (nw) {
    const void* fn = nullptr;
    switch (dtype) {
      case ASC_F32: fn = pick_bwd_wg<IoF32>(nw, dirs, aln); break;
      case ASC_F16: fn = pick_bwd_wg<IoF16>(nw, dirs, aln); break;
      default: fn = pick_bwd_wg<IoBF16>(nw, dirs, aln); break;
    }
    return launch(fn, items, nw, p, stream);
  }
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = pick_bwd<IoF32>(dirs, aln); break;
    case ASC_F16: fn = pick_bwd<IoF16>(dirs, aln); break;
    default: fn = pick_bwd<IoBF16>(dirs, aln); break;
  }
  return launch(fn, (items + kWPB - 1) / kWPB, kWPB, p, stream);
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
  return launch(fn, (p.C * p.chunks + 3) / 4, 4, p, stream);
}

}  // extern "C"
