// libassocscan: gfx950 kernels and C ABI for the first-order linear
// recurrence h[t] = g[t]*h[t-1] + x[t] over packed segments.
//
// Three walks share one sub-tile scan; the host picks one per call:
//   * one wave per (segment, channel) item, carry in a register (short
//     segments, most fp16/bf16 problems, the gate-product output);
//   * one 8- or 16-wave workgroup per item, wave aggregates folded through
//     LDS once per iteration (long segments: fp32, and fp16/bf16 with few
//     items);
//   * decoupled look-back over 16384-element tiles of the flat array (one
//     16-wave workgroup each), carries chained through a caller-provided
//     workspace (few items, e.g. one long sequence).
// Design of the sub-tile scan:
//   * A segment of one row is walked in "sub-tiles" of 64 x 16 bytes: lane l
//     owns one 16-byte vector (4 fp32 or 8 fp16/bf16 elements), so every
//     global load/store instruction of the wave covers 1 KiB contiguously
//     (global_load_dwordx4).  Vectors are aligned in memory; a segment start
//     or end that falls inside a vector is handled by per-element masking on
//     the first and last sub-tile only (the look-back walk, whose tiles
//     may hold several segments, masks every element of a tile that does).
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

#include <type_traits>

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
  __device__ static inline uint32_t bits(float v) { return __float_as_uint(v); }
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
  __device__ static inline uint32_t bits(float v) { return RND(v); }
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
  int64_t pend;    // end of the tensor (phase + C*T): vectors below it read in full
  int64_t v0, v1;  // first / last vector (inclusive)
  int64_t nv;      // number of vectors
  int64_t nsub;    // number of 64-vector sub-tiles
  int64_t kfast;   // sub-tiles [1, kfast) are interior (no masking)

  __device__ inline Walk(int64_t p0, int64_t p1, int64_t pe)
      : P0(p0), P1(p1), pend(pe) {
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
// WIDE: a vector that straddles P0 or P1 but lies inside the tensor (vector
// index >= 1, ends at or below pend) is read with one 16-byte load and
// masked in registers; only the tensor's own first and last vectors are
// read element by element.  (The one-wave walk uses it: for fp16/bf16 items
// with unaligned edges it saves 7 of 8 load instructions per edge vector.
// The workgroup walks do not: the extra branch slowed their loop.)
template <class IO, bool ALN, bool MASKED, bool WIDE = false>
__device__ inline void load_vec(const char* origin, int64_t vi, bool lane_ok,
                                int64_t P0, int64_t P1, float ident,
                                float* f, int64_t pend = 0) {
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
  if (WIDE && ALN && lane_ok && vi >= 1 && pv + V <= pend && pv + V > P0 &&
      pv < P1) {
    IO::unpack(ld16(origin + vi * 16), f);
#pragma unroll
    for (int j = 0; j < V; ++j)
      if (pv + j < P0 || pv + j >= P1) f[j] = ident;
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

// dy of a gradient that is constant along time: value v for the elements
// inside [P0, P1) (of a valid lane), 0 (the identity) elsewhere.
template <class IO, bool MASKED>
__device__ inline void dyc_vec(float v, int64_t vi, bool lane_ok, int64_t P0,
                               int64_t P1, float* f) {
  constexpr int V = IO::V;
  const int64_t pv = vi * V;
#pragma unroll
  for (int j = 0; j < V; ++j)
    f[j] = (!MASKED || (lane_ok && pv + j >= P0 && pv + j < P1)) ? v : 0.0f;
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
  int64_t pend;   // phase + C*T: the tensors end there in the phase frame
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
    load_vec<IO, ALN, MASKED, true>(t.g, vi, ok, w.P0, w.P1, 1.0f, g[u], w.pend);
    load_vec<IO, ALN, MASKED, true>(t.x, vi, ok, w.P0, w.P1, 0.0f, x[u], w.pend);
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
  const Walk<IO, REV> w(P0, P1, t.pend);
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
  int64_t pend;   // phase + C*T: the tensors end there in the phase frame
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

// DYC: the gradient is the constant dyv along the item (dy is not read).
template <class IO, bool RB, bool ALN, bool MASKED, int NS, bool DYC>
__device__ inline void bwd_block(const BwdPtrs& t, const Walk<IO, RB>& w,
                                 int64_t k0, int lane, float& carry,
                                 float& carry_g, float dyv) {
  constexpr int V = IO::V;
  float g[NS][V], dy[NS][V], h[NS][V];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int64_t vi = w.vec(k0 + u, lane);
    const bool ok = !MASKED || w.lane_valid(k0 + u, lane);
    if (DYC)
      dyc_vec<IO, MASKED>(dyv, vi, ok, w.P0, w.P1, dy[u]);
    else
      load_vec<IO, ALN, MASKED, true>(t.dy, vi, ok, w.P0, w.P1, 0.0f, dy[u], w.pend);
    load_vec<IO, ALN, MASKED, true>(t.g, vi, ok, w.P0, w.P1, 1.0f, g[u], w.pend);
    load_vec<IO, ALN, MASKED, true>(t.h, vi, ok, w.P0, w.P1, 0.0f, h[u], w.pend);
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
template <class IO, bool RB, int U, bool DYC>
__device__ inline void bwd_fast(const BwdPtrs& t, const Walk<IO, RB>& w,
                                int64_t k, int64_t kend, int lane,
                                float& carry, float& carry_g, float dyv) {
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
      if (!DYC) y[u] = ld16(yp + u * STEP);
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
      if (DYC) {
#pragma unroll
        for (int j = 0; j < V; ++j) yf[j] = dyv;
      } else {
        IO::unpack(y[u], yf);
      }
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

template <class IO, bool RB, bool ALN, bool DYC>
__device__ void bwd_item(const BwdPtrs& t, int64_t P0, int64_t P1, int lane,
                         float dyv) {
  constexpr int U = ASC_BWD_UNROLL;
  const Walk<IO, RB> w(P0, P1, t.pend);
  float carry = 0.0f, carry_g = 1.0f;
  bwd_block<IO, RB, ALN, true, 1, DYC>(t, w, 0, lane, carry, carry_g, dyv);
  int64_t k = 1;
  if (ALN) {
    const int64_t nfull = (w.kfast - 1) / U * U;
    if (nfull > 0) {
      bwd_fast<IO, RB, U, DYC>(t, w, 1, 1 + nfull, lane, carry, carry_g, dyv);
      k = 1 + nfull;
    }
  } else {
    for (; k + U <= w.kfast; k += U)
      bwd_block<IO, RB, ALN, false, U, DYC>(t, w, k, lane, carry, carry_g, dyv);
  }
  for (; k < w.kfast; ++k)
    bwd_block<IO, RB, ALN, false, 1, DYC>(t, w, k, lane, carry, carry_g, dyv);
  for (; k < w.nsub; ++k)
    bwd_block<IO, RB, ALN, true, 1, DYC>(t, w, k, lane, carry, carry_g, dyv);
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

// Decodes item w; returns false for an empty segment.
// BLOCKS: channels go in blocks of kItemChanBlock; inside a block, items
// w, w+1, ... are one segment of the block's channels, then the next
// segment.  Waves (workgroups) that run at the same time then work on
// segments of equal length in a few neighbouring rows.  One wave per item:
// cfg3 (ragged varlen) 0.95 -> 0.76 ms against row-major order, uniform
// segments within 5% (channel-major order over all C rows gained as much on
// cfg3 but lost 8-14% on uniform segments).  Workgroup walks: +5-12% for
// segments of 8K-32K fp32 elements, -2% from 64K, so the host sets
// the order (the BLK instantiation) from the mean segment length.
// Otherwise: the same segment of neighbouring channels (channel-major).
constexpr int64_t kItemChanBlock = 8;
__device__ inline bool item_range(const Geometry& geo, int64_t w, int& br,
                                  int64_t& P0, int64_t& P1, int64_t& row,
                                  bool blocks) {
  br = w >= geo.items ? 1 : 0;
  const int64_t r = w - br * geo.items;
  int64_t s, c;
  if (blocks) {
    // blocks of kItemChanBlock channels; inside a block the same segment of
    // its channels, then the next segment
    constexpr int64_t CB = kItemChanBlock;
    const int64_t full = (geo.C / CB) * CB * geo.S;
    if (r < full) {
      const int64_t blk = r / (CB * geo.S);
      const int64_t rem = r - blk * CB * geo.S;
      s = rem / CB;
      c = blk * CB + (rem - s * CB);
    } else {
      const int64_t cb = geo.C - (geo.C / CB) * CB;
      const int64_t rem = r - full;
      s = rem / cb;
      c = (geo.C / CB) * CB + (rem - s * cb);
    }
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
  row = c;
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
    int64_t P0, P1, row;
    if (!item_range(p.geo, w, br, P0, P1, row, true)) continue;
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
  int64_t dy_rs;  // DYC: element stride between rows of the gradient
};

// DYC: the gradient of row c is the one value dy[c * dy_rs] (unshifted dy).
template <class IO, bool DYC>
__device__ inline float dyc_value(const BwdParams& p, int br, int64_t row) {
  if (!DYC) return 0.0f;
  return IO::load1(p.br[br].dy + row * p.dy_rs * IO::ES);
}

// DIRS refers to the forward scan being differentiated: 1 = causal forward
// (adjoint runs in reverse), 2 = reverse forward (adjoint runs forward),
// 3 = branch 0 causal / branch 1 reverse.
template <class IO, int DIRS, bool ALN, bool DYC>
__global__ void __launch_bounds__(kWPB* kWave) k_scan_bwd(BwdParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t W = p.geo.items * p.geo.nbranch;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWPB;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * kWPB + wave_id(); w < W;
       w += stride) {
    int br;
    int64_t P0, P1, row;
    if (!item_range(p.geo, w, br, P0, P1, row, true)) continue;
    const BwdPtrs& t = p.br[br];
    const float dyv = dyc_value<IO, DYC>(p, br, row);
    if (DIRS == 1 || (DIRS == 3 && br == 0))
      bwd_item<IO, true, ALN, DYC>(t, P0, P1, lane, dyv);
    else
      bwd_item<IO, false, ALN, DYC>(t, P0, P1, lane, dyv);
  }
}

// Workgroup-cooperative kernels: one item per workgroup of NW waves.
#ifndef ASC_WG_ATTR
#define ASC_WG_ATTR
#endif
// BLK: item order in channel blocks (item_range).
template <class IO, int DIRS, bool ALN, int NW, bool BLK>
__global__ void __launch_bounds__(NW* kWave) ASC_WG_ATTR k_scan_fwd_wg(FwdParams p) {
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
__global__ void __launch_bounds__(NW* kWave) ASC_WG_ATTR k_scan_bwd_wg(BwdParams p) {
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

// Vectorised shift_pad for tensors whose data and out share one phase (the
// usual case): each wave copies a chunk of kShiftVecPerLane * 64 aligned
// 16-byte vectors of one row in a single pass (one-shot, in row order) and
// moves elements by one position in registers: inside a vector by index,
// across lanes by DPP, across the wave's vector groups by readlane, and
// from outside the chunk by a one-element halo load.  Values are moved as
// raw bits (no conversion).  Row ends (the wrap / clamp source) and pad
// positions are patched per element afterwards.
#ifndef ASC_SHIFT_NJ
#define ASC_SHIFT_NJ 4
#endif
constexpr int kShiftVecPerLane = ASC_SHIFT_NJ;
#ifndef ASC_SHIFT_VEC
#define ASC_SHIFT_VEC 1
#endif

struct ShiftVecParams {
  const char* data;  // origins (tensor base - phase * ES)
  char* out;
  const void* cu;
  int cu64;
  int64_t S, C, L;
  int phase;
  int64_t chunks;    // chunks per row
  float pad;         // rounded to the element type on the device
  int backward;
  int wrap;
};

template <class IO>
__device__ inline uint32_t raw_load1(const char* origin, int64_t pos) {
  if (IO::ES == 4) return *reinterpret_cast<const uint32_t*>(origin + pos * 4);
  return *reinterpret_cast<const unsigned short*>(origin + pos * 2);
}
template <class IO>
__device__ inline void raw_store1(char* origin, int64_t pos, uint32_t v) {
  if (IO::ES == 4)
    *reinterpret_cast<uint32_t*>(origin + pos * 4) = v;
  else
    *reinterpret_cast<unsigned short*>(origin + pos * 2) = static_cast<unsigned short>(v);
}
// Element j of a 16-byte vector / set element j.
template <class IO>
__device__ inline uint32_t raw_get(const uint4& q, int j) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if (IO::ES == 4) return w[j];
  return (w[j >> 1] >> (16 * (j & 1))) & 0xffffu;
}
template <class IO>
__device__ inline uint4 raw_pack(const uint32_t* e) {
  if (IO::ES == 4) return make_uint4(e[0], e[1], e[2], e[3]);
  return make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                    e[6] | (e[7] << 16));
}

template <class IO>
__global__ void __launch_bounds__(4 * kWave) k_shift_pad_vec(ShiftVecParams p) {
  constexpr int V = IO::V;
  constexpr int NJ = kShiftVecPerLane;
  constexpr int64_t CHV = static_cast<int64_t>(NJ) * kWave;  // vectors per chunk
  const int lane = threadIdx.x % kWave;
  const int64_t W = p.C * p.chunks;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 4;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + wave_id(); w < W;
       w += stride) {
    const int64_t c = uniform(w / p.chunks);
    const int64_t k = w - c * p.chunks;
    const int64_t r0 = c * p.L + p.phase;  // row [r0, r1) in the phase frame
    const int64_t r1 = r0 + p.L;
    const int64_t vlo = uniform(r0 / V + k * CHV);
    const int64_t vend = (r1 - 1) / V + 1;  // one past the row's last vector
    if (vlo >= vend) continue;
    // load: vector vlo + j*64 + lane; elements outside the row read 0
    uint32_t e[NJ][V];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t vi = vlo + j * kWave + lane;
      const int64_t pv = vi * V;
      uint4 q = make_uint4(0u, 0u, 0u, 0u);
      if (vi < vend) {
        if (pv >= r0 && pv + V <= r1) {
          q = ld16(p.data + vi * 16);
        } else {
          uint32_t t[V];
#pragma unroll
          for (int i = 0; i < V; ++i)
            t[i] = (pv + i >= r0 && pv + i < r1) ? raw_load1<IO>(p.data, pv + i) : 0u;
          q = raw_pack<IO>(t);
        }
      }
#pragma unroll
      for (int i = 0; i < V; ++i) e[j][i] = raw_get<IO>(q, i);
    }
    // shifted values
    uint32_t o[NJ][V];
    if (p.backward) {
      // out[P] = in[P - 1]; the element before the chunk is a halo
      const int64_t hp = vlo * V - 1;
      const uint32_t halo = hp >= r0 ? raw_load1<IO>(p.data, hp) : 0u;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const uint32_t prev_last =
            j == 0 ? halo : static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(e[j - 1][V - 1]), kWave - 1));
        const uint32_t from_left = static_cast<uint32_t>(
            __builtin_amdgcn_update_dpp(static_cast<int>(prev_last), static_cast<int>(e[j][V - 1]),
                                        kWaveShr1, 0xf, 0xf, false));
        o[j][0] = from_left;
#pragma unroll
        for (int i = 1; i < V; ++i) o[j][i] = e[j][i - 1];
      }
    } else {
      // out[P] = in[P + 1]; the element after the chunk is a halo
      const int64_t hp = (vlo + CHV) * V;
      const uint32_t halo = hp < r1 ? raw_load1<IO>(p.data, hp) : 0u;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const uint32_t next_first =
            j == NJ - 1 ? halo : static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(e[j + 1][0]), 0));
        const uint32_t from_right = static_cast<uint32_t>(
            __builtin_amdgcn_update_dpp(static_cast<int>(next_first), static_cast<int>(e[j][0]),
                                        kWaveShl1, 0xf, 0xf, false));
#pragma unroll
        for (int i = 0; i < V - 1; ++i) o[j][i] = e[j][i + 1];
        o[j][V - 1] = from_right;
      }
    }
    // patch one element (row offset t) if this wave holds it
    auto patch = [&](int64_t t, uint32_t v) {
      const int64_t pos = r0 + t;
      const int64_t off = pos / V - vlo;
      if (off < 0 || off >= CHV) return;
      const int j = static_cast<int>(off / kWave);
      const int l = static_cast<int>(off % kWave);
      const int i = static_cast<int>(pos - (pos / V) * V);
      if (lane != l) return;
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int ii = 0; ii < V; ++ii)
          if (jj == j && ii == i) o[jj][ii] = v;
    };
    const int64_t t_lo = vlo * V - r0;        // row offsets covered (may be < 0)
    const int64_t t_hi = (vlo + CHV) * V - r0;  // exclusive (may be > L)
    // the row end whose neighbour lies outside the row: wrap or clamp
    if (p.backward) {
      if (t_lo <= 0 && 0 < t_hi)
        patch(0, raw_load1<IO>(p.data, p.wrap ? r1 - 1 : r0));
    } else {
      if (t_lo <= p.L - 1 && p.L - 1 < t_hi)
        patch(p.L - 1, raw_load1<IO>(p.data, p.wrap ? r0 : r1 - 1));
    }
    // pad positions: first boundary >= t_lo, then every one below t_hi
    const uint32_t pad_bits = IO::bits(p.pad);
    const ShiftParams bp{nullptr, nullptr, p.cu, p.cu64, p.S, p.C, p.L, 0, 0.0f,
                         p.backward, p.wrap};
    int64_t lo = 0, hi = p.S;
    while (lo < hi) {
      const int64_t mid = (lo + hi) / 2;
      if (shift_boundary(bp, mid) < t_lo)
        lo = mid + 1;
      else
        hi = mid;
    }
    for (int64_t kk = lo; kk < p.S; ++kk) {
      const int64_t q = shift_boundary(bp, kk);
      if (q >= t_hi) break;
      if (q >= 0 && q < p.L) patch(q, pad_bits);
    }
    // a negative boundary (end of a zero-length first segment) counts from
    // the row end, as torch indexing does in the reference
    for (int64_t kk = 0; kk < p.S; ++kk) {
      const int64_t q = shift_boundary(bp, kk);
      if (q >= 0) break;
      if (q + p.L >= t_lo && q + p.L < t_hi && q + p.L >= 0) patch(q + p.L, pad_bits);
    }
    // store the elements inside the row
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t vi = vlo + j * kWave + lane;
      const int64_t pv = vi * V;
      if (vi >= vend) continue;
      if (pv >= r0 && pv + V <= r1) {
        st16(p.out + vi * 16, raw_pack<IO>(o[j]));
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i)
          if (pv + i >= r0 && pv + i < r1) raw_store1<IO>(p.out, pv + i, o[j][i]);
      }
    }
  }
}

// ===========================================================================
// Decoupled look-back walk (single pass over in-order tiles).
//
// The walks above give each (segment, channel) item to one wave or one
// workgroup, so a problem with few items (one long sequence, a handful of
// channels) leaves most of the 256 CUs idle.  This walk cuts the flat array
// of all rows into tiles of 16384 elements instead, so its parallelism is
// the element count.  Workgroup b (kLbWaves waves) owns tile b in scan order
// (address order, or reverse address order for a reverse-direction scan);
// wave w owns part w of it, 1024 elements.  A part may hold the end of one
// segment and the start of others (or the end of one row and the start of
// the next): segment heads reset the scan inside it.  Each tile
//   1. loads its data and scans it locally, one part per wave, and the part
//      maps meet in LDS;
//   2. (wave 0) publishes the tile's aggregate map (A, X) in its workspace
//      slot -- or, if a segment starts inside the tile, directly its
//      inclusive value, which no longer depends on earlier tiles;
//   3. (wave 0) unless its first element in a segment is a head, looks back
//      over the slots of the preceding tiles, 64 at a time (one per lane),
//      composing aggregates with the same DPP scan until it meets an
//      inclusive value, and publishes its own inclusive value;
//   4. every wave takes the tile carry through the parts before its own and
//      writes its outputs.
// Slot words are (status << 32 | float bits), written and read with
// agent-scope atomics (the 8 XCDs have separate L2 caches, so every poll is
// a round trip past them); the workspace is zero-filled by a small kernel
// before every launch.  Every wait is bounded: after g_spin_limit (2^14 by
// default) unsuccessful polls the waiting wave computes the missing
// predecessor's map from that tile's inputs itself, so progress never
// depends on the order in which workgroups are scheduled.
//
// Measured on MI355X, a poll round trip under full HBM load costs about as
// much as a tile's own loads, so with many items the per-item walks (which
// need no inter-workgroup communication) stream faster; the host picks this
// walk only for problems with few items (lb_use).  Which predecessor a tile
// meets as inclusive depends on timing, so the last bits of the results can
// vary from run to run.
// ===========================================================================
// Parts are 1024 elements for every element type: 4 sub-tiles of 64 lanes x
// 4 fp32, or 2 sub-tiles of 64 lanes x 8 fp16/bf16 (ASC_LB_U_F32 sets the
// fp32 part for experiments).
#ifndef ASC_LB_U_F32
#define ASC_LB_U_F32 4
#endif
template <class IO>
constexpr int LbU = IO::V == 4 ? ASC_LB_U_F32 : 2;  // sub-tiles per part
template <class IO>
constexpr int64_t LbTileVec = static_cast<int64_t>(LbU<IO>) * kWave;  // per part
// 16 waves (16384-element tiles): a poll costs the same for any tile size,
// so fewer, larger tiles stream faster (measured with one 2^27-element row:
// 4.1 / 4.7 TB/s fwd / bwd fp32 against 3.3 / 4.0 with 4 waves; 8 waves
// were no better than 4 at the occupancy their register use allows).
#ifndef ASC_LB_WAVES
#define ASC_LB_WAVES 16
#endif
constexpr int kLbWaves = ASC_LB_WAVES;  // parts (waves) per workgroup tile
// Elements per part for v elements per vector (host side; matches LbU).
constexpr int64_t lb_part_elems(int v) {
  return v == 4 ? 256 * ASC_LB_U_F32 : 2 * 512;
}

typedef unsigned long long u64;
// One carry slot per tile, two tagged words: x holds (status << 32 | value)
// with status kLbAgg (the tile's aggregate X) or kLbIncl (its inclusive
// value, the state after the tile); a holds (kLbAgg << 32 | A).  Each word is
// read and written whole, so a reader never sees a value without its tag.
struct LbSlot {
  u64 x, a;
};
enum : uint32_t { kLbNone = 0, kLbAgg = 1, kLbIncl = 2 };

__device__ inline void lb_put(u64* p, uint32_t st, float v) {
  const u64 w = (static_cast<u64>(st) << 32) | __float_as_uint(v);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline u64 lb_get(u64* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t lb_status(u64 w) { return static_cast<uint32_t>(w >> 32); }
__device__ inline float lb_value(u64 w) {
  return __uint_as_float(static_cast<uint32_t>(w));
}
// Both words of a slot in one round trip; returns the slot's kind.
__device__ inline int lb_read(LbSlot* s, float& a, float& x) {
  const u64 wx = lb_get(&s->x);
  const u64 wa = lb_get(&s->a);
  x = lb_value(wx);
  a = lb_value(wa);
  const uint32_t sx = lb_status(wx);
  if (sx == kLbIncl) return kLbIncl;
  return (sx == kLbAgg && lb_status(wa) == kLbAgg) ? kLbAgg : kLbNone;
}

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

// Vector owned by `lane` in sub-tile u of tile t (scan order).
template <class IO, bool REV>
__device__ inline int64_t lb_vec(const LbGeo& g, int64_t t, int u, int lane) {
  const int64_t i = t * LbTileVec<IO> + static_cast<int64_t>(u) * kWave + lane;
  return REV ? g.nvec - 1 - i : i;
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

template <class IO, bool REV>
__device__ inline LbTile lb_classify(const LbGeo& g, int64_t t) {
  constexpr int V = IO::V;
  LbTile r{false, -1, -1, 0, 0, 0};
  const int64_t v_lo = REV ? g.nvec - (t + 1) * LbTileVec<IO> : t * LbTileVec<IO>;
  const int64_t e_lo = uniform(v_lo * V - g.phase);
  const int64_t e_hi = e_lo + LbTileVec<IO> * V;
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
  const int64_t hd = REV ? ce - 1 : cs;   // segment's first scan element
  const int64_t tl_ = REV ? cs : ce - 1;  // segment's last scan element
  if (hd == (REV ? th - 1 : tl)) r.phead = base + hd;
  if (tl_ == (REV ? tl : th - 1)) r.ptail = base + tl_;
  return r;
}

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

// Per-tile scan state of the forward kernel.
template <class IO>
struct FwdTile {
  float g[LbU<IO>][IO::V], x[LbU<IO>][IO::V];
  uint32_t valid[LbU<IO>], head[LbU<IO>];
  SegScan sc[LbU<IO>];
  float A, X;
  int F;
  bool need_carry;
  bool any;  // some element of the part lies in a segment
};

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

// Whether the tile needs a carry: it does unless the first element (scan
// order) that lies in a segment is a segment head.  Slow path only.
template <class IO, bool REV>
__device__ inline bool lb_needs_carry(const uint32_t* valid, const uint32_t* head) {
  constexpr int V = IO::V;
#pragma unroll
  for (int u = 0; u < LbU<IO>; ++u) {
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

// Loads and scans tile t locally (no stores); fills the tile map.  The data
// loads depend on the tensor bounds only, so they are issued before the
// segment lookup and their latency covers it.
template <class IO, bool REV, bool ALN>
__device__ inline void fwd_tile_local(const FwdPtrs& p, const LbGeo& geo,
                                      int64_t t, int lane, FwdTile<IO>& s) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  uint32_t inten[LbU<IO>];
#pragma unroll
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    inten[u] = lb_inten<IO>(geo, vi);
    lb_load<IO, ALN>(p.g, vi, inten[u], 1.0f, s.g[u]);
    lb_load<IO, ALN>(p.x, vi, inten[u], 0.0f, s.x[u]);
  }
  const LbTile ti = lb_classify<IO, REV>(geo, t);
  s.A = 1.0f;
  s.X = 0.0f;
  s.F = 0;
  if (ti.fast) {
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      s.valid[u] = full;
      s.head[u] = 0;
    }
    if (ti.phead >= 0 && lane == 0) s.head[0] = 1u << mem_idx<V, REV>(0);
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      const int64_t pv = lb_vec<IO, REV>(geo, t, u, lane) * V;
      SubScan ss;
      if (u == 0)
        ss = fwd_local<IO, REV, true>(s.g[u], s.x[u], pv, ti.phead);
      else
        ss = fwd_local<IO, REV, false>(s.g[u], s.x[u], pv, -1);
      s.sc[u] = seg_from(ss, u == 0 && ti.phead >= 0);
      lb_compose(s.A, s.X, s.F, s.sc[u].ta, s.sc[u].tx, s.sc[u].tf);
    }
    s.need_carry = ti.phead < 0;
    s.any = true;
    return;
  }
  uint32_t anyv = 0;
#pragma unroll
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    uint32_t in2, tail;
    lb_flags<IO, REV>(geo, ti, vi, in2, s.valid[u], s.head[u], tail);
    anyv |= s.valid[u];
    s.sc[u] = fwd_local_seg<IO, REV>(s.g[u], s.x[u], s.valid[u], s.head[u]);
    lb_compose(s.A, s.X, s.F, s.sc[u].ta, s.sc[u].tx, s.sc[u].tf);
  }
  s.need_carry = lb_needs_carry<IO, REV>(s.valid, s.head);
  s.any = __builtin_amdgcn_ballot_w64(anyv != 0) != 0;
}

// Composes the maps of the tiles before t (scan order) until an inclusive
// value; returns the carry into tile t.  Window of 64 tiles: lane r polls
// tile top - 63 + r, so lane 63 is the nearest and one DPP scan composes
// the window in scan order.  (Wider windows, several slots per lane, were
// slower: every extra slot is another device-coherent load per poll.)
// `compute(j, A, X, F)` recomputes tile j's map from its inputs (the
// bounded-wait fallback).
template <class Compute>
__device__ float lb_lookback(const LbGeo& geo, LbSlot* slots, int64_t t,
                             int lane, Compute compute) {
  float acc_a = 1.0f, acc_x = 0.0f;
  int64_t top = t - 1;
  uint32_t spins = 0;
  while (true) {
    const int64_t j = top - (kWave - 1) + lane;
    float a, x;
    int kind = lb_read(&slots[j < 0 ? 0 : j], a, x);
    if (j < 0) {  // before the first tile: inclusive 0
      kind = kLbIncl;
      x = 0.0f;
    }
    u64 incl = __builtin_amdgcn_ballot_w64(kind == kLbIncl);
    int r_inc = incl ? 63 - __builtin_clzll(incl) : -1;
    u64 above = r_inc >= 63 ? 0ull : (~0ull << (r_inc + 1));
    u64 missing = __builtin_amdgcn_ballot_w64(kind == kLbNone) & above;
    if (missing) {
      if (++spins <= geo.spin_limit) {
        __builtin_amdgcn_s_sleep(2);
        continue;
      }
      // Bounded wait expired: compute the missing maps from the tiles'
      // inputs, nearest first (a tile with a segment head is inclusive).
      while (missing) {
        const int r = 63 - __builtin_clzll(missing);
        float ma, mx;
        int mf;
        compute(top - (kWave - 1) + r, ma, mx, mf);
        if (lane == r) {
          kind = mf ? kLbIncl : kLbAgg;
          a = ma;
          x = mx;
        }
        incl = __builtin_amdgcn_ballot_w64(kind == kLbIncl);
        r_inc = incl ? 63 - __builtin_clzll(incl) : -1;
        above = r_inc >= 63 ? 0ull : (~0ull << (r_inc + 1));
        missing = __builtin_amdgcn_ballot_w64(kind == kLbNone) & above;
      }
      spins = 0;
    }
    float ma = a, mx = x;
    if (lane < r_inc) {
      ma = 1.0f;
      mx = 0.0f;
    } else if (lane == r_inc) {
      ma = 0.0f;
    }
    wave_scan_affine(ma, mx);
    const float ra = readlane(ma, kWave - 1);
    const float rx = readlane(mx, kWave - 1);
    acc_x = fmaf(acc_a, rx, acc_x);
    acc_a = acc_a * ra;
    if (r_inc >= 0) return acc_x;
    top -= kWave;
  }
}

// The map (A, X, F) of tile t computed from its inputs one sub-tile at a
// time (the bounded-wait fallback of the look-back; nothing is stored).
template <class IO, bool REV, bool ALN>
__device__ __attribute__((noinline)) void fwd_tile_map(const FwdPtrs p, const LbGeo geo,
                                                       int64_t t, int lane, float& A,
                                                       float& X, int& F) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  const LbTile ti = lb_classify<IO, REV>(geo, t);
  A = 1.0f;
  X = 0.0f;
  F = 0;
#pragma unroll 1
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    float g[V], x[V];
    if (ti.fast) {
      lb_load<IO, ALN>(p.g, vi, full, 1.0f, g);
      lb_load<IO, ALN>(p.x, vi, full, 0.0f, x);
      const SubScan ss = fwd_local<IO, REV, true>(g, x, vi * V,
                                                  u == 0 ? ti.phead : -1);
      lb_compose(A, X, F, ss.ta, ss.tx, u == 0 && ti.phead >= 0);
    } else {
      uint32_t inten, valid, head, tail;
      lb_flags<IO, REV>(geo, ti, vi, inten, valid, head, tail);
      lb_load<IO, ALN>(p.g, vi, inten, 1.0f, g);
      lb_load<IO, ALN>(p.x, vi, inten, 0.0f, x);
      const SegScan sc = fwd_local_seg<IO, REV>(g, x, valid, head);
      lb_compose(A, X, F, sc.ta, sc.tx, sc.tf);
    }
  }
}

// A workgroup tile is kLbWaves consecutive parts, one per wave.  The waves
// share their part maps through LDS; wave 0 composes them into the tile
// map, publishes it, looks back and hands the tile's carry-in to the others.
struct LbPart {
  float a, x;
  int f;      // a segment head lies inside the part
  int flags;  // bit 1: some element lies in a segment; bit 0: needs a carry
};

// Tile map (A, X, F) from the parts and whether the tile needs a carry (the
// first part that holds segment elements needs one).
__device__ inline bool lb_tile_from_parts(const LbPart* parts, float& A,
                                          float& X, int& F) {
  A = 1.0f;
  X = 0.0f;
  F = 0;
  int nc = -1;
#pragma unroll
  for (int k = 0; k < kLbWaves; ++k) {
    const LbPart q = parts[k];
    lb_compose(A, X, F, q.a, q.x, q.f);
    if (nc < 0 && (q.flags & 2)) nc = q.flags & 1;
  }
  return nc > 0;
}

// Carry into part wv from the tile's carry-in.
__device__ inline float lb_part_carry(const LbPart* parts, int wv, float carry) {
  for (int k = 0; k < wv; ++k) {
    const LbPart q = parts[k];
    carry = q.f ? q.x : fmaf(q.a, carry, q.x);
  }
  return carry;
}

struct LbFwdParams {
  LbGeo geo;
  FwdPtrs br[2];
  LbSlot* slots;  // nbranch * ntiles
};

template <class IO, int DIRS, bool ALN>
__global__ void __launch_bounds__(kLbWaves* kWave) k_scan_fwd_lb(LbFwdParams p) {
  __shared__ LbPart parts[kLbWaves];
  __shared__ float tile_carry;
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  const int64_t gt = blockIdx.x;
  const int br = gt >= p.geo.ntiles ? 1 : 0;
  const int64_t t = gt - br * p.geo.ntiles;
  if (br >= p.geo.nbranch) return;  // whole workgroup
  LbSlot* slots = p.slots + br * p.geo.ntiles;
  auto run = [&](auto rev_tag) {
    constexpr bool REV = decltype(rev_tag)::value;
    constexpr int V = IO::V;
    const FwdPtrs q = p.br[br];
    FwdTile<IO> s;
    fwd_tile_local<IO, REV, ALN>(q, p.geo, t * kLbWaves + wv, lane, s);
    if (lane == 0)
      parts[wv] = LbPart{s.A, s.X, s.F, (s.any ? 2 : 0) | (s.need_carry ? 1 : 0)};
    __syncthreads();
    if (wv == 0) {
      float A, X;
      int F;
      const bool need = lb_tile_from_parts(parts, A, X, F);
      if (lane == 0) {
        if (F) {
          lb_put(&slots[t].x, kLbIncl, X);
        } else {
          lb_put(&slots[t].a, kLbAgg, A);
          lb_put(&slots[t].x, kLbAgg, X);
        }
      }
      float carry = 0.0f;
      if (need)
        carry = lb_lookback(p.geo, slots, t, lane,
                            [&](int64_t j, float& a, float& x, int& f) {
                              a = 1.0f;
                              x = 0.0f;
                              f = 0;
                              for (int k = 0; k < kLbWaves; ++k) {
                                float ma, mx;
                                int mf;
                                fwd_tile_map<IO, REV, ALN>(q, p.geo, j * kLbWaves + k,
                                                           lane, ma, mx, mf);
                                lb_compose(a, x, f, ma, mx, mf);
                              }
                            });
      if (lane == 0) {
        if (!F) lb_put(&slots[t].x, kLbIncl, fmaf(A, carry, X));
        tile_carry = carry;
      }
    }
    __syncthreads();
    float carry = lb_part_carry(parts, wv, tile_carry);
    const int64_t pt = t * kLbWaves + wv;
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      const int64_t vi = lb_vec<IO, REV>(p.geo, pt, u, lane);
      float hf[V];
      fwd_apply_seg<IO, REV>(s.g[u], s.x[u], s.valid[u], s.head[u], s.sc[u],
                             carry, hf);
      lb_store<IO, ALN>(q.h, vi, s.valid[u], hf);
      carry = seg_apply_total(s.sc[u].ta, s.sc[u].tx, s.sc[u].tf, carry);
    }
  };
  if (DIRS == 1 || (DIRS == 3 && br == 0))
    run(std::integral_constant<bool, false>{});
  else
    run(std::integral_constant<bool, true>{});
}

// Per-tile scan state of the backward kernel (B order = REV).
template <class IO>
struct BwdTile {
  float y[LbU<IO>][IO::V], g[LbU<IO>][IO::V], h[LbU<IO>][IO::V];
  uint32_t valid[LbU<IO>], head[LbU<IO>], tail[LbU<IO>];
  float gprev[LbU<IO>];
  SegScan sc[LbU<IO>];
  float hn;  // state just after the part in B order (0 outside the tensor)
  float A, X;
  int F;
  bool need_carry;
  bool any;  // some element of the part lies in a segment
};

template <class IO, bool REV, bool ALN>
__device__ inline void bwd_tile_local(const BwdPtrs& p, const LbGeo& geo,
                                      int64_t t, int lane, BwdTile<IO>& s) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  constexpr int jl = mem_idx<V, REV>(V - 1);
  // data and halos first (tensor bounds only): the gate before the tile and
  // the state after it (B order)
  uint32_t inten[LbU<IO>];
#pragma unroll
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    inten[u] = lb_inten<IO>(geo, vi);
    lb_load<IO, ALN>(p.dy, vi, inten[u], 0.0f, s.y[u]);
    lb_load<IO, ALN>(p.g, vi, inten[u], 1.0f, s.g[u]);
    lb_load<IO, ALN>(p.h, vi, inten[u], 0.0f, s.h[u]);
  }
  float cg = 1.0f;
  {
    const int64_t pf = lb_vec<IO, REV>(geo, t, 0, 0) * V + mem_idx<V, REV>(0);
    const int64_t pp = REV ? pf + 1 : pf - 1;
    const int64_t e = pp - geo.phase;
    if (e >= 0 && e < geo.n) cg = IO::load1(p.g + pp * IO::ES);
    const int64_t pl =
        lb_vec<IO, REV>(geo, t, LbU<IO> - 1, kWave - 1) * V + mem_idx<V, REV>(V - 1);
    const int64_t pn = REV ? pl - 1 : pl + 1;
    const int64_t en = pn - geo.phase;
    s.hn = (en >= 0 && en < geo.n) ? IO::load1(p.h + pn * IO::ES) : 0.0f;
  }
  const LbTile ti = lb_classify<IO, REV>(geo, t);
  s.A = 1.0f;
  s.X = 0.0f;
  s.F = 0;
  if (ti.fast) {
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      s.valid[u] = full;
      s.head[u] = 0;
      s.tail[u] = 0;
    }
    if (ti.phead >= 0 && lane == 0) s.head[0] = 1u << mem_idx<V, REV>(0);
    if (ti.ptail >= 0 && lane == kWave - 1)
      s.tail[LbU<IO> - 1] = 1u << mem_idx<V, REV>(V - 1);
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      const int64_t pv = lb_vec<IO, REV>(geo, t, u, lane) * V;
      SubScan ss;
      if (u == 0)
        ss = bwd_local<IO, REV, true>(s.g[u], s.y[u], pv, ti.phead, cg, s.gprev[u]);
      else
        ss = bwd_local<IO, REV, false>(s.g[u], s.y[u], pv, -1, cg, s.gprev[u]);
      cg = readlane(s.g[u][jl], kWave - 1);
      s.sc[u] = seg_from(ss, u == 0 && ti.phead >= 0);
      lb_compose(s.A, s.X, s.F, s.sc[u].ta, s.sc[u].tx, s.sc[u].tf);
    }
    s.need_carry = ti.phead < 0;
    s.any = true;
    return;
  }
  uint32_t anyv = 0;
#pragma unroll
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    uint32_t in2;
    lb_flags<IO, REV>(geo, ti, vi, in2, s.valid[u], s.head[u], s.tail[u]);
    anyv |= s.valid[u];
    s.sc[u] = bwd_local_seg<IO, REV>(s.g[u], s.y[u], s.valid[u], s.head[u], cg,
                                     s.gprev[u]);
    cg = readlane(s.g[u][jl], kWave - 1);
    lb_compose(s.A, s.X, s.F, s.sc[u].ta, s.sc[u].tx, s.sc[u].tf);
  }
  s.need_carry = lb_needs_carry<IO, REV>(s.valid, s.head);
  s.any = __builtin_amdgcn_ballot_w64(anyv != 0) != 0;
}

template <class IO, bool REV, bool ALN>
__device__ __attribute__((noinline)) void bwd_tile_map(const BwdPtrs p, const LbGeo geo,
                                                       int64_t t, int lane, float& A,
                                                       float& X, int& F) {
  constexpr int V = IO::V;
  constexpr uint32_t full = (1u << V) - 1;
  constexpr int jl = mem_idx<V, REV>(V - 1);
  const LbTile ti = lb_classify<IO, REV>(geo, t);
  float cg = 1.0f;
  {
    const int64_t pf = lb_vec<IO, REV>(geo, t, 0, 0) * V + mem_idx<V, REV>(0);
    const int64_t pp = REV ? pf + 1 : pf - 1;
    const int64_t e = pp - geo.phase;
    if (e >= 0 && e < geo.n) cg = IO::load1(p.g + pp * IO::ES);
  }
  A = 1.0f;
  X = 0.0f;
  F = 0;
#pragma unroll 1
  for (int u = 0; u < LbU<IO>; ++u) {
    const int64_t vi = lb_vec<IO, REV>(geo, t, u, lane);
    float g[V], y[V], gprev;
    if (ti.fast) {
      lb_load<IO, ALN>(p.g, vi, full, 1.0f, g);
      lb_load<IO, ALN>(p.dy, vi, full, 0.0f, y);
      const SubScan ss = bwd_local<IO, REV, true>(g, y, vi * V,
                                                  u == 0 ? ti.phead : -1, cg, gprev);
      lb_compose(A, X, F, ss.ta, ss.tx, u == 0 && ti.phead >= 0);
    } else {
      uint32_t inten, valid, head, tail;
      lb_flags<IO, REV>(geo, ti, vi, inten, valid, head, tail);
      lb_load<IO, ALN>(p.g, vi, inten, 1.0f, g);
      lb_load<IO, ALN>(p.dy, vi, inten, 0.0f, y);
      const SegScan sc = bwd_local_seg<IO, REV>(g, y, valid, head, cg, gprev);
      lb_compose(A, X, F, sc.ta, sc.tx, sc.tf);
    }
    cg = readlane(g[jl], kWave - 1);
  }
}

struct LbBwdParams {
  LbGeo geo;
  BwdPtrs br[2];
  LbSlot* slots;
};

// DIRS as k_scan_bwd: 1 = causal (B order reverse), 2 = anti-causal,
// 3 = branch 0 causal / branch 1 anti-causal.
template <class IO, int DIRS, bool ALN>
__global__ void __launch_bounds__(kLbWaves* kWave) k_scan_bwd_lb(LbBwdParams p) {
  __shared__ LbPart parts[kLbWaves];
  __shared__ float tile_carry;
  const int lane = threadIdx.x % kWave;
  const int wv = wave_id();
  const int64_t gt = blockIdx.x;
  const int br = gt >= p.geo.ntiles ? 1 : 0;
  const int64_t t = gt - br * p.geo.ntiles;
  if (br >= p.geo.nbranch) return;  // whole workgroup
  LbSlot* slots = p.slots + br * p.geo.ntiles;
  auto run = [&](auto rev_tag) {
    constexpr bool REV = decltype(rev_tag)::value;
    constexpr int V = IO::V;
    constexpr int jf = mem_idx<V, REV>(0);
    const BwdPtrs q = p.br[br];
    const int64_t pt = t * kLbWaves + wv;
    BwdTile<IO> s;
    bwd_tile_local<IO, REV, ALN>(q, p.geo, pt, lane, s);
    if (lane == 0)
      parts[wv] = LbPart{s.A, s.X, s.F, (s.any ? 2 : 0) | (s.need_carry ? 1 : 0)};
    __syncthreads();
    if (wv == 0) {
      float A, X;
      int F;
      const bool need = lb_tile_from_parts(parts, A, X, F);
      if (lane == 0) {
        if (F) {
          lb_put(&slots[t].x, kLbIncl, X);
        } else {
          lb_put(&slots[t].a, kLbAgg, A);
          lb_put(&slots[t].x, kLbAgg, X);
        }
      }
      float carry = 0.0f;
      if (need)
        carry = lb_lookback(p.geo, slots, t, lane,
                            [&](int64_t j, float& a, float& x, int& f) {
                              a = 1.0f;
                              x = 0.0f;
                              f = 0;
                              for (int k = 0; k < kLbWaves; ++k) {
                                float ma, mx;
                                int mf;
                                bwd_tile_map<IO, REV, ALN>(q, p.geo, j * kLbWaves + k,
                                                           lane, ma, mx, mf);
                                lb_compose(a, x, f, ma, mx, mf);
                              }
                            });
      if (lane == 0) {
        if (!F) lb_put(&slots[t].x, kLbIncl, fmaf(A, carry, X));
        tile_carry = carry;
      }
    }
    __syncthreads();
    float carry = lb_part_carry(parts, wv, tile_carry);
#pragma unroll
    for (int u = 0; u < LbU<IO>; ++u) {
      const int64_t vi = lb_vec<IO, REV>(p.geo, pt, u, lane);
      const float hin = (u + 1 < LbU<IO>) ? readlane(s.h[u + 1][jf], 0) : s.hn;
      float dx[V], dg[V];
      bwd_apply_seg<IO, REV>(s.g[u], s.y[u], s.h[u], s.valid[u], s.head[u],
                             s.tail[u], s.gprev[u], hin, s.sc[u], carry, dx, dg);
      lb_store<IO, ALN>(q.dx, vi, s.valid[u], dx);
      lb_store<IO, ALN>(q.dg, vi, s.valid[u], dg);
      carry = seg_apply_total(s.sc[u].ta, s.sc[u].tx, s.sc[u].tf, carry);
    }
  };
  if (DIRS == 1 || (DIRS == 3 && br == 0))
    run(std::integral_constant<bool, true>{});
  else
    run(std::integral_constant<bool, false>{});
}

__global__ void __launch_bounds__(256) k_fill_zero(u64* p, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += stride)
    p[i] = 0;
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

// Look-back walk: polls before a waiting wave computes a missing
// predecessor itself (a test hook can lower it to exercise that path).
uint32_t g_spin_limit = 1u << 14;

// One workgroup per tile and no grid-stride loop: every tile needs its own
// workgroup.
bool lb_grid_fits(int64_t tiles) { return tiles <= kMaxGrid; }

// Tiles of the look-back walk: kLbWaves parts each, from the start of the
// phase frame (the vectors of every element type divide 1024).
int64_t lb_ntiles(int64_t n, int phase, int v) {
  const int64_t te = lb_part_elems(v) * kLbWaves;
  return (phase + n + te - 1) / te;
}

// Workspace bytes for the worst-case phase (v - 1).
int64_t lb_bytes(int64_t n, int v, int nbranch) {
  return lb_ntiles(n, v - 1, v) * nbranch * static_cast<int64_t>(sizeof(LbSlot));
}

// Walk choice: the look-back walk for problems with few (segment, channel)
// items (each item of the other walks is one wave or one workgroup, which
// leaves most CUs idle), the per-item walks otherwise.  Measured on MI355X
// (2^27 elements): the look-back walk streams about 4.1 / 4.7 TB/s (fwd /
// bwd) fp32 and 2.4 / 3.0 bf16 at any item count; 16-wave workgroups per
// item reach 2.4 / 2.6 (fp32) and 1.5 / 1.3 (bf16) at 64 items, 4.4 / 4.6
// and 2.8 / 2.3 at 128, and overtake beyond.  The look-back kernels also
// keep row offsets and segment indices in 32 bits, and need one workgroup
// per tile.
#ifndef ASC_LB_MAX_ITEMS_F32
#define ASC_LB_MAX_ITEMS_F32 128
#endif
#ifndef ASC_LB_MAX_ITEMS_HALF
#define ASC_LB_MAX_ITEMS_HALF 128
#endif
bool lb_use(int64_t S, int64_t C, int64_t T, int nbranch, int v) {
  if (S <= 0 || C <= 0 || T <= 0) return false;
  if (T >= (int64_t(1) << 30) || S >= (int64_t(1) << 30)) return false;
  const int64_t max_items = v == 4 ? ASC_LB_MAX_ITEMS_F32 : ASC_LB_MAX_ITEMS_HALF;
  if (S * C * nbranch > max_items) return false;
  return lb_grid_fits(lb_ntiles(C * T, v - 1, v) * nbranch);
}

int fill_zero(void* ws, int64_t bytes, void* stream) {
  const int64_t words = bytes / 8;
  int64_t blocks = (words + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  u64* p = static_cast<u64*>(ws);
  int64_t n = words;
  void* args[] = {&p, &n};
  const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&k_fill_zero),
                                       dim3(static_cast<unsigned>(blocks)), dim3(256),
                                       args, 0, static_cast<hipStream_t>(stream));
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
#ifndef ASC_HALF_WG_MAX_ITEMS
#define ASC_HALF_WG_MAX_ITEMS 512
#endif
int pick_walk(int64_t S, int64_t C, int64_t T, int nbranch, int v, bool bwd) {
  const int64_t mean = T / (S > 0 ? S : 1);
  const int64_t tile1 = static_cast<int64_t>(kUW) * kWave * v;  // per wave
  if (v != 4) {
    // fp16/bf16: the workgroup walks hold 8 elements per lane in each of
    // their ping-pong buffers (128+ VGPRs, spills in the backward), so one
    // wave per item streams faster once there are enough items to fill the
    // chip (bf16, 64K segments x 12288 items: 5.3 vs 4.6 TB/s forward, 5.3
    // vs 3.8 backward).  With fewer than 512 long items it leaves SIMDs
    // idle and 16 waves per item win (bf16, 256 items of 512K: 4.9 / 3.3
    // against 2.7 / 2.2 TB/s; even at 512 items).
    const int64_t items = S * C * nbranch;
    return items < ASC_HALF_WG_MAX_ITEMS && mean >= 16 * 16 * tile1 ? 16 : 0;
  }
  const int64_t it16 = bwd ? ASC_BWD_WG16_MIN_ITERS : ASC_FWD_WG16_MIN_ITERS;
  if (mean >= it16 * 16 * tile1) return 16;
  if (mean >= static_cast<int64_t>(ASC_WG8_MIN_ITERS) * 8 * tile1) return 8;
  return 0;
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
  if (dyc) {  // single-branch calls only
    if (dirs == 1) return aln ? ASC_B(1, true, true) : ASC_B(1, false, true);
    return aln ? ASC_B(2, true, true) : ASC_B(2, false, true);
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

template <class IO>
const void* pick_fwd_lb(int dirs, bool aln) {
#define ASC_F(D, A) reinterpret_cast<const void*>(&k_scan_fwd_lb<IO, D, A>)
  if (dirs == 1) return aln ? ASC_F(1, true) : ASC_F(1, false);
  if (dirs == 2) return aln ? ASC_F(2, true) : ASC_F(2, false);
  return aln ? ASC_F(3, true) : ASC_F(3, false);
#undef ASC_F
}

template <class IO>
const void* pick_bwd_lb(int dirs, bool aln) {
#define ASC_B(D, A) reinterpret_cast<const void*>(&k_scan_bwd_lb<IO, D, A>)
  if (dirs == 1) return aln ? ASC_B(1, true) : ASC_B(1, false);
  if (dirs == 2) return aln ? ASC_B(2, true) : ASC_B(2, false);
  return aln ? ASC_B(3, true) : ASC_B(3, false);
#undef ASC_B
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
const void* pick_bwd(int dirs, bool aln, bool dyc) {
#define ASC_B(D, A, Y) reinterpret_cast<const void*>(&k_scan_bwd<IO, D, A, Y>)
  if (dyc) {  // single-branch calls only
    if (dirs == 1) return aln ? ASC_B(1, true, true) : ASC_B(1, false, true);
    return aln ? ASC_B(2, true, true) : ASC_B(2, false, true);
  }
  if (dirs == 1) return aln ? ASC_B(1, true, false) : ASC_B(1, false, false);
  if (dirs == 2) return aln ? ASC_B(2, true, false) : ASC_B(2, false, false);
  return aln ? ASC_B(3, true, false) : ASC_B(3, false, false);
#undef ASC_B
}

// Item order of the workgroup walks: channel blocks up to a mean segment
// of 32K elements, channel-major beyond (measured, fp32, see item_range).
int wg_chan_blocks(int64_t S, int64_t T) {
  return T / (S > 0 ? S : 1) <= 32768 ? 1 : 0;
}

int run_fwd(const void* const* g, const void* const* x, void* const* h,
            void* a, int nbranch, int dirs, const void* cu, int cu_dtype,
            int64_t S, int64_t C, int64_t T, int dtype, void* ws,
            int64_t ws_bytes, void* stream) {
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
    p.br[b].pend = p.geo.phase + C * T;
  }
  const bool wa = a != nullptr;
  const int64_t items = p.geo.items * nbranch;
  if (!wa && ws && reinterpret_cast<uintptr_t>(ws) % 32 == 0 &&
      lb_use(S, C, T, nbranch, v)) {
    LbFwdParams q{};
    q.geo = LbGeo{cu, cu_dtype == ASC_CU_I64, S, C, T, C * T, p.geo.phase,
                  0, 0, nbranch, g_spin_limit};
    q.geo.nvec = (q.geo.phase + q.geo.n + v - 1) / v;
    q.geo.ntiles = lb_ntiles(q.geo.n, q.geo.phase, v);
    const int64_t need = q.geo.ntiles * nbranch * static_cast<int64_t>(sizeof(LbSlot));
    if (ws_bytes >= need) {
      for (int b = 0; b < nbranch; ++b) q.br[b] = p.br[b];
      q.slots = static_cast<LbSlot*>(ws);
      if ((st = fill_zero(ws, need, stream))) return st;
      const void* fn = nullptr;
      switch (dtype) {
        case ASC_F32: fn = pick_fwd_lb<IoF32>(dirs, aln); break;
        case ASC_F16: fn = pick_fwd_lb<IoF16>(dirs, aln); break;
        default: fn = pick_fwd_lb<IoBF16>(dirs, aln); break;
      }
      return launch(fn, q.geo.ntiles * nbranch, kLbWaves, q, stream);
    }
  }
  const int nw = wa ? 0 : pick_walk(S, C, T, nbranch, v, false);
  if (nw) {
    const bool blk = wg_chan_blocks(S, T) != 0;
    const void* fn = nullptr;
    switch (dtype) {
      case ASC_F32: fn = pick_fwd_wg<IoF32>(nw, dirs, aln, blk); break;
      case ASC_F16: fn = pick_fwd_wg<IoF16>(nw, dirs, aln, blk); break;
      default: fn = pick_fwd_wg<IoBF16>(nw, dirs, aln, blk); break;
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

// dyc: dy[0] holds one gradient value per row (element stride dy_rs between
// rows) that is constant along time; single-branch calls only.
int run_bwd(const void* const* dy, const void* const* g, const void* const* h,
            void* const* dx, void* const* dg, int nbranch, int dirs,
            const void* cu, int cu_dtype, int64_t S, int64_t C, int64_t T,
            int dtype, void* ws, int64_t ws_bytes, void* stream,
            bool dyc = false, int64_t dy_rs = 0) {
  int st = check_geometry(cu, cu_dtype, S, C, T, dtype);
  if (st) return st;
  for (int b = 0; b < nbranch; ++b)
    if (!dy[b] || !g[b] || !h[b] || !dx[b] || !dg[b]) return ASC_E_NULL;
  const int es = elem_size(dtype);
  const int v = 16 / es;
  if (dyc && (nbranch != 1 || dy_rs < 0)) return ASC_E_ARG;
  const void* all[10];
  int n = 0;
  for (int b = 0; b < nbranch; ++b) {
    all[n++] = g[b];
    all[n++] = h[b];
    all[n++] = dx[b];
    all[n++] = dg[b];
  }
  if ((st = check_ptrs(all, n, es))) return st;
  if ((st = check_ptrs(dy, nbranch, es))) return st;
  if (S == 0 || C == 0 || T == 0) return ASC_OK;
  // the per-row gradient of dyc is read by scalar loads: its alignment does
  // not enter the phase
  if (!dyc)
    for (int b = 0; b < nbranch; ++b) all[n++] = dy[b];
  const int ph = common_phase(all, n, es, v);
  const bool aln = ph >= 0;
  BwdParams p{};
  p.geo = Geometry{cu, cu_dtype == ASC_CU_I64, S, C, T, S * C, nbranch,
                   aln ? ph : 0};
  const int64_t shift = static_cast<int64_t>(p.geo.phase) * es;
  for (int b = 0; b < nbranch; ++b) {
    p.br[b].dy = static_cast<const char*>(dy[b]) - (dyc ? 0 : shift);
    p.br[b].g = static_cast<const char*>(g[b]) - shift;
    p.br[b].h = static_cast<const char*>(h[b]) - shift;
    p.br[b].dx = static_cast<char*>(dx[b]) - shift;
    p.br[b].dg = static_cast<char*>(dg[b]) - shift;
    p.br[b].pend = p.geo.phase + C * T;
  }
  p.dy_rs = dy_rs;
  const int64_t items = p.geo.items * nbranch;
  if (!dyc && ws && reinterpret_cast<uintptr_t>(ws) % 32 == 0 &&
      lb_use(S, C, T, nbranch, v)) {
    LbBwdParams q{};
    q.geo = LbGeo{cu, cu_dtype == ASC_CU_I64, S, C, T, C * T, p.geo.phase,
                  0, 0, nbranch, g_spin_limit};
    q.geo.nvec = (q.geo.phase + q.geo.n + v - 1) / v;
    q.geo.ntiles = lb_ntiles(q.geo.n, q.geo.phase, v);
    const int64_t need = q.geo.ntiles * nbranch * static_cast<int64_t>(sizeof(LbSlot));
    if (ws_bytes >= need) {
      for (int b = 0; b < nbranch; ++b) q.br[b] = p.br[b];
      q.slots = static_cast<LbSlot*>(ws);
      if ((st = fill_zero(ws, need, stream))) return st;
      const void* fn = nullptr;
      switch (dtype) {
        case ASC_F32: fn = pick_bwd_lb<IoF32>(dirs, aln); break;
        case ASC_F16: fn = pick_bwd_lb<IoF16>(dirs, aln); break;
        default: fn = pick_bwd_lb<IoBF16>(dirs, aln); break;
      }
      return launch(fn, q.geo.ntiles * nbranch, kLbWaves, q, stream);
    }
  }
  const int nw = pick_walk(S, C, T, nbranch, v, true);
  if (nw) {
    const bool blk = wg_chan_blocks(S, T) != 0;
    const void* fn = nullptr;
    switch (dtype) {
      case ASC_F32: fn = pick_bwd_wg<IoF32>(nw, dirs, aln, dyc, blk); break;
      case ASC_F16: fn = pick_bwd_wg<IoF16>(nw, dirs, aln, dyc, blk); break;
      default: fn = pick_bwd_wg<IoBF16>(nw, dirs, aln, dyc, blk); break;
    }
    return launch(fn, items, nw, p, stream);
  }
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = pick_bwd<IoF32>(dirs, aln, dyc); break;
    case ASC_F16: fn = pick_bwd<IoF16>(dirs, aln, dyc); break;
    default: fn = pick_bwd<IoBF16>(dirs, aln, dyc); break;
  }
  return launch(fn, (items + kWPB - 1) / kWPB, kWPB, p, stream);
}

}  // namespace

extern "C" {

int asc_abi_version(void) { return ASC_ABI_VERSION; }

int64_t asc_scan_workspace_bytes(int64_t num_seq, int64_t num_channels,
                                 int64_t seq_stride, int dtype, int nbranch) {
  const int es = elem_size(dtype);
  if (es == 0 || num_seq < 0 || num_channels < 0 || seq_stride < 0 ||
      nbranch < 1 || nbranch > 2)
    return ASC_E_ARG;
  if (num_channels > 0 && seq_stride > (INT64_MAX / 64) / num_channels)
    return ASC_E_SIZE;
  if (!lb_use(num_seq, num_channels, seq_stride, nbranch, 16 / es)) return 0;
  return lb_bytes(num_channels * seq_stride, 16 / es, nbranch);
}

unsigned asc_set_lookback_spin_limit(unsigned polls) {
  const unsigned prev = g_spin_limit;
  g_spin_limit = polls;
  return prev;
}

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
                 int dtype, int reverse, void* workspace,
                 int64_t workspace_bytes, void* stream) {
  const void* g[1] = {gates};
  const void* x[1] = {tokens};
  void* h[1] = {h_out};
  return run_fwd(g, x, h, gate_prod_out, 1, reverse ? 2 : 1, cu_seqlens,
                 cu_dtype, num_seq, num_channels, seq_stride, dtype, workspace,
                 workspace_bytes, stream);
}

int asc_scan_bwd(const void* grad, const void* gates, const void* states,
                 void* d_tokens, void* d_gates, const void* cu_seqlens,
                 int cu_dtype, int64_t num_seq, int64_t num_channels,
                 int64_t seq_stride, int dtype, int causal, void* workspace,
                 int64_t workspace_bytes, void* stream) {
  const void* dy[1] = {grad};
  const void* g[1] = {gates};
  const void* h[1] = {states};
  void* dx[1] = {d_tokens};
  void* dg[1] = {d_gates};
  return run_bwd(dy, g, h, dx, dg, 1, causal ? 1 : 2, cu_seqlens, cu_dtype,
                 num_seq, num_channels, seq_stride, dtype, workspace,
                 workspace_bytes, stream);
}

int asc_scan_bwd_rowgrad(const void* grad_rows, int64_t grad_row_stride,
                         const void* gates, const void* states, void* d_tokens,
                         void* d_gates, const void* cu_seqlens, int cu_dtype,
                         int64_t num_seq, int64_t num_channels,
                         int64_t seq_stride, int dtype, int causal,
                         void* stream) {
  const void* dy[1] = {grad_rows};
  const void* g[1] = {gates};
  const void* h[1] = {states};
  void* dx[1] = {d_tokens};
  void* dg[1] = {d_gates};
  if (grad_row_stride < 0) return ASC_E_ARG;
  return run_bwd(dy, g, h, dx, dg, 1, causal ? 1 : 2, cu_seqlens, cu_dtype,
                 num_seq, num_channels, seq_stride, dtype, nullptr, 0, stream,
                 true, grad_row_stride);
}

int asc_scan_bidi_fwd(const void* gates_fwd, const void* tokens_fwd,
                      const void* gates_bwd, const void* tokens_bwd,
                      void* h_fwd, void* h_bwd, const void* cu_seqlens,
                      int cu_dtype, int64_t num_seq, int64_t num_channels,
                      int64_t seq_stride, int dtype, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  const void* g[2] = {gates_fwd, gates_bwd};
  const void* x[2] = {tokens_fwd, tokens_bwd};
  void* h[2] = {h_fwd, h_bwd};
  return run_fwd(g, x, h, nullptr, 2, 3, cu_seqlens, cu_dtype, num_seq,
                 num_channels, seq_stride, dtype, workspace, workspace_bytes,
                 stream);
}

int asc_scan_bidi_bwd(const void* grad_fwd, const void* grad_bwd,
                      const void* gates_fwd, const void* gates_bwd,
                      const void* states_fwd, const void* states_bwd,
                      void* d_tokens_fwd, void* d_gates_fwd,
                      void* d_tokens_bwd, void* d_gates_bwd,
                      const void* cu_seqlens, int cu_dtype, int64_t num_seq,
                      int64_t num_channels, int64_t seq_stride, int dtype,
                      void* workspace, int64_t workspace_bytes, void* stream) {
  const void* dy[2] = {grad_fwd, grad_bwd};
  const void* g[2] = {gates_fwd, gates_bwd};
  const void* h[2] = {states_fwd, states_bwd};
  void* dx[2] = {d_tokens_fwd, d_tokens_bwd};
  void* dg[2] = {d_gates_fwd, d_gates_bwd};
  return run_bwd(dy, g, h, dx, dg, 2, 3, cu_seqlens, cu_dtype, num_seq,
                 num_channels, seq_stride, dtype, workspace, workspace_bytes,
                 stream);
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
  const int v = 16 / es;
  const int ph = common_phase(all, 2, es, v);
  if (ph >= 0 && ASC_SHIFT_VEC) {
    ShiftVecParams q{};
    q.data = p.data - static_cast<int64_t>(ph) * es;
    q.out = p.out - static_cast<int64_t>(ph) * es;
    q.cu = p.cu;
    q.cu64 = p.cu64;
    q.S = p.S;
    q.C = p.C;
    q.L = p.L;
    q.phase = ph;
    const int64_t chv = static_cast<int64_t>(kShiftVecPerLane) * kWave;
    // vectors a row touches, at most (L + 2 v - 2) / v; one chunk per chv
    q.chunks = ((seq_len + 2 * v - 2) / v + chv - 1) / chv;
    q.pad = p.pad;
    q.backward = p.backward;
    q.wrap = p.wrap;
    const void* fn = nullptr;
    switch (dtype) {
      case ASC_F32: fn = reinterpret_cast<const void*>(&k_shift_pad_vec<IoF32>); break;
      case ASC_F16: fn = reinterpret_cast<const void*>(&k_shift_pad_vec<IoF16>); break;
      default: fn = reinterpret_cast<const void*>(&k_shift_pad_vec<IoBF16>); break;
    }
    return launch(fn, (q.C * q.chunks + 3) / 4, 4, q, stream);
  }
  const void* fn = nullptr;
  switch (dtype) {
    case ASC_F32: fn = reinterpret_cast<const void*>(&k_shift_pad<IoF32>); break;
    case ASC_F16: fn = reinterpret_cast<const void*>(&k_shift_pad<IoF16>); break;
    default: fn = reinterpret_cast<const void*>(&k_shift_pad<IoBF16>); break;
  }
  return launch(fn, (p.C * p.chunks + 3) / 4, 4, p, stream);
}

}  // extern "C"
