// libassocscan (gfx950): the first-order linear recurrence
// h[t] = g[t]*h[t-1] + x[t] over packed segments.  This header holds what
// every translation unit shares: storage types, wave-level scan
// primitives, the sub-tile scan, item geometry and the host-side argument
// checks; each walk's kernels live in a unit of their own.
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
//     (global_load_dwordx4).  Vectors are aligned in memory and sub-tiles
//     start on 128-byte lines; a segment start or end that falls inside a
//     sub-tile is handled by per-element masking on the first and last
//     sub-tile only (the look-back walk, whose tiles
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

#ifndef ASC_COMMON_H
#define ASC_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "assocscan.h"

#ifndef ASC_WAVES_PER_BLOCK
#define ASC_WAVES_PER_BLOCK 1
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


namespace asc {


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

// Two elements rounded into one word (lo in bits 0-15) by one packed
// conversion (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32, round-to-nearest-even
// like the scalar ones above).
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ inline uint32_t f2h2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}
__device__ inline uint32_t f2b2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

template <float (*CVT)(uint32_t), uint32_t (*RND)(float),
          uint32_t (*RND2)(float, float)>
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
    for (int i = 0; i < 4; ++i) w[i] = RND2(f[2 * i], f[2 * i + 1]);
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
using IoF16 = IoHalf<h2f, f2h, f2h2>;
using IoBF16 = IoHalf<b2f, f2b, f2b2>;

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

template <int CTRL, int ROWMASK>
__device__ inline void mul_step(float& p) {
  p = p * dpp<CTRL, ROWMASK>(1.0f, p);
}

// The lane scans below put the DPP source on the arithmetic itself
// (v_fmac_f32_dpp x, x, a: x = x[src] * a + x; v_mul_f32_dpp a, a, a:
// a = a[src] * a).  Without bound_ctrl a lane whose source is out of its row,
// or whose row is masked off, is not written, which is the identity; the
// builtin form above spends a v_mov of the identity and a v_mov_b32_dpp per
// operand and step on the same thing.  A VALU result read as a DPP source
// needs two wait states: each block starts and ends with s_nop 1 for the
// code around it, and within a block the other operation of the step and an
// s_nop 0 separate a write from its DPP read.
#ifndef ASC_DPP_ASM
#define ASC_DPP_ASM 1
#endif
#define ASC_DPP_SHR(n) "row_shr:" #n " row_mask:0xf bank_mask:0xf"
#define ASC_DPP_BC15 "row_bcast:15 row_mask:0xa bank_mask:0xf"
#define ASC_DPP_BC31 "row_bcast:31 row_mask:0xc bank_mask:0xf"
#define ASC_AFFINE(c) \
  "v_fmac_f32_dpp %1, %1, %0 " c "\n\tv_mul_f32_dpp %0, %0, %0 " c "\n\t"
#define ASC_MUL(c) "v_mul_f32_dpp %0, %0, %0 " c "\n\ts_nop 1\n\t"
#define ASC_AFFINE_ROWS                                              \
  "s_nop 1\n\t" ASC_AFFINE(ASC_DPP_SHR(1)) "s_nop 0\n\t"            \
      ASC_AFFINE(ASC_DPP_SHR(2)) "s_nop 0\n\t" ASC_AFFINE(ASC_DPP_SHR(4)) \
          "s_nop 0\n\t" ASC_AFFINE(ASC_DPP_SHR(8)) "s_nop 0\n\t"        \
              ASC_AFFINE(ASC_DPP_BC15)

// Inclusive scan of affine maps over the 64 lanes (lane 0 first).
__device__ inline void wave_scan_affine(float& a, float& x) {
  if (ASC_DPP_ASM) {
    asm(ASC_AFFINE_ROWS "s_nop 0\n\t" ASC_AFFINE(ASC_DPP_BC31) "s_nop 1"
        : "+v"(a), "+v"(x));
    return;
  }
  affine_step<kRowShr1, 0xf>(a, x);
  affine_step<kRowShr2, 0xf>(a, x);
  affine_step<kRowShr4, 0xf>(a, x);
  affine_step<kRowShr8, 0xf>(a, x);
  affine_step<kRowBcast15, 0xa>(a, x);
  affine_step<kRowBcast31, 0xc>(a, x);
}

// Inclusive scan of affine maps within each 32-lane half (rows 0-1 and
// 2-3): the scan above without its last step.
__device__ inline void half_scan_affine(float& a, float& x) {
  if (ASC_DPP_ASM) {
    asm(ASC_AFFINE_ROWS "s_nop 1" : "+v"(a), "+v"(x));
    return;
  }
  affine_step<kRowShr1, 0xf>(a, x);
  affine_step<kRowShr2, 0xf>(a, x);
  affine_step<kRowShr4, 0xf>(a, x);
  affine_step<kRowShr8, 0xf>(a, x);
  affine_step<kRowBcast15, 0xa>(a, x);
}

// Inclusive product scan over the 64 lanes.
__device__ inline void wave_scan_mul(float& p) {
  if (ASC_DPP_ASM) {
    asm("s_nop 1\n\t" ASC_MUL(ASC_DPP_SHR(1)) ASC_MUL(ASC_DPP_SHR(2))
            ASC_MUL(ASC_DPP_SHR(4)) ASC_MUL(ASC_DPP_SHR(8))
                ASC_MUL(ASC_DPP_BC15) ASC_MUL(ASC_DPP_BC31)
        : "+v"(p));
    return;
  }
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
constexpr int64_t kLineVecs = 8;  // 16-byte vectors per 128-byte line

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
    // The first sub-tile in scan order is widened to start on a multiple
    // of 8 vectors from the origin (a 128-byte line when the tensor base is
    // 128-byte aligned, as torch's allocations are; the extra lanes lie
    // outside the item and are masked like any edge element), so every
    // later sub-tile covers exactly 8 lines.  Sub-tiles that start mid-line make each load and store touch
    // one line more and split lines between consecutive sub-tiles
    // (measured, cfg3-like ragged bf16 segments: +6% forward, +10%
    // backward; aligned segments unchanged).
    if (REV) v1 |= kLineVecs - 1;
    else v0 &= ~(kLineVecs - 1);
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

// One vector of N tensors (same index), masked as load_vec<IO, true, true,
// true>.  load_vec masks each vector as soon as it is read, so the wave
// waits for one tensor's load before it issues the next one's; here every
// load is issued first and the masks follow.  Vectors that need element
// loads (the tensor's own first and last vectors) take load_vec, for the
// whole wave when any of its lanes has one.
template <class IO, int N>
__device__ inline void load_vecs(const char* const (&origin)[N], int64_t vi,
                                 bool lane_ok, int64_t P0, int64_t P1,
                                 const float (&ident)[N],
                                 float (&f)[N][IO::V], int64_t pend) {
  constexpr int V = IO::V;
  const int64_t pv = vi * V;
  const bool touch = lane_ok && pv + V > P0 && pv < P1;
  const bool wide = vi >= 1 && pv + V <= pend;
  if (__builtin_amdgcn_ballot_w64(touch && !wide) != 0) {
#pragma unroll
    for (int n = 0; n < N; ++n)
      load_vec<IO, true, true, true>(origin[n], vi, lane_ok, P0, P1, ident[n],
                                     f[n], pend);
    return;
  }
  uint4 q[N];
  if (touch) {
#pragma unroll
    for (int n = 0; n < N; ++n) q[n] = ld16(origin[n] + vi * 16);
  }
#pragma unroll
  for (int n = 0; n < N; ++n) {
    float v[V];
    IO::unpack(q[n], v);
#pragma unroll
    for (int j = 0; j < V; ++j)
      f[n][j] = touch && pv + j >= P0 && pv + j < P1 ? v[j] : ident[n];
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
__device__ inline void fwd_lanes(const float* g, const float* x, int64_t pv,
                                 int64_t phead, float& A, float& X) {
  constexpr int V = IO::V;
  A = 1.0f;
  X = 0.0f;
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
}

// The lane's exclusive prefix and the sub-tile total from the inclusive
// lane scan (A, X).
__device__ inline SubScan sub_scan(float A, float X) {
  SubScan r;
  r.ta = readlane(A, kWave - 1);
  r.tx = readlane(X, kWave - 1);
  r.ea = dpp<kWaveShr1, 0xf>(1.0f, A);
  r.ex = dpp<kWaveShr1, 0xf>(0.0f, X);
  return r;
}

template <class IO, bool REV, bool MASKED>
__device__ inline SubScan fwd_local(const float* g, const float* x, int64_t pv,
                                    int64_t phead) {
  float A, X;
  fwd_lanes<IO, REV, MASKED>(g, x, pv, phead, A, X);
  return sub_scan(A, X);
}

// With the carry into the sub-tile already known: y = the lane's inclusive
// map applied to the carry; lane l starts from y of lane l-1 (lane 0 from
// the carry) and the carry out is y of lane 63.  The same fmas as applying
// the exclusive prefix and the total to the carry (lane 0 takes the carry
// itself, where fma(1, carry, 0) turns a -0 carry into +0), in three VALU
// operations and one readlane instead of six and two.
__device__ inline float carried_start(float A, float X, float& carry) {
  const float y = fmaf(A, carry, X);
  const float start = dpp<kWaveShr1, 0xf>(carry, y);
  carry = readlane(y, kWave - 1);
  return start;
}

// Second phase: the lane re-walks its elements from its start value hh
// (its prefix applied to the carry into the sub-tile); h in memory order.
template <class IO, bool REV, bool MASKED>
__device__ inline void fwd_walk(const float* g, const float* x, int64_t pv,
                                int64_t phead, float hh, float* hout) {
  constexpr int V = IO::V;
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

template <class IO, bool REV, bool MASKED>
__device__ inline void fwd_apply(const float* g, const float* x, int64_t pv,
                                 int64_t phead, const SubScan& s, float carry,
                                 float* hout) {
  fwd_walk<IO, REV, MASKED>(g, x, pv, phead, fmaf(s.ea, carry, s.ex), hout);
}

// One sub-tile with a carry in a register; writes h (and the gate product
// when WA) in memory order.
template <class IO, bool REV, bool MASKED, bool WA>
__device__ inline void fwd_subtile(const float* g, const float* x, int64_t pv,
                                   int64_t phead, float& carry, float& carry_a,
                                   float* hout, float* aout) {
  constexpr int V = IO::V;
  float A, X;
  fwd_lanes<IO, REV, MASKED>(g, x, pv, phead, A, X);
  fwd_walk<IO, REV, MASKED>(g, x, pv, phead, carried_start(A, X, carry), hout);
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
__device__ inline void bwd_lanes(const float* g, const float* dy, int64_t pv,
                                 int64_t phead, float carry_g, float& gprev,
                                 float& A, float& X) {
  constexpr int V = IO::V;
  constexpr int jl = mem_idx<V, RB>(V - 1);  // last element in B order
  gprev = dpp<kWaveShr1, 0xf>(carry_g, g[jl]);
  A = 1.0f;
  X = 0.0f;
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
}

template <class IO, bool RB, bool MASKED>
__device__ inline SubScan bwd_local(const float* g, const float* dy, int64_t pv,
                                    int64_t phead, float carry_g,
                                    float& gprev) {
  float A, X;
  bwd_lanes<IO, RB, MASKED>(g, dy, pv, phead, carry_g, gprev, A, X);
  return sub_scan(A, X);
}

// Second phase: dx by re-walking from the prefix, dg = shifted state * dx.
// hnext_in is the state of the element just after the sub-tile in B order
// (it shifts into lane 63); ptail is the segment's last element in B order,
// whose shifted state is the pad 0.
template <class IO, bool RB, bool MASKED>
__device__ inline void bwd_walk(const float* g, const float* dy,
                                const float* h, int64_t pv, int64_t phead,
                                int64_t ptail, float gprev, float hnext_in,
                                float d, float* dxo, float* dgo) {
  constexpr int V = IO::V;
  constexpr int jf = mem_idx<V, RB>(0);  // first element in B order
  const float hnx = dpp<kWaveShl1, 0xf>(hnext_in, h[jf]);
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
__device__ inline void bwd_apply(const float* g, const float* dy,
                                 const float* h, int64_t pv, int64_t phead,
                                 int64_t ptail, float gprev, float hnext_in,
                                 const SubScan& s, float carry, float* dxo,
                                 float* dgo) {
  bwd_walk<IO, RB, MASKED>(g, dy, h, pv, phead, ptail, gprev, hnext_in,
                           fmaf(s.ea, carry, s.ex), dxo, dgo);
}

template <class IO, bool RB, bool MASKED>
__device__ inline void bwd_subtile(const float* g, const float* dy,
                                   const float* h, int64_t pv, int64_t phead,
                                   int64_t ptail, float& carry,
                                   float& carry_g, float hnext_in,
                                   float* dxo, float* dgo) {
  constexpr int V = IO::V;
  float gprev, A, X;
  bwd_lanes<IO, RB, MASKED>(g, dy, pv, phead, carry_g, gprev, A, X);
  bwd_walk<IO, RB, MASKED>(g, dy, h, pv, phead, ptail, gprev, hnext_in,
                           carried_start(A, X, carry), dxo, dgo);
  carry_g = readlane(g[mem_idx<V, RB>(V - 1)], kWave - 1);
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
  // Set when the chained walk (scan_chain.hip) runs right after this
  // per-item walk (one wave per item) in the same call: the per-item walk
  // clears the chained walk's slots (chain_words 64-bit words), its first
  // wave writes *chain_flag (chain_survey), and it leaves every item
  // whose segment has both edges on the chunk grid (chain_ch elements, a
  // power of two) to the chained walk.  chain_ch = 0: no chained walk.
  int64_t chain_ch;
  unsigned long long* chain_slots;
  int64_t chain_words;
  uint32_t* chain_flag;
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

// Both edges of segment s.  The two loads are issued before either value
// is used: two cu_at calls each wait for their load (the value is moved to
// a scalar register at once), which put two memory round trips in front of
// every item's first data load.
__device__ inline void cu_edges(const Geometry& geo, int64_t s, int64_t& t0,
                                int64_t& t1) {
  int64_t a, b;
  if (geo.cu64) {
    const int64_t* p = reinterpret_cast<const int64_t*>(geo.cu) + s;
    a = p[0];
    b = p[1];
  } else {
    const int32_t* p = reinterpret_cast<const int32_t*>(geo.cu) + s;
    a = p[0];
    b = p[1];
  }
  t0 = uniform(a);
  t1 = uniform(b);
}

// Segments the chained walk takes when it runs after a per-item walk (see
// Geometry::chain_ch): non-empty, inside [0, T], both edges on the chunk
// grid of ch elements (a power of two; raw cu_seqlens values;
// chain_common.h applies the same test).
__device__ inline bool chain_takes(int64_t ch, int64_t T, int64_t t0,
                                   int64_t t1) {
  return ch > 0 && t0 >= 0 && t0 < t1 && t1 <= T && ((t0 | t1) & (ch - 1)) == 0;
}

// Survey of cu_seqlens for the chained walk: which non-empty segments
// (after the clamping of item_range) it takes (chain_takes).  kChainAll:
// every one (a per-item walk launched before it then has nothing to do,
// and the chained walk may read a chunk before it looks up its segment);
// kChainNone: none (the chained grid has nothing to do); kChainSome: some,
// or more than smax segments (not surveyed: both walks test each item or
// chunk on its own).  Each lane looks at 4 segments per batch of 256, its
// loads in flight together.  Returns the same value in every lane.
enum : uint32_t { kChainNone = 0, kChainAll = 1, kChainSome = 2 };
constexpr int64_t kChainBatch = 4 * kWave;
__device__ inline uint32_t chain_survey(const void* cu, int cu64, int64_t S,
                                        int64_t T, int64_t ch, int lane,
                                        int64_t smax) {
  if (ch == 0 || S > smax) return kChainSome;
  bool all = true, any = false;
  for (int64_t base = 0; base < S; base += kChainBatch) {
    int64_t lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t s = base + k * kWave + lane;
      lo[k] = hi[k] = 0;
      if (s < S) {
        lo[k] = cu64 ? reinterpret_cast<const int64_t*>(cu)[s]
                     : reinterpret_cast<const int32_t*>(cu)[s];
        hi[k] = cu64 ? reinterpret_cast<const int64_t*>(cu)[s + 1]
                     : reinterpret_cast<const int32_t*>(cu)[s + 1];
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t t0 = lo[k] < 0 ? 0 : (lo[k] > T ? T : lo[k]);
      const int64_t t1 = hi[k] < t0 ? t0 : (hi[k] > T ? T : hi[k]);
      const bool taken = chain_takes(ch, T, lo[k], hi[k]);
      if (t1 > t0 && !taken) all = false;
      if (taken) any = true;
    }
  }
  if (__builtin_amdgcn_ballot_w64(!all) == 0) return kChainAll;
  return __builtin_amdgcn_ballot_w64(any) != 0 ? kChainSome : kChainNone;
}

// Prologue of a per-item walk launched before the chained walk (see
// Geometry::chain_ch), for wave gw of the grid's nw: clears its share of
// the chained walk's slots; the waves of the first workgroup survey up to
// kChainSurveyMax segments (a loop of batches) and its first wave writes
// the flag the chained walk reads, the others survey one batch.  Returns
// true when the walk has no item to take (the same value in every wave of
// a workgroup, so that they all return together).
constexpr int64_t kChainSurveyMax = 16 * kChainBatch - 1;
__device__ inline bool chain_prologue(const Geometry& geo, int64_t gw,
                                      int64_t nw, int lane) {
  for (int64_t i = gw * kWave + lane; i < geo.chain_words; i += nw * kWave)
    geo.chain_slots[i] = 0ull;
  const bool first = blockIdx.x == 0;
  const uint32_t sv =
      chain_survey(geo.cu, geo.cu64, geo.S, geo.T, geo.chain_ch, lane,
                   first ? kChainSurveyMax : kChainBatch - 1);
  if (gw == 0 && lane == 0) *geo.chain_flag = sv;
  return sv == kChainAll;
}

// Decodes item w; returns false for an empty segment and, in a walk that
// can run before the chained walk (CHAIN), for an item the chained walk
// takes.
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
// Segment s and channel c of item r of a branch (the orders above).
__device__ inline void item_seg_chan(const Geometry& geo, int64_t r,
                                     bool blocks, int64_t& s, int64_t& c) {
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
}

template <bool CHAIN = false>
__device__ inline bool item_range(const Geometry& geo, int64_t w, int& br,
                                  int64_t& P0, int64_t& P1, int64_t& row,
                                  bool blocks) {
  br = w >= geo.items ? 1 : 0;
  const int64_t r = w - br * geo.items;
  int64_t s, c;
  item_seg_chan(geo, r, blocks, s, c);
  int64_t t0, t1;
  cu_edges(geo, s, t0, t1);
  if (CHAIN && chain_takes(geo.chain_ch, geo.T, t0, t1)) return false;
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

// skip: nullptr, or a flag in device memory that makes every workgroup
// return at once when it is set or, with skip_if_clear, when it is clear
// (the tree walk ran and no wait of it failed; see scan_tree.hip).
struct FwdParams {
  Geometry geo;
  FwdPtrs br[2];
  const uint32_t* skip;
  int skip_if_clear;
};

struct BwdParams {
  Geometry geo;
  BwdPtrs br[2];
  int64_t dy_rs[2];  // DYC: element stride between rows of each gradient
  const uint32_t* skip;
  int skip_if_clear;
};

template <class Params>
__device__ inline bool skipped(const Params& p) {
  return p.skip != nullptr && ((*p.skip != 0u) != (p.skip_if_clear != 0));
}

// Grid of a per-item walk that is usually skipped (behind the tree walk)
// or left to the chained walk launched after it: at most 131072 waves (512
// per CU), the grid-stride loops take the rest, so that the skip costs a
// bounded number of workgroups, not one per item.  A tighter cap hands each workgroup several ragged items when
// the walk does run (varlen, 32 segments of 1000-15000 fp32 elements x 1024
// rows, 8-wave walk: 32768 waves 807 / 1201 us fwd / bwd, 131072 waves
// 726 / 1048, uncapped 721 / 1011); a looser one costs more when skipped
// (bidirectional 8 x 16K x 1536: uncapped 683 us bwd against 673-675).
constexpr int64_t kSkippableWaves = 131072;
template <class Params>
inline int64_t walk_grid(const Params& p, int64_t blocks, int waves_per_block) {
  const int64_t cap = kSkippableWaves / waves_per_block;
  return (p.skip != nullptr || p.geo.chain_ch > 0) && blocks > cap ? cap
                                                                   : blocks;
}

// DYC: the gradient of row c of branch br is the one value
// dy[c * dy_rs[br]] (unshifted dy).
template <class IO, bool DYC>
__device__ inline float dyc_value(const BwdParams& p, int br, int64_t row) {
  if (!DYC) return 0.0f;
  return IO::load1(p.br[br].dy + row * p.dy_rs[br] * IO::ES);
}


// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
inline int elem_size(int dtype) {
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

inline int check_geometry(const void* cu, int cu_dtype, int64_t S, int64_t C,
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
inline int common_phase(const void* const* ptrs, int n, int es, int v) {
  int ph = -1;
  for (int i = 0; i < n; ++i) {
    if (!ptrs[i]) continue;
    const int q = static_cast<int>((reinterpret_cast<uintptr_t>(ptrs[i]) / es) % v);
    if (ph < 0) ph = q;
    else if (ph != q) return -1;
  }
  return ph < 0 ? 0 : ph;
}

inline int check_ptrs(const void* const* ptrs, int n, int es) {
  for (int i = 0; i < n; ++i)
    if (ptrs[i] && reinterpret_cast<uintptr_t>(ptrs[i]) % es) return ASC_E_ALIGN;
  return ASC_OK;
}

// How the byte ranges [p, p + np) and [q, q + nq) meet: 0 = disjoint (or
// either is empty or NULL), 1 = the same range, 2 = a partial overlap.
enum { kDisjoint = 0, kSame = 1, kPartial = 2 };
inline int overlap(const void* p, int64_t np, const void* q, int64_t nq) {
  if (!p || !q || np <= 0 || nq <= 0) return kDisjoint;
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uintptr_t b = reinterpret_cast<uintptr_t>(q);
  if (a + static_cast<uintptr_t>(np) <= b || b + static_cast<uintptr_t>(nq) <= a)
    return kDisjoint;
  return (a == b && np == nq) ? kSame : kPartial;
}

// An output tensor and the one input it may replace in place (nullptr:
// none), for the aliasing rule of the scan entry points.
struct OutArg {
  const void* p;
  int64_t bytes;
  const void* may_equal;
};
struct InArg {
  const void* p;
  int64_t bytes;
};

// Aliasing rule: an output may coincide exactly with the one input it is
// allowed to replace; any other overlap of an output with an input or with
// another output is ASC_E_ARG.  *inplace tells whether some output does
// replace its input.
inline int check_alias(const OutArg* outs, int nout, const InArg* ins, int nin,
                       bool* inplace) {
  *inplace = false;
  for (int i = 0; i < nout; ++i) {
    for (int j = 0; j < nin; ++j) {
      const int ov = overlap(outs[i].p, outs[i].bytes, ins[j].p, ins[j].bytes);
      if (ov == kDisjoint) continue;
      if (ov == kSame && outs[i].may_equal == ins[j].p) {
        *inplace = true;
        continue;
      }
      return ASC_E_ARG;
    }
    for (int j = i + 1; j < nout; ++j)
      if (overlap(outs[i].p, outs[i].bytes, outs[j].p, outs[j].bytes) != kDisjoint)
        return ASC_E_ARG;
  }
  return ASC_OK;
}

template <class Params>
int launch(const void* fn, int64_t blocks, int waves_per_block, Params p,
           void* stream) {
  if (blocks > kMaxGrid) blocks = kMaxGrid;
  void* args[] = {&p};
  const hipError_t e = hipLaunchKernel(fn, dim3(static_cast<unsigned>(blocks)),
                                       dim3(waves_per_block * kWave), args, 0,
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ASC_OK : static_cast<int>(e);
}


// Walk launchers, one translation unit each.  Each takes the per-call
// parameters (tensor origins in the phase frame), picks the kernel
// instantiation for the storage type and directions, and launches it on
// `stream`; the return value is an ASC_* status or a hipError_t.
// dirs: 1 = every item causal, 2 = every item reverse, 3 = branch 0 causal,
// branch 1 reverse (for the backward: the direction of the forward scan).

// scan_item.hip: one wave per item.
int item_fwd(FwdParams p, int dtype, int dirs, bool aln, bool wa, void* stream);
int item_bwd(BwdParams p, int dtype, int dirs, bool aln, bool dyc, void* stream);

// scan_wg.hip: one workgroup of nw (8 or 16) waves per item.
int wg_fwd(FwdParams p, int nw, int dtype, int dirs, bool aln, void* stream);
int wg_bwd(BwdParams p, int nw, int dtype, int dirs, bool aln, bool dyc,
           void* stream);

// scan_lookback.hip: decoupled look-back over tiles of the flat array.
// lb_use: whether the geometry runs this walk; lb_bytes: its workspace for n
// elements per branch.  lb_fwd / lb_bwd return false (nothing launched) when
// the workspace is missing, not 32-byte aligned or too small, else true with
// the launch status in `status`.
bool lb_use(int64_t S, int64_t C, int64_t T, int nbranch, int v);
int64_t lb_bytes(int64_t n, int v, int nbranch);
unsigned lb_set_spin_limit(unsigned polls);
unsigned lb_spin_limit();
// Zeroes `bytes` (a multiple of 8) of a workspace with a kernel on `stream`.
int fill_zero(void* ws, int64_t bytes, void* stream);
bool lb_fwd(const FwdParams& p, int dtype, int dirs, bool aln, void* ws,
            int64_t ws_bytes, void* stream, int& status);
bool lb_bwd(const BwdParams& p, int dtype, int dirs, bool aln, void* ws,
            int64_t ws_bytes, void* stream, int& status);

// scan_tree.hip: the tree walk over chunks of the flat array (few items;
// any cu_seqlens; tensors of one phase).  tree_bytes: its workspace for n
// elements per branch (0 when it cannot run); tree_fwd returns false
// (nothing launched) when it cannot run or the workspace is missing or too
// small, else true with the launch status in `status` and *fail pointing
// at a device flag that is set exactly when a bounded wait expired: the
// caller then launches a workspace-free walk that runs only when it is set.
int64_t tree_bytes(int64_t n, int v, int nbranch);
bool tree_fwd(const FwdParams& p, int dtype, int dirs, bool aln, void* ws,
              int64_t ws_bytes, void* stream, int& status,
              const uint32_t** fail);
// The backward, as tree_fwd (dyc: gradients constant along time, one value
// per row at p.dy_rs).
bool tree_bwd(const BwdParams& p, int dtype, int dirs, bool aln, bool dyc,
              void* ws, int64_t ws_bytes, void* stream, int& status,
              const uint32_t** fail);

// scan_group.hip: two or four items per wave (one per group of 32 or 16
// lanes) for short segments.  group_walk_use: the geometry's mean segment
// fits one step of a half (32 vectors); group_walk_fwd / group_walk_bwd
// launch it (16-byte aligned tensors, no gate product; arguments
// validated).
bool group_walk_use(const Geometry& geo, int v);
int group_walk_fwd(const FwdParams& p, int dtype, int dirs, void* stream);
int group_walk_bwd(const BwdParams& p, int dtype, int dirs, bool dyc,
                   void* stream);

// scan_chain.hip: chained chunks for segments aligned to the chunk size.
// chain_bytes: its workspace (0 when the geometry cannot use it).
// chain_plan returns false when the geometry or the workspace rules the
// walk out; otherwise it sets g.chain_* (see Geometry), and the caller
// launches its per-item walk with that geometry (it clears the slots and
// walks the unaligned segments), then chain_fwd / chain_bwd (the chunks of
// the aligned ones).
int64_t chain_bytes(int64_t S, int64_t C, int64_t T, int v, int nbranch);
bool chain_plan(Geometry& g, bool aln, int dtype, void* ws, int64_t ws_bytes,
                bool bwd);
int chain_fwd(const FwdParams& p, int dtype, int dirs, void* stream);
int chain_bwd(const BwdParams& p, int dtype, bool dyc, int dirs,
              void* stream);

// scan_recompute.hip: the backward that recomputes the forward states from
// its inputs and per-chunk checkpoints (asc_scan_bwd_recompute).
// rc_chunks_per_row: checkpoints per row; rc_checkpoints samples them from
// the forward's states; rc_bwd launches the recompute walks (arguments
// already validated; phase 0 and T a multiple of the vector width).
struct RcArgs {
  const void* dy;
  int64_t dy_rs;  // < 0: dy is a dense [C, T] tensor; else one value per row
  const void* g;
  const void* x;
  const float* ckpt;
  void* dx;
  void* dg;
  const void* cu;
  int cu64;
  int64_t S, C, T;
  int dtype;
  bool causal;
  bool inplace;  // dx is dy: only the per-item walk
  void* ws;
  int64_t ws_bytes;
};
int64_t rc_chunks_per_row(int64_t T, int v);
int rc_checkpoints(const void* h, float* ckpt, const void* cu, int cu_dtype,
                   int64_t S, int64_t C, int64_t T, int dtype, int reverse,
                   void* stream);
int rc_bwd(const RcArgs& a, void* stream);

}  // namespace asc

#endif  // ASC_COMMON_H
