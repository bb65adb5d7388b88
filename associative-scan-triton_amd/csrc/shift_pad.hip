// shift_pad: segment-aware shift of a [C, L] tensor by one position, with
// a pad value at segment edges, following the reference _shift_pad.py:18-55
// (shift_pad, row ends wrap around) and :63-165 (_shift_pad_kernel and
// shift_pad_compiled, row ends clamped).

#include "asc_common.h"

namespace asc {
namespace {

// ---------------------------------------------------------------------------
// shift_pad: elementwise, for any strides of data and out (element (c, t) at
// c * row_stride + t * col_stride), lanes interleaved (element t0 + 64*j +
// lane) so that with unit column strides every load/store instruction is
// one contiguous run.  Values move as raw bits.  Boundaries of the wave's
// range are found by a binary search over cu_seqlens.
// ---------------------------------------------------------------------------
constexpr int kShiftPerLane = 8;
constexpr int64_t kShiftChunk = kWave * kShiftPerLane;

struct ShiftParams {
  const char* data;
  char* out;
  const void* cu;
  int cu64;
  int64_t S, C, L;
  int64_t ds0, ds1;  // data strides (elements): row, column
  int64_t os0, os1;  // out strides
  int64_t chunks;    // chunks per row
  float pad;         // rounded to the element type on the device
  int backward;
  int wrap;
};

template <class IO>
__device__ inline uint32_t raw_ld(const char* p) {
  if (IO::ES == 4) return *reinterpret_cast<const uint32_t*>(p);
  return *reinterpret_cast<const unsigned short*>(p);
}
template <class IO>
__device__ inline void raw_st(char* p, uint32_t v) {
  if (IO::ES == 4)
    *reinterpret_cast<uint32_t*>(p) = v;
  else
    *reinterpret_cast<unsigned short*>(p) = static_cast<unsigned short>(v);
}

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
    const char* row = p.data + c * p.ds0 * IO::ES;
    char* orow = p.out + c * p.os0 * IO::ES;
    const uint32_t padb = IO::bits(p.pad);
    uint32_t v[kShiftPerLane];
#pragma unroll
    for (int j = 0; j < kShiftPerLane; ++j) {
      const int64_t t = t0 + j * kWave + lane;
      v[j] = 0u;
      if (t < t1) {
        int64_t src = p.backward ? t - 1 : t + 1;
        if (src < 0) src = p.wrap ? p.L - 1 : 0;
        if (src >= p.L) src = p.wrap ? 0 : p.L - 1;
        v[j] = raw_ld<IO>(row + src * p.ds1 * IO::ES);
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
          if (jj == j) v[jj] = padb;
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
      if (t < t1) raw_st<IO>(orow + t * p.os1 * IO::ES, v[j]);
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
    ShiftParams bp{};
    bp.cu = p.cu;
    bp.cu64 = p.cu64;
    bp.S = p.S;
    bp.C = p.C;
    bp.L = p.L;
    bp.backward = p.backward;
    bp.wrap = p.wrap;
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

}  // namespace
}  // namespace asc

using namespace asc;

#pragma GCC visibility push(default)
extern "C" {

int asc_shift_pad_strided(const void* data, int64_t data_row_stride,
                          int64_t data_col_stride, void* out,
                          int64_t out_row_stride, int64_t out_col_stride,
                          const void* cu_seqlens, int cu_dtype, int64_t num_seq,
                          int64_t num_channels, int64_t seq_len, int dtype,
                          double pad_value, int backward, int wrap,
                          void* stream) {
  int st = check_geometry(cu_seqlens, cu_dtype, num_seq, num_channels,
                          seq_len, dtype);
  if (st) return st;
  if (!data || !out) return ASC_E_NULL;
  const int es = elem_size(dtype);
  const void* all[2] = {data, out};
  if ((st = check_ptrs(all, 2, es))) return st;
  const int64_t C = num_channels, L = seq_len;
  if (data_row_stride < 0 || data_col_stride < 0 || out_row_stride < 0 ||
      out_col_stride < 0)
    return ASC_E_ARG;
  if (C == 0 || L == 0) return ASC_OK;
  // out must not overlap itself (each element its own address) ...
  const int64_t a0 = C > 1 ? out_row_stride : 0, a1 = L > 1 ? out_col_stride : 0;
  const int64_t lo = a0 < a1 ? a0 : a1, hi = a0 < a1 ? a1 : a0;
  const int64_t lo_n = a0 < a1 ? C : L;
  if ((C > 1 && out_row_stride == 0) || (L > 1 && out_col_stride == 0) ||
      (lo > 0 && hi < lo * lo_n))
    return ASC_E_ARG;
  // ... nor the data (the shift is not done in place)
  const int64_t dspan = ((C - 1) * data_row_stride + (L - 1) * data_col_stride + 1) * es;
  const int64_t ospan = ((C - 1) * out_row_stride + (L - 1) * out_col_stride + 1) * es;
  if (overlap(data, dspan, out, ospan) != kDisjoint) return ASC_E_ARG;
  ShiftParams p{};
  p.data = static_cast<const char*>(data);
  p.out = static_cast<char*>(out);
  p.cu = cu_seqlens;
  p.cu64 = cu_dtype == ASC_CU_I64;
  p.S = num_seq;
  p.C = C;
  p.L = L;
  p.ds0 = data_row_stride;
  p.ds1 = data_col_stride;
  p.os0 = out_row_stride;
  p.os1 = out_col_stride;
  p.chunks = (L + kShiftChunk - 1) / kShiftChunk;
  p.pad = static_cast<float>(pad_value);
  p.backward = backward ? 1 : 0;
  p.wrap = wrap ? 1 : 0;
  const int v = 16 / es;
  const bool dense = data_col_stride == 1 && out_col_stride == 1 &&
                     (C == 1 || (data_row_stride == L && out_row_stride == L));
  const int ph = dense ? common_phase(all, 2, es, v) : -1;
  if (ph >= 0) {
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

int asc_shift_pad(const void* data, void* out, const void* cu_seqlens,
                  int cu_dtype, int64_t num_seq, int64_t num_channels,
                  int64_t seq_len, int dtype, double pad_value, int backward,
                  int wrap, void* stream) {
  return asc_shift_pad_strided(data, seq_len, 1, out, seq_len, 1, cu_seqlens,
                               cu_dtype, num_seq, num_channels, seq_len, dtype,
                               pad_value, backward, wrap, stream);
}

}  // extern "C"
#pragma GCC visibility pop
