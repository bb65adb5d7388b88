/*
 * scan_oracle.c - CPU restatement of the reference scan, for TESTS ONLY.
 *
 * This file is test infrastructure: only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it, and only as the checker
 * or the timed CPU baseline.  No product code path calls it.
 *
 * Everything is sequential in the time direction and, in the fp64 entry
 * points, computed in double precision with one rounding per operation:
 * compile with -ffp-contract=off so that `g*h + x` is a multiply followed by
 * an add, exactly as the reference's torch fp64 gold label
 * (tests/test_scan_dtypes.py:26-38, bench/bench_accuracy.py:40-49).
 *
 * Layout: C rows of T elements, row c at offset c*T; segment s of every row
 * covers [cu[s], cu[s+1]).
 */
#include <stdint.h>
#include <stdlib.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int cu_ok(const int64_t* cu, int64_t S, int64_t T) {
  if (cu[0] < 0) return 0;
  for (int64_t s = 0; s < S; ++s)
    if (cu[s + 1] < cu[s]) return 0;
  return cu[S] <= T;
}

/*
 * Forward scan per segment.
 *   reverse = 0: h[start] = x[start]; h[t] = g[t]*h[t-1] + x[t]
 *                (test_scan_dtypes.py:34-37 applied to each segment)
 *   reverse = 1: h[end-1] = x[end-1]; h[t] = g[t]*h[t+1] + x[t]
 *                (_kernels.py:55-58: reversed indices within the segment)
 * a (nullable): running gate product, a[t] = prod of g from the segment
 *   head (in scan order) through t (_kernels.py:72-76 with TESTING).
 * Returns 0, or -1 for a malformed cu.
 */
int oracle_scan_fwd(const double* g, const double* x, double* h, double* a,
                    const int64_t* cu, int64_t S, int64_t C, int64_t T,
                    int reverse) {
  if (!cu_ok(cu, S, T)) return -1;
  for (int64_t c = 0; c < C; ++c) {
    const int64_t row = c * T;
    for (int64_t s = 0; s < S; ++s) {
      const int64_t b = cu[s], e = cu[s + 1];
      if (e <= b) continue;
      if (!reverse) {
        h[row + b] = x[row + b];
        if (a) a[row + b] = g[row + b];
        for (int64_t t = b + 1; t < e; ++t) {
          h[row + t] = g[row + t] * h[row + t - 1] + x[row + t];
          if (a) a[row + t] = a[row + t - 1] * g[row + t];
        }
      } else {
        h[row + e - 1] = x[row + e - 1];
        if (a) a[row + e - 1] = g[row + e - 1];
        for (int64_t t = e - 2; t >= b; --t) {
          h[row + t] = g[row + t] * h[row + t + 1] + x[row + t];
          if (a) a[row + t] = a[row + t + 1] * g[row + t];
        }
      }
    }
  }
  return 0;
}

/*
 * Backward of the forward scan (reverse-recurrence form of the hand
 * derivation in tests/test_scan_kernels.py:873-897, and the shifted
 * gate / state pads of _kernels.py:232-247 and :266-283).
 *   causal = 1:  dx[e-1] = dy[e-1]; dx[t] = dy[t] + dx[t+1]*g[t+1]
 *                dg[t] = hprev * dx[t], hprev = h[t-1], and 0 at t = start
 *   causal = 0:  dx[b] = dy[b];     dx[t] = dy[t] + dx[t-1]*g[t-1]
 *                dg[t] = hnext * dx[t], hnext = h[t+1], and 0 at t = end-1
 */
int oracle_scan_bwd(const double* dy, const double* g, const double* h,
                    double* dx, double* dg, const int64_t* cu, int64_t S,
                    int64_t C, int64_t T, int causal) {
  if (!cu_ok(cu, S, T)) return -1;
  for (int64_t c = 0; c < C; ++c) {
    const int64_t row = c * T;
    for (int64_t s = 0; s < S; ++s) {
      const int64_t b = cu[s], e = cu[s + 1];
      if (e <= b) continue;
      if (causal) {
        for (int64_t t = e - 1; t >= b; --t) {
          const double d = (t == e - 1)
              ? dy[row + t]
              : dy[row + t] + dx[row + t + 1] * g[row + t + 1];
          dx[row + t] = d;
          const double hp = (t == b) ? 0.0 : h[row + t - 1];
          dg[row + t] = hp * d;
        }
      } else {
        for (int64_t t = b; t < e; ++t) {
          const double d = (t == b)
              ? dy[row + t]
              : dy[row + t] + dx[row + t - 1] * g[row + t - 1];
          dx[row + t] = d;
          const double hn = (t == e - 1) ? 0.0 : h[row + t + 1];
          dg[row + t] = hn * d;
        }
      }
    }
  }
  return 0;
}

/*
 * shift_pad (_shift_pad.py:41-53 eager roll + mask, and :63-118 compiled
 * clamp + mask).  backward = 1: out[p] = data[p-1], pad at cu[s] (s < S);
 * backward = 0: out[p] = data[p+1], pad at cu[s]-1 (s >= 1).  Boundary
 * positions follow torch indexing: a negative position counts from the end
 * (mask[-1] is the last element).  wrap = 1: neighbour index wraps
 * (torch.roll); wrap = 0: neighbour index is clamped into [0, L).
 */
int oracle_shift_pad(const double* data, double* out, const int64_t* cu,
                     int64_t S, int64_t C, int64_t L, double pad,
                     int backward, int wrap) {
  unsigned char* mask = (unsigned char*)calloc((size_t)(L > 0 ? L : 1), 1);
  if (!mask) return -2;
  for (int64_t s = 0; s < S; ++s) {
    int64_t p = backward ? cu[s] : cu[s + 1] - 1;
    if (p < 0) p += L;
    if (p < 0 || p >= L) {
      free(mask);
      return -1;
    }
    mask[p] = 1;
  }
  for (int64_t c = 0; c < C; ++c) {
    const double* r = data + c * L;
    double* o = out + c * L;
    for (int64_t p = 0; p < L; ++p) {
      int64_t q = backward ? p - 1 : p + 1;
      if (q < 0) q = wrap ? L - 1 : 0;
      if (q >= L) q = wrap ? 0 : L - 1;
      o[p] = mask[p] ? pad : r[q];
    }
  }
  free(mask);
  return 0;
}

/*
 * CPU baseline: the same forward + backward on fp32 storage with fp64
 * accumulation (the reference's CPU path is the fp64 sequential scan),
 * parallelised over (segment, channel) items with `threads` OpenMP threads.
 */
int oracle_fwd_bwd_f32io(const float* g, const float* x, const float* dy,
                         float* h, float* dx, float* dg, const int64_t* cu,
                         int64_t S, int64_t C, int64_t T, int threads) {
  if (!cu_ok(cu, S, T)) return -1;
  const int64_t items = S * C;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
  for (int64_t w = 0; w < items; ++w) {
    const int64_t c = w % C, s = w / C;
    const int64_t row = c * T, b = cu[s], e = cu[s + 1];
    if (e <= b) continue;
    double hh = x[row + b];
    h[row + b] = (float)hh;
    for (int64_t t = b + 1; t < e; ++t) {
      hh = (double)g[row + t] * hh + (double)x[row + t];
      h[row + t] = (float)hh;
    }
    double d = 0.0, gn = 0.0;
    for (int64_t t = e - 1; t >= b; --t) {
      d = (t == e - 1) ? (double)dy[row + t] : (double)dy[row + t] + d * gn;
      gn = g[row + t];
      dx[row + t] = (float)d;
      const double hp = (t == b) ? 0.0 : (double)h[row + t - 1];
      dg[row + t] = (float)(hp * d);
    }
  }
  (void)threads;
  return 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
