// libassocscan C entry points: argument checks, the phase frame of the
// tensor pointers, and the choice of walk for each call.  The kernels of each
// walk live in their own translation unit (scan_item.hip: one wave per
// (segment, channel) item; scan_wg.hip: one workgroup per item;
// scan_lookback.hip: decoupled look-back over tiles of the flat array;
// shift_pad.hip: the shift entry point), over the shared sub-tile scan of
// asc_common.h.

#include <atomic>
#include <mutex>

#include "asc_common.h"

// Workspace of the allocation-free forward (asc_scan_fwd_noalloc, below):
// each GPU the library runs on holds its own copy until the process ends.
// On the host this name is a host-side stand-in, not a device address; the
// device address of the current GPU's copy comes from hipGetSymbolAddress.
constexpr int64_t kScratchBytes = int64_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Short segments: two items per wave (1) or one (0).
#ifndef ASC_GROUP_WALK
#define ASC_GROUP_WALK 1
#endif

// Few-item problems: the tree walk (1) or the look-back walk (0).
#ifndef ASC_USE_TREE
#define ASC_USE_TREE 1
#endif

namespace asc {
namespace {

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
  // h may replace the tokens of its branch and the gate product the gates
  // (the reference's INPLACE and TESTING writes, _kernels.py:74-81).  Such
  // a call runs the per-item walks, which read every element before they
  // overwrite it: the bounded-wait fallbacks of the chained and look-back
  // walks re-read inputs of earlier chunks, which an in-place call may
  // already have overwritten.
  const int64_t nbytes = C * T * es;
  OutArg outs[3];
  InArg ins[4];
  int no = 0, ni = 0;
  for (int b = 0; b < nbranch; ++b) {
    outs[no++] = OutArg{h[b], nbytes, x[b]};
    ins[ni++] = InArg{g[b], nbytes};
    ins[ni++] = InArg{x[b], nbytes};
  }
  if (a) outs[no++] = OutArg{a, nbytes, g[0]};
  bool inplace = false;
  if ((st = check_alias(outs, no, ins, ni, &inplace))) return st;
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
  // the look-back walks do not write the gate product and are not used in
  // place; they need the caller's workspace (else the per-item walks run)
  const bool walks_ok = !wa && !inplace;
  bool chained = false;
  if (walks_ok && lb_use(S, C, T, nbranch, v)) {
    // few items: the tree walk (deterministic), or the look-back walk for
    // tensors of different phases
    if (ASC_USE_TREE &&
        tree_fwd(p, dtype, dirs, aln, ws, ws_bytes, stream, st, &p.skip)) {
      // the workspace-free walk below runs only if a tree wait failed
      if (st) return st;
      p.skip_if_clear = 1;
    } else if (lb_fwd(p, dtype, dirs, aln, ws, ws_bytes, stream, st)) {
      return st;
    }
  } else if (walks_ok) {
    // long segments: the per-item walk below takes the unaligned ones, the
    // chained walk after it the chunk-aligned ones
    chained = chain_plan(p.geo, aln, dtype, ws, ws_bytes, false);
  }
  // (the chained walk's partner is the one-wave walk: its launch costs a
  // few microseconds when it has nothing to do, the workgroup walks' 20-30)
  const int nw = wa || chained ? 0 : pick_walk(S, C, T, nbranch, v, false);
  if (nw)
    st = wg_fwd(p, nw, dtype, dirs, aln, stream);
  else if (ASC_GROUP_WALK && aln && !wa && !chained && group_walk_use(p.geo, v))
    st = group_walk_fwd(p, dtype, dirs, stream);
  else
    st = item_fwd(p, dtype, dirs, aln, wa, stream);
  if (st || !chained) return st;
  return chain_fwd(p, dtype, dirs, stream);
}

// dyc: dy[b] holds one gradient value per row (element stride dy_rs[b]
// between rows) that is constant along time.
int run_bwd(const void* const* dy, const void* const* g, const void* const* h,
            void* const* dx, void* const* dg, int nbranch, int dirs,
            const void* cu, int cu_dtype, int64_t S, int64_t C, int64_t T,
            int dtype, void* ws, int64_t ws_bytes, void* stream,
            bool dyc = false, const int64_t* dy_rs = nullptr) {
  int st = check_geometry(cu, cu_dtype, S, C, T, dtype);
  if (st) return st;
  for (int b = 0; b < nbranch; ++b)
    if (!dy[b] || !g[b] || !h[b] || !dx[b] || !dg[b]) return ASC_E_NULL;
  const int es = elem_size(dtype);
  const int v = 16 / es;
  if (dyc)
    for (int b = 0; b < nbranch; ++b)
      if (dy_rs[b] < 0) return ASC_E_ARG;
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
  // d_tokens may replace the (dense) gradient of its branch, and such a call
  // runs the per-item walks (see run_fwd); any other overlap of an output
  // with an input or another output is an error: the shifted gates and
  // states are read across sub-tile and wave edges after neighbouring
  // elements' outputs may have been stored.
  const int64_t nbytes = C * T * es;
  OutArg outs[4];
  InArg ins[6];
  int no = 0, ni = 0;
  for (int b = 0; b < nbranch; ++b) {
    const int64_t dyb = dyc ? ((C > 0 ? C - 1 : 0) * dy_rs[b] + 1) * es : nbytes;
    outs[no++] = OutArg{dx[b], nbytes, dyc ? nullptr : dy[b]};
    outs[no++] = OutArg{dg[b], nbytes, nullptr};
    ins[ni++] = InArg{dy[b], dyb};
    ins[ni++] = InArg{g[b], nbytes};
    ins[ni++] = InArg{h[b], nbytes};
  }
  bool inplace = false;
  if ((st = check_alias(outs, no, ins, ni, &inplace))) return st;
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
  for (int b = 0; b < nbranch; ++b) p.dy_rs[b] = dyc ? dy_rs[b] : 0;
  // few items: the tree walk, else (tensors of different phases) the
  // look-back walk, which takes dense gradients only
  const bool few = !inplace && lb_use(S, C, T, nbranch, v);
  bool chained = false;
  if (few && ASC_USE_TREE &&
      tree_bwd(p, dtype, dirs, aln, dyc, ws, ws_bytes, stream, st, &p.skip)) {
    // the workspace-free walk below runs only if a tree wait failed
    if (st) return st;
    p.skip_if_clear = 1;
  } else if (few && !dyc) {
    if (lb_bwd(p, dtype, dirs, aln, ws, ws_bytes, stream, st)) return st;
  } else if (!inplace) {
    // as in run_fwd: the per-item walk, then the chained walk
    chained = chain_plan(p.geo, aln, dtype, ws, ws_bytes, true);
  }
  const int nw = chained ? 0 : pick_walk(S, C, T, nbranch, v, true);
  if (nw)
    st = wg_bwd(p, nw, dtype, dirs, aln, dyc, stream);
  else if (ASC_GROUP_WALK && aln && !chained && group_walk_use(p.geo, v))
    st = group_walk_bwd(p, dtype, dirs, dyc, stream);
  else
    st = item_bwd(p, dtype, dirs, aln, dyc, stream);
  if (st || !chained) return st;
  return chain_bwd(p, dtype, dyc, dirs, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free forward (asc_scan_fwd_noalloc): the device address of the
// current GPU's copy of `scratch` is looked up once per device and only
// that address is ever handed to kernels.
// ---------------------------------------------------------------------------
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's `scratch`; `stream` (if not NULL)
// must belong to the current device.
int scratch_ptr(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return ASC_E_ARG;
  if (stream) {
    int sdev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) return static_cast<int>(e);
    if (sdev != dev) return ASC_E_ARG;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return static_cast<int>(e);
      if (!p) return ASC_E_NULL;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return ASC_OK;
}

}  // namespace
}  // namespace asc

using namespace asc;

#pragma GCC visibility push(default)

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
  if (lb_use(num_seq, num_channels, seq_stride, nbranch, 16 / es)) {
    const int64_t lb = lb_bytes(num_channels * seq_stride, 16 / es, nbranch);
    const int64_t tr = tree_bytes(num_channels * seq_stride, 16 / es, nbranch);
    return lb > tr ? lb : tr;
  }
  return chain_bytes(num_seq, num_channels, seq_stride, 16 / es, nbranch);
}

int asc_scan_workspace_walk(int64_t num_seq, int64_t num_channels,
                            int64_t seq_stride, int dtype, int nbranch) {
  const int64_t nb = asc_scan_workspace_bytes(num_seq, num_channels,
                                              seq_stride, dtype, nbranch);
  if (nb <= 0) return static_cast<int>(nb);
  return lb_use(num_seq, num_channels, seq_stride, nbranch,
                16 / elem_size(dtype))
             ? ASC_WALK_LOOKBACK
             : ASC_WALK_CHAINED;
}

unsigned asc_set_lookback_spin_limit(unsigned polls) {
  return lb_set_spin_limit(polls);
}

const char* asc_strerror(int status) {
  switch (status) {
    case ASC_OK: return "success";
    case ASC_E_NULL: return "a required pointer argument is NULL";
    case ASC_E_DTYPE: return "unsupported dtype or cu_seqlens dtype";
    case ASC_E_SIZE: return "invalid (negative or overflowing) size argument";
    case ASC_E_ALIGN: return "pointer not aligned to its element size";
    case ASC_E_ARG: return "invalid argument";
    case ASC_E_SCRATCH:
      return "the geometry needs more workspace than the static scratch "
             "buffer of asc_scan_fwd_noalloc holds (8 MiB)";
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

int asc_scan_fwd_noalloc(const void* gates, const void* tokens, void* h_out,
                         void* gate_prod_out, const void* cu_seqlens,
                         int cu_dtype, int64_t num_seq, int64_t num_channels,
                         int64_t seq_stride, int dtype, int reverse,
                         void* stream) {
  // the workspace asc_scan_fwd would be given for this geometry, taken from
  // the static array (the walks clear what must start at zero themselves)
  const int64_t need = asc_scan_workspace_bytes(num_seq, num_channels,
                                                seq_stride, dtype, 1);
  if (need < 0) return static_cast<int>(need);
  if (need > kScratchBytes) return ASC_E_SCRATCH;
  void* ws = nullptr;
  if (need > 0) {
    const int st = scratch_ptr(stream, &ws);
    if (st) return st;
  }
  const void* g[1] = {gates};
  const void* x[1] = {tokens};
  void* h[1] = {h_out};
  return run_fwd(g, x, h, gate_prod_out, 1, reverse ? 2 : 1, cu_seqlens,
                 cu_dtype, num_seq, num_channels, seq_stride, dtype, ws,
                 need > 0 ? kScratchBytes : 0, stream);
}

int64_t asc_scan_checkpoint_elems(int64_t num_channels, int64_t seq_stride,
                                  int dtype) {
  const int es = elem_size(dtype);
  if (es == 0 || num_channels < 0 || seq_stride < 0) return ASC_E_ARG;
  const int64_t kr = rc_chunks_per_row(seq_stride, 16 / es);
  if (kr > 0 && num_channels > INT64_MAX / kr) return ASC_E_SIZE;
  return num_channels * kr;
}

int asc_scan_checkpoints(const void* states, float* checkpoints,
                         const void* cu_seqlens, int cu_dtype, int64_t num_seq,
                         int64_t num_channels, int64_t seq_stride, int dtype,
                         int reverse, void* stream) {
  int st = check_geometry(cu_seqlens, cu_dtype, num_seq, num_channels,
                          seq_stride, dtype);
  if (st) return st;
  if (!states || !checkpoints) return ASC_E_NULL;
  const int es = elem_size(dtype);
  const void* p[1] = {states};
  if ((st = check_ptrs(p, 1, es))) return st;
  if (reinterpret_cast<uintptr_t>(checkpoints) % 4) return ASC_E_ALIGN;
  const int64_t nck = asc_scan_checkpoint_elems(num_channels, seq_stride, dtype);
  if (overlap(states, num_channels * seq_stride * es, checkpoints, nck * 4))
    return ASC_E_ARG;
  if (nck == 0) return ASC_OK;
  return rc_checkpoints(states, checkpoints, cu_seqlens, cu_dtype, num_seq,
                        num_channels, seq_stride, dtype, reverse, stream);
}

int asc_scan_bwd_recompute(const void* grad, int64_t grad_row_stride,
                           const void* gates, const void* tokens,
                           const float* checkpoints, void* d_tokens,
                           void* d_gates, const void* cu_seqlens, int cu_dtype,
                           int64_t num_seq, int64_t num_channels,
                           int64_t seq_stride, int dtype, int causal,
                           void* workspace, int64_t workspace_bytes,
                           void* stream) {
  const int64_t S = num_seq, C = num_channels, T = seq_stride;
  int st = check_geometry(cu_seqlens, cu_dtype, S, C, T, dtype);
  if (st) return st;
  if (!grad || !gates || !tokens || !checkpoints || !d_tokens || !d_gates)
    return ASC_E_NULL;
  const int es = elem_size(dtype);
  const int v = 16 / es;
  const bool dense = grad_row_stride < 0;
  const void* all[5] = {gates, tokens, d_tokens, d_gates, grad};
  if ((st = check_ptrs(all, 5, es))) return st;
  if (reinterpret_cast<uintptr_t>(checkpoints) % 4) return ASC_E_ALIGN;
  // the recompute walks address whole 16-byte vectors of every row
  for (int i = 0; i < (dense ? 5 : 4); ++i)
    if (reinterpret_cast<uintptr_t>(all[i]) % 16) return ASC_E_ALIGN;
  if (T % v) return ASC_E_ALIGN;
  const int64_t nbytes = C * T * es;
  const int64_t gbytes =
      dense ? nbytes : ((C > 0 ? C - 1 : 0) * grad_row_stride + 1) * es;
  const int64_t nck = asc_scan_checkpoint_elems(C, T, dtype);
  if (nck < 0) return static_cast<int>(nck);
  const OutArg outs[2] = {{d_tokens, nbytes, dense ? grad : nullptr},
                          {d_gates, nbytes, nullptr}};
  const InArg ins[4] = {{grad, gbytes}, {gates, nbytes}, {tokens, nbytes},
                        {checkpoints, nck * 4}};
  bool inplace = false;
  if ((st = check_alias(outs, 2, ins, 4, &inplace))) return st;
  if (S == 0 || C == 0 || T == 0) return ASC_OK;
  RcArgs a{};
  a.dy = grad;
  a.dy_rs = grad_row_stride;
  a.g = gates;
  a.x = tokens;
  a.ckpt = checkpoints;
  a.dx = d_tokens;
  a.dg = d_gates;
  a.cu = cu_seqlens;
  a.cu64 = cu_dtype == ASC_CU_I64;
  a.S = S;
  a.C = C;
  a.T = T;
  a.dtype = dtype;
  a.causal = causal != 0;
  a.inplace = inplace;
  a.ws = workspace;
  a.ws_bytes = workspace_bytes;
  return rc_bwd(a, stream);
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
                         void* workspace, int64_t workspace_bytes,
                         void* stream) {
  const void* dy[1] = {grad_rows};
  const void* g[1] = {gates};
  const void* h[1] = {states};
  void* dx[1] = {d_tokens};
  void* dg[1] = {d_gates};
  const int64_t rs[1] = {grad_row_stride};
  if (grad_row_stride < 0) return ASC_E_ARG;
  return run_bwd(dy, g, h, dx, dg, 1, causal ? 1 : 2, cu_seqlens, cu_dtype,
                 num_seq, num_channels, seq_stride, dtype, workspace,
                 workspace_bytes, stream, true, rs);
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

int asc_scan_bidi_bwd_rowgrad(
    const void* grad_fwd_rows, int64_t grad_fwd_row_stride,
    const void* grad_bwd_rows, int64_t grad_bwd_row_stride,
    const void* gates_fwd, const void* gates_bwd, const void* states_fwd,
    const void* states_bwd, void* d_tokens_fwd, void* d_gates_fwd,
    void* d_tokens_bwd, void* d_gates_bwd, const void* cu_seqlens,
    int cu_dtype, int64_t num_seq, int64_t num_channels, int64_t seq_stride,
    int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  const void* dy[2] = {grad_fwd_rows, grad_bwd_rows};
  const void* g[2] = {gates_fwd, gates_bwd};
  const void* h[2] = {states_fwd, states_bwd};
  void* dx[2] = {d_tokens_fwd, d_tokens_bwd};
  void* dg[2] = {d_gates_fwd, d_gates_bwd};
  const int64_t rs[2] = {grad_fwd_row_stride, grad_bwd_row_stride};
  if (grad_fwd_row_stride < 0 || grad_bwd_row_stride < 0) return ASC_E_ARG;
  return run_bwd(dy, g, h, dx, dg, 2, 3, cu_seqlens, cu_dtype, num_seq,
                 num_channels, seq_stride, dtype, workspace, workspace_bytes,
                 stream, true, rs);
}

}  // extern "C"
#pragma GCC visibility pop
