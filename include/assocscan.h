/*
 * assocscan.h - C ABI of libassocscan, the MI355X (gfx950) chunked
 * linear-recurrence scan  h[t] = g[t] * h[t-1] + x[t].
 *
 * Layout shared by every entry point: a tensor is C rows ("channels") of
 * T = seq_stride elements each, time contiguous (element (c, t) lives at
 * index c * T + t).  Packed variable-length sequences ("segments") are given
 * by cu_seqlens[0..num_seq]: segment s of every row covers the time range
 * [cu_seqlens[s], cu_seqlens[s+1]).  cu_seqlens lives in device memory and is
 * read by the kernels; values are clamped to [0, T] on the device so that a
 * malformed cu_seqlens can never make a kernel touch memory outside the
 * tensors (it yields meaningless results instead).
 *
 * All pointers are device pointers.  Every call is asynchronous on `stream`
 * (a hipStream_t; NULL = the legacy default stream).  The library never
 * allocates, frees or synchronises.  Return value: 0 on success, a negative
 * ASC_E_* code for an invalid argument (nothing is launched), or a positive
 * hipError_t from the launch.  asc_strerror() turns any of them into text.
 *
 * Workspace: the scan entry points take an optional caller-owned device
 * buffer (32-byte aligned, asc_scan_workspace_bytes() bytes).  Problems
 * with few (segment, channel) items -- one long sequence, a handful of
 * channels -- want it: with it they run a single-pass walk over chunks of
 * 8192 fp32 / 16384 fp16-bf16 elements that keeps every CU busy, whose
 * carries go through a tree of 16-byte slots in the buffer (when every
 * tensor of the call has the same address modulo 16 bytes; otherwise a
 * decoupled look-back walk over tiles of 16384 elements, one slot per
 * tile).  Long chunk-aligned segments use it for a chained-chunk walk (see
 * asc_scan_workspace_walk).  The call clears what it uses on `stream`.
 * Every other problem, and any call given NULL or a buffer too small, runs
 * the workspace-free walks (one wave or one workgroup per item).  Results
 * agree to fp32 rounding; every walk but the look-back walk is bitwise
 * reproducible, the look-back walk's last bits can vary from run to run.
 * Two calls that run at the same time must not share a workspace.
 *
 * The reference is the Triton package associative-scan-triton 1.0.0; the
 * citations below name the reference function each entry point replaces.
 */
#ifndef ASSOCSCAN_H
#define ASSOCSCAN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of the scanned tensors (accumulation is always fp32). */
enum {
  ASC_F32 = 0,
  ASC_F16 = 1,
  ASC_BF16 = 2
};

/* Element types of cu_seqlens. */
enum {
  ASC_CU_I32 = 0,
  ASC_CU_I64 = 1
};

/* Negative status codes (positive codes are hipError_t values). */
enum {
  ASC_OK = 0,
  ASC_E_NULL = -1,       /* a required pointer is NULL                     */
  ASC_E_DTYPE = -2,      /* unknown dtype / cu dtype                      */
  ASC_E_SIZE = -3,       /* negative or overflowing sizes                 */
  ASC_E_ALIGN = -4,      /* a pointer is not aligned to its element size  */
  ASC_E_ARG = -5,        /* any other invalid argument                    */
  ASC_E_SCRATCH = -6     /* asc_scan_fwd_noalloc: geometry needs more
                            workspace than its static buffer holds        */
};

/* ABI version of this header; bumped on any signature change. */
#define ASC_ABI_VERSION 6
int asc_abi_version(void);

/*
 * Workspace bytes a scan entry point wants for this geometry, for
 * nbranch = 1 (asc_scan_fwd / asc_scan_bwd) or 2 (the bidirectional calls):
 * 0 when it runs a workspace-free walk anyway, a negative ASC_E_* code for
 * invalid arguments.  No reference counterpart: the reference's Triton
 * kernels carry their chunk carry in registers of one program per
 * (sequence, channel) and need no workspace.
 */
int64_t asc_scan_workspace_bytes(int64_t num_seq, int64_t num_channels,
                                 int64_t seq_stride, int dtype, int nbranch);

/*
 * Which walk a workspace of asc_scan_workspace_bytes() buys for this
 * geometry: 0 = none (the workspace-free walks run), ASC_WALK_LOOKBACK (few
 * items, any cu_seqlens: the tree walk, or the look-back walk for tensors at
 * different 16-byte phases), ASC_WALK_CHAINED (long segments; the chained
 * walk takes every segment whose edges are both multiples of the chunk size
 * -- 4096 fp32 / 8192 fp16-bf16 elements -- and the one-wave walk, launched
 * first in the same call, every other segment; cu_seqlens is read on the
 * device), or a negative ASC_E_* code.  The row-gradient entry points
 * below cannot use the look-back walk (they take the workspace-free walks
 * instead).  No reference counterpart.
 */
enum { ASC_WALK_LOOKBACK = 1, ASC_WALK_CHAINED = 2 };
int asc_scan_workspace_walk(int64_t num_seq, int64_t num_channels,
                            int64_t seq_stride, int dtype, int nbranch);

/*
 * Test hook, no reference counterpart: sets how many times a wave of the
 * look-back, chained or tree walk polls a preceding tile's slot before it
 * gives up waiting: a look-back wave then computes that tile's carry map
 * from the tile's inputs itself, a chained-walk chunk scans its segment's
 * prefix from the inputs itself, and a tree walk's call is redone by a
 * workspace-free walk (0 = give up at once; the default keeps the
 * fallback for pathological scheduling only).  Returns the previous value.
 * Process-wide (an atomic: safe to call from any host thread); affects
 * launches issued after the call.
 */
unsigned asc_set_lookback_spin_limit(unsigned polls);

/* Human-readable text for a status code returned by any entry point. */
const char* asc_strerror(int status);

/*
 * Forward scan over every (segment, channel) pair.
 *   reverse = 0:  h[t] = g[t]*h[t-1] + x[t],  h[start]  = x[start]
 *   reverse = 1:  h[t] = g[t]*h[t+1] + x[t],  h[end-1]  = x[end-1]
 * gate_prod_out (nullable): also writes the running gate product
 *   A[t] = prod g over [start..t] (reverse: over [t..end-1]).
 * In-place use is allowed: h_out may equal tokens and gate_prod_out may
 * equal gates (each element is read before it is overwritten).  Such a call,
 * and any call with gate_prod_out, runs the workspace-free walks (the
 * bounded-wait fallbacks of the tree, look-back and chained walks re-read
 * inputs of earlier tiles, which an in-place call may already have
 * overwritten).
 * Any other overlap between an output and an input, or between the two
 * outputs, returns ASC_E_ARG.
 *
 * Replaces: _dispatcher.py:12-70 forward_scan_full, which launches
 *   _kernels.py:19-81  forward_scan_chunked (one chunk) or
 *   _kernels.py:84-168 forward_scan_onepass_pipelined (many chunks);
 *   TESTING=True there corresponds to gate_prod_out = gates here and
 *   INPLACE=True to h_out = tokens.
 */
int asc_scan_fwd(const void* gates, const void* tokens, void* h_out,
                 void* gate_prod_out, const void* cu_seqlens, int cu_dtype,
                 int64_t num_seq, int64_t num_channels, int64_t seq_stride,
                 int dtype, int reverse, void* workspace,
                 int64_t workspace_bytes, void* stream);

/*
 * asc_scan_fwd without a workspace argument and without any allocation:
 * the tree, look-back and chained walks take their carry slots from a static
 * device array of 8 MiB that the library holds on each GPU it runs on
 * until the process ends (looked up once per device, with hipGetSymbolAddress,
 * on the first call).  Same arguments, results and aliasing rule as
 * asc_scan_fwd given a workspace of asc_scan_workspace_bytes(); a geometry
 * that would need more than 8 MiB of workspace returns ASC_E_SCRATCH
 * (nothing is launched).  `stream` must belong to the current device
 * (ASC_E_ARG otherwise).  Every call on one GPU shares that GPU's array:
 * calls that overlap in time on one GPU (other streams, other host threads)
 * race, so the caller serialises them.  The array keeps the last call's
 * contents; each call clears the slots it uses on `stream` with a kernel
 * (no memset, so the call can be captured in a HIP graph).
 *
 * No reference counterpart: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc), which with asc_scan_fwd could only pass NULL and lose the
 * tree, look-back and chained walks.
 */
int asc_scan_fwd_noalloc(const void* gates, const void* tokens, void* h_out,
                         void* gate_prod_out, const void* cu_seqlens,
                         int cu_dtype, int64_t num_seq, int64_t num_channels,
                         int64_t seq_stride, int dtype, int reverse,
                         void* stream);

/*
 * Fused backward of a forward scan (reads dy, g, h once; writes dx, dg).
 *   causal = 1 (backward of reverse=0):
 *     dx[t] = dy[t] + g[t+1]*dx[t+1],  dx[end-1] = dy[end-1]
 *     dg[t] = h[t-1]*dx[t],            h[start-1] := 0
 *   causal = 0 (backward of reverse=1):
 *     dx[t] = dy[t] + g[t-1]*dx[t-1],  dx[start] = dy[start]
 *     dg[t] = h[t+1]*dx[t],            h[end] := 0
 * d_tokens may equal grad (then the workspace-free walks run); any other
 * overlap between an output and an input or the other output returns
 * ASC_E_ARG (the shifted gates and states are read across the edges of
 * other waves' elements, which may already have been stored).  The same
 * rule holds for the bidirectional and row-gradient entry points below, per
 * branch.
 *
 * Replaces: _dispatcher.py:73-117 backward_scan_fused_full, which launches
 *   _kernels.py:171-287 backward_scan_fused or
 *   _kernels.py:290-374 backward_scan_fused_single_chunk.
 */
int asc_scan_bwd(const void* grad, const void* gates, const void* states,
                 void* d_tokens, void* d_gates, const void* cu_seqlens,
                 int cu_dtype, int64_t num_seq, int64_t num_channels,
                 int64_t seq_stride, int dtype, int causal, void* workspace,
                 int64_t workspace_bytes, void* stream);

/*
 * The same fused backward for a gradient that is constant along time in
 * every row: grad[c, t] = grad_rows[c * grad_row_stride] for all t
 * (grad_row_stride = 0: one value for the whole tensor).  This is the
 * gradient of out.sum() (or of any loss that reduces over time first), which
 * PyTorch hands over as a stride-0 expanded tensor.  The kernels read one
 * value per row instead of a [C, T] tensor: 4 of the 5 tensors' traffic, and
 * no materialised copy.  The workspace is used as by asc_scan_bwd, except
 * that the look-back walk for few items (tensors at different 16-byte
 * phases) does not take this form of the gradient (those calls run the
 * workspace-free walks).
 *
 * Replaces: scan_eager.py:58-63 (grad_output.contiguous() followed by
 *   backward_scan_fused_full) and scan_compiled.py:158-166 when the incoming
 *   gradient is such an expanded tensor.
 */
int asc_scan_bwd_rowgrad(const void* grad_rows, int64_t grad_row_stride,
                         const void* gates, const void* states, void* d_tokens,
                         void* d_gates, const void* cu_seqlens, int cu_dtype,
                         int64_t num_seq, int64_t num_channels,
                         int64_t seq_stride, int dtype, int causal,
                         void* workspace, int64_t workspace_bytes,
                         void* stream);

/*
 * Recompute mode (an opt-in of the autograd functions that keeps the
 * forward's inputs instead of its output for the backward).
 *
 * Checkpoints: one fp32 value per chunk of each row, chunks of 4096 (fp32)
 * or 8192 (fp16, bf16) elements along the row, the last one partial when
 * the row is not a whole number of chunks; asc_scan_checkpoint_elems(C, T,
 * dtype) = C * ceil(T / chunk) of them.  asc_scan_checkpoints samples them
 * from the states h of a finished forward scan (reverse = that scan's
 * direction): checkpoint (c, k) is the state adjacent to chunk k on the side
 * the scan comes from (causal: element k*chunk - 1 of row c; reverse: the
 * element just after the chunk) when it lies in the same segment as the
 * chunk's first element in scan order, else 0.
 *
 * asc_scan_bwd_recompute is asc_scan_bwd (causal = 1: the backward of
 * reverse = 0) reading the forward's tokens and the checkpoints instead of
 * the states: it recomputes the states chunk by chunk in registers, rounds
 * them to the storage type, and writes d_tokens and d_gates; HBM traffic is
 * that of asc_scan_bwd (dy, g, x read once; dx, dg written once).
 * grad_row_stride < 0: grad is a dense [C, T] tensor; >= 0: one value per
 * row, grad[c * grad_row_stride], as in asc_scan_bwd_rowgrad.  Every tensor
 * (and the dense gradient) must be 16-byte aligned and T a multiple of 4
 * (fp32) or 8 (fp16, bf16) elements, else ASC_E_ALIGN.  The workspace (as
 * asc_scan_workspace_bytes(..., nbranch = 1) says) buys the chained walk for
 * chunk-aligned segments; without it, for unaligned segments and for any
 * other geometry one workgroup per (segment, channel) item walks the chunks
 * (correct for every geometry, but slow for problems with few items, which
 * callers serve better by recomputing the states with asc_scan_fwd and
 * calling asc_scan_bwd).  Aliasing as asc_scan_bwd (d_tokens may equal a
 * dense grad; the checkpoints are an input).
 *
 * Replaces: scan_eager.py:42-47 and :50-64 (the states saved for the
 * backward, and backward_scan_fused_full on them) for callers that trade
 * the recompute for one [C, T] tensor of memory per call; the reference
 * lists it as future work (the recompute-states backward).
 */
int64_t asc_scan_checkpoint_elems(int64_t num_channels, int64_t seq_stride,
                                  int dtype);
int asc_scan_checkpoints(const void* states, float* checkpoints,
                         const void* cu_seqlens, int cu_dtype, int64_t num_seq,
                         int64_t num_channels, int64_t seq_stride, int dtype,
                         int reverse, void* stream);
int asc_scan_bwd_recompute(const void* grad, int64_t grad_row_stride,
                           const void* gates, const void* tokens,
                           const float* checkpoints, void* d_tokens,
                           void* d_gates, const void* cu_seqlens, int cu_dtype,
                           int64_t num_seq, int64_t num_channels,
                           int64_t seq_stride, int dtype, int causal,
                           void* workspace, int64_t workspace_bytes,
                           void* stream);

/*
 * Both branches of the bidirectional scan in ONE launch: a causal scan of
 * (gates_fwd, tokens_fwd) into h_fwd and a reverse scan of
 * (gates_bwd, tokens_bwd) into h_bwd.
 *
 * Replaces: scan_eager.py:122-131 (two forward_scan_full launches in
 *   ScanBidirectionalBranched.forward) and scan_compiled.py:229-238.
 */
int asc_scan_bidi_fwd(const void* gates_fwd, const void* tokens_fwd,
                      const void* gates_bwd, const void* tokens_bwd,
                      void* h_fwd, void* h_bwd, const void* cu_seqlens,
                      int cu_dtype, int64_t num_seq, int64_t num_channels,
                      int64_t seq_stride, int dtype, void* workspace,
                      int64_t workspace_bytes, void* stream);

/*
 * Backward of both bidirectional branches in ONE launch: causal backward of
 * the forward branch and anti-causal backward of the reverse branch.
 *
 * Replaces: scan_eager.py:160-169 (two backward_scan_fused_full launches in
 *   ScanBidirectionalBranched.backward) and scan_compiled.py:270-277.
 */
int asc_scan_bidi_bwd(const void* grad_fwd, const void* grad_bwd,
                      const void* gates_fwd, const void* gates_bwd,
                      const void* states_fwd, const void* states_bwd,
                      void* d_tokens_fwd, void* d_gates_fwd,
                      void* d_tokens_bwd, void* d_gates_bwd,
                      const void* cu_seqlens, int cu_dtype, int64_t num_seq,
                      int64_t num_channels, int64_t seq_stride, int dtype,
                      void* workspace, int64_t workspace_bytes, void* stream);

/*
 * asc_scan_bidi_bwd for gradients that are constant along time in every
 * row (as asc_scan_bwd_rowgrad): grad_fwd[c, t] =
 * grad_fwd_rows[c * grad_fwd_row_stride], and likewise for the reverse
 * branch.  A stride of 0 with a single zero value stands for a branch whose
 * output received no gradient.  The workspace is used as by
 * asc_scan_bidi_bwd.
 *
 * Replaces: scan_eager.py:160-169 and scan_compiled.py:262-277 when both
 *   incoming gradients are expanded (stride-0 in time) tensors, which the
 *   reference materialises with .contiguous() (scan_eager.py:161,166;
 *   scan_compiled.py:262-263).
 */
int asc_scan_bidi_bwd_rowgrad(
    const void* grad_fwd_rows, int64_t grad_fwd_row_stride,
    const void* grad_bwd_rows, int64_t grad_bwd_row_stride,
    const void* gates_fwd, const void* gates_bwd, const void* states_fwd,
    const void* states_bwd, void* d_tokens_fwd, void* d_gates_fwd,
    void* d_tokens_bwd, void* d_gates_bwd, const void* cu_seqlens,
    int cu_dtype, int64_t num_seq, int64_t num_channels, int64_t seq_stride,
    int dtype, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Segment-aware shift by one position with padding, on a contiguous
 * [num_channels, seq_len] tensor.
 *   backward = 1: out[:, p] = data[:, p-1], pad at every segment start
 *                 (p = cu_seqlens[s], s < num_seq)
 *   backward = 0: out[:, p] = data[:, p+1], pad at every segment end
 *                 (p = cu_seqlens[s] - 1, s >= 1)
 * Positions that are not a boundary read their neighbour; at the two row
 * ends the neighbour index wraps around (wrap = 1, torch.roll semantics of
 * the eager reference) or is clamped into the row (wrap = 0, the compiled
 * reference kernel).  pad_value is rounded to the tensor dtype.
 *
 * Replaces: _shift_pad.py:18-55 shift_pad (wrap = 1) and
 *   _shift_pad.py:63-165 _shift_pad_kernel / shift_pad_compiled (wrap = 0).
 */
int asc_shift_pad(const void* data, void* out, const void* cu_seqlens,
                  int cu_dtype, int64_t num_seq, int64_t num_channels,
                  int64_t seq_len, int dtype, double pad_value, int backward,
                  int wrap, void* stream);

/*
 * asc_shift_pad for any element strides: element (c, p) of data lives at
 * data + (c * data_row_stride + p * data_col_stride) elements, and likewise
 * for out (a transposed or sliced view needs no copy).  Strides are >= 0;
 * out must not overlap itself or data (ASC_E_ARG).  Values move as raw bits.
 * asc_shift_pad is this call with contiguous rows (strides seq_len, 1).
 *
 * Replaces: _shift_pad.py:140-157, whose kernel takes data.stride(0) and
 *   data.stride(1) and writes torch.empty_like(data).
 */
int asc_shift_pad_strided(const void* data, int64_t data_row_stride,
                          int64_t data_col_stride, void* out,
                          int64_t out_row_stride, int64_t out_col_stride,
                          const void* cu_seqlens, int cu_dtype, int64_t num_seq,
                          int64_t num_channels, int64_t seq_len, int dtype,
                          double pad_value, int backward, int wrap,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ASSOCSCAN_H */
