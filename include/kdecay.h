/*
 * kdecay.h — C ABI of libkdecay.so, the gfx950 (MI355X) global-decay scan.
 *
 * The operation (per batch b, head h, channel d, position t):
 *
 *     s_t = lam_h * s_{t-1} + V_t                 (s_{-1} = init state, or 0)
 *     z_t = (1 - lam_h^(t+1)) / ((1 - lam_h) + 1e-6)
 *     y_t = s_t / z_t
 *
 * with t counted from `t_offset` (0 for a whole sequence).  This is the
 * recurrence of the reference's CPU path
 *     /root/reference/src/kilat/arc/triton_ops.py:232-247  (_cpu_global_decay)
 * which is also what its Triton kernel approximates
 *     /root/reference/src/kilat/arc/triton_ops.py:6-230    (flash_decay_fwd_kernel)
 * and of the inline incremental update in the attention layer
 *     /root/reference/src/kilat/arc/attention.py:344-360   (twin :710-717).
 *
 * Conventions of every entry point:
 *   - returns 0 on success; a negative KDECAY_E* code for a rejected argument
 *     (nothing was launched); a positive hipError_t if a HIP call failed.
 *     kdecay_last_error_string() describes the last failure of the calling
 *     thread.
 *   - pointers are device pointers unless stated otherwise; strides are in
 *     elements, never bytes.
 *   - nothing is allocated and nothing is synchronised: work is enqueued on
 *     `stream` (a hipStream_t; NULL is the legacy default stream).
 *   - lam is float32 [H]: decay factors, already passed through the sigmoid
 *     (the reference computes lam = sigmoid(log_lambda) in the caller,
 *     attention.py:319).
 */
#ifndef KDECAY_H
#define KDECAY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of V, y, v_t and the step output.  KDECAY_F64 is taken by
 * the three forward scans only (kdecay_scan_fwd, kdecay_scan_fwd_noalloc,
 * kdecay_scan_fwd_sequential), for V and out together; every other entry
 * point returns KDECAY_EDTYPE for it.  Arithmetic is fp32 for every type, as
 * in the reference's kernel, which accumulates in fp32 whatever V's dtype
 * (triton_ops.py:149-152) and stores into out = empty_like(V) (:309). */
enum {
  KDECAY_F32 = 0,
  KDECAY_BF16 = 1,
  KDECAY_F16 = 2,
  KDECAY_F64 = 3
};

/* Rejected-argument codes (negative). */
enum {
  KDECAY_EINVAL = -1,     /* null pointer where one is required, negative size */
  KDECAY_EDTYPE = -2,     /* unsupported dtype code or dtype combination       */
  KDECAY_ESHAPE = -3,     /* unsupported head dim D                            */
  KDECAY_ELAYOUT = -4,    /* strides / alignment the vector path cannot take   */
  KDECAY_EWORKSPACE = -5  /* workspace missing or smaller than required        */
};

/*
 * Full-sequence scan.
 * Replaces triton_global_decay(lam_scores, V) -> out
 *   /root/reference/src/kilat/arc/triton_ops.py:249-330
 * whose GPU branch launches flash_decay_fwd_kernel (:6-230) with V's and
 * out's four strides (:324-330) into out = torch.empty_like(V) (:309).
 *
 *   V            [B,H,N,D] of v_dtype, strides v_strides[4]
 *   out          [B,H,N,D] of out_dtype, strides out_strides[4]
 *                (out_dtype == v_dtype reproduces the reference; F32 out for
 *                 a BF16/F16 V is also accepted; an F64 V takes F64 out only)
 *   init_state   nullable; fp32 [B,H,D] contiguous: state before position 0
 *                (chunked prefill).  NULL means zeros, as the reference.
 *   final_state  nullable; fp32 [B,H,D] contiguous: receives s_{N-1}, the
 *                unnormalised state the reference seeds its decode cache
 *                with in a Python loop (attention.py:383-394, :722-727).
 *   t_offset     absolute position of row 0 (enters z only); 0 for a whole
 *                sequence.
 *   stream       the HIP stream the work goes to: one kernel launch, or for
 *                heads of one 128-byte channel group with more than one
 *                resident round of short streams, a few launches over
 *                slices of the batch, in order on this stream (also under
 *                stream capture).
 *   workspace    device memory of kdecay_scan_workspace_bytes() bytes,
 *                256-byte aligned, zeroed once by the caller before its first
 *                use.  It holds the look-back words of the chunks and a
 *                header (launch epoch, completion counts, a sticky error
 *                word).  Each launch advances the epoch on the device,
 *                so the workspace needs no clearing between launches (also
 *                under stream capture and graph replay), but it must not be
 *                shared by two launches that can run at the same time (use
 *                one per stream).  A non-zero error word (header word 1,
 *                bytes 4-7: a look-back gave up waiting) stays set until the
 *                caller zeroes the whole workspace.  Outputs the launch that
 *                gave up could not compute (the rows of a chunk whose
 *                look-back gave up, and any later rows or final state whose
 *                carry came through that chunk) are written as NaN, never as
 *                finite wrong values.  While the word is set, every later
 *                launch on that workspace writes NaN to all its outputs (out
 *                and final_state) without waiting on anything: the launch
 *                that gave up may have left look-back words tagged as a later
 *                launch's, so only a zeroed workspace computes again.  (A
 *                launch of one chunk per stream uses no workspace and is not
 *                affected.)  It may be NULL when
 *                kdecay_scan_workspace_bytes() returns 0.
 *
 * Requirements of this (vector) path: D = 16, 32, or a multiple of 64 (bf16,
 * fp16), 32 (fp32) or 16 (fp64) channels; d-stride 1; 16-byte aligned V and
 * out; the other strides multiples of 16 bytes.
 * Anything else returns KDECAY_ELAYOUT / KDECAY_ESHAPE without launching.
 */
int kdecay_scan_fwd(const void* V, int v_dtype, const int64_t* v_strides,
                    void* out, int out_dtype, const int64_t* out_strides,
                    const float* lam, const float* init_state,
                    float* final_state, int64_t B, int64_t H, int64_t N,
                    int64_t D, int64_t t_offset, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Bytes of workspace kdecay_scan_fwd needs for this shape (0: none). */
size_t kdecay_scan_workspace_bytes(int64_t B, int64_t H, int64_t N, int64_t D,
                                   int v_dtype);

/* Size of the fixed device array kdecay_scan_fwd_noalloc uses as workspace. */
#define KDECAY_NOALLOC_WORKSPACE_BYTES ((size_t)8 << 20)

/*
 * Full-sequence scan that allocates nothing: kdecay_scan_fwd with the same
 * kernels and the same results, but its look-back workspace is a fixed array
 * of KDECAY_NOALLOC_WORKSPACE_BYTES (8 MiB) in the library's own device
 * memory, one per GPU, held until the process ends.
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory or own a workspace: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  The caller still passes
 * V, out, lam and the optional states; no hipMalloc, hipFree or other
 * allocating call is made.
 *   - Shapes whose kdecay_scan_workspace_bytes() exceeds
 *     KDECAY_NOALLOC_WORKSPACE_BYTES (about 16K chunks: 1 GiB of bf16 V) are
 *     rejected with KDECAY_EWORKSPACE before anything is launched.
 *   - The array is zero-filled when the library's code object is loaded on
 *     a GPU; the first call only looks its address up (nothing is launched
 *     or recorded for it, also under stream capture), and nothing clears it
 *     again.
 *   - Every call on one GPU in a process shares that GPU's array (each
 *     process has its own): calls that can overlap on one GPU (two streams,
 *     two threads) race and give wrong results; serialise them, e.g. on one
 *     stream.  The array keeps the last call's contents (launch epoch and
 *     look-back words), which the next call needs no clearing for.
 *   - A look-back give-up leaves NaN in the outputs it could not compute, as
 *     kdecay_scan_fwd does, and sets the sticky error word in the array.
 *     That word is not readable through this API and the array is never
 *     cleared: from then on every call of this entry point on that GPU in the
 *     process that needs a workspace (several chunks per stream) writes NaN
 *     to all its outputs, which a caller checking for finite outputs sees.
 * Every other argument as kdecay_scan_fwd.
 */
int kdecay_scan_fwd_noalloc(const void* V, int v_dtype,
                            const int64_t* v_strides, void* out,
                            int out_dtype, const int64_t* out_strides,
                            const float* lam, const float* init_state,
                            float* final_state, int64_t B, int64_t H,
                            int64_t N, int64_t D, int64_t t_offset,
                            void* stream);

/*
 * Straight sequential scan: one lane per (b,h,d) column walks all N
 * positions.  Same arguments and results as kdecay_scan_fwd (any strides, any
 * D in 1..1024), no workspace.  Slow; it is the structurally independent
 * second implementation the parity tests cross-check the chunked scan with.
 * Same reference interface as kdecay_scan_fwd.
 */
int kdecay_scan_fwd_sequential(const void* V, int v_dtype,
                               const int64_t* v_strides, void* out,
                               int out_dtype, const int64_t* out_strides,
                               const float* lam, const float* init_state,
                               float* final_state, int64_t B, int64_t H,
                               int64_t N, int64_t D, int64_t t_offset,
                               void* stream);

/*
 * Forward scan for training: kdecay_scan_fwd, plus what the backward pass
 * needs: the state at every kdecay_scan_bwd chunk boundary (so the backward
 * recomputes s inside each chunk without a second look-back), and each row's
 * 1/z and d(1/z)/dlam for every head (so the backward loads them instead of
 * computing them before its first row).
 * The reference has no GPU backward (its Triton path returns a tensor with no
 * autograd graph, triton_ops.py:309-330); its CPU path is differentiated by
 * torch autograd through /root/reference/src/kilat/arc/triton_ops.py:240-246.
 * This pair replaces that autograd path on the GPU.
 *
 *   states         fp32, kdecay_scan_saved_states_floats() floats (may be NULL
 *                  when that is 0); pass it unchanged to kdecay_scan_bwd.
 * Every other argument as kdecay_scan_fwd.
 */
int kdecay_scan_fwd_train(const void* V, int v_dtype, const int64_t* v_strides,
                          void* out, int out_dtype, const int64_t* out_strides,
                          const float* lam, const float* init_state,
                          float* final_state, float* states,
                          size_t states_floats, int64_t B, int64_t H,
                          int64_t N, int64_t D, int64_t t_offset,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/* Floats of the states buffer kdecay_scan_fwd_train fills (0: none needed):
 * B*H*D per backward chunk boundary plus 2*H*N row terms. */
size_t kdecay_scan_saved_states_floats(int64_t B, int64_t H, int64_t N,
                                       int64_t D, int v_dtype);

/*
 * Backward of the full-sequence scan (see kdecay_scan_fwd_train):
 *   g_t  = gy_t / z_t + lam * g_{t+1}   (+ g_final at t = N-1; g_N = 0)
 *   dV   = g,   d_init = lam * g_0,
 *   dlam[h] = sum over b, d, t of  g_t * s_{t-1} + gy_t * s_t * d(1/z_t)/dlam
 * with s the forward states (s_{-1} = init_state or 0).
 *
 *   V, gy, dV    [B,H,N,D] of v_dtype (gy and dV share V's dtype), strided as
 *                kdecay_scan_fwd's V; the row strides of V and gy must not
 *                be negative, and one backward chunk of rows must span less
 *                than 2^31 bytes (rows are addressed by 32-bit offsets), else
 *                KDECAY_ELAYOUT.  A chunk is 4 wavefronts x (64 / lanes per
 *                row) x 16 rows: 512 rows for a 128-byte channel group (D >=
 *                64 bf16/fp16, D >= 32 fp32), 1024 for 64 bytes, 2048 for 32
 *                bytes; a quarter of that for small grids; 256 rows of whole
 *                256-byte rows for bf16/fp16 heads with a multiple of 128
 *                channels on large grids with chains of at most 32 chunks;
 *                256 rows of a 128-byte group for heads of two or more such
 *                groups on grids of more than one round with at least 48
 *                streams.  (The library checks the limit itself; these
 *                sizes say which row strides it accepts.)
 *   lam, init_state, t_offset   as given to the forward call (the row terms
 *                come from the states buffer, computed with the forward's
 *                lam and t_offset)
 *   states       the forward call's states (NULL allowed when
 *                kdecay_scan_saved_states_floats() is 0)
 *   g_final      nullable fp32 [B,H,D]: gradient of the forward's final state
 *   dlam         fp32 [H], overwritten (summed over B, D and t in a fixed
 *                order: deterministic).  One-group heads whose grid is exactly
 *                two or three resident rounds run as that many launches over
 *                slices of the batch, in order on `stream`; the last adds
 *                the earlier slices' sums (kept in double in the workspace)
 *                in slice order, so dlam is still one value per head.
 *   d_init       nullable fp32 [B,H,D]
 *   workspace    kdecay_scan_bwd_workspace_bytes() bytes, 256-byte aligned,
 *                zeroed once; same rules as kdecay_scan_fwd's (it may be the
 *                same buffer when large enough).  A bounded wait that gives
 *                up sets the error word and leaves NaN in the gradients it
 *                could not compute (dV rows, the head's dlam).  While the
 *                word is set, every later backward on that workspace writes
 *                NaN to all of dV, dlam and d_init, as the forward does.
 */
int kdecay_scan_bwd(const void* V, int v_dtype, const int64_t* v_strides,
                    const void* gy, const int64_t* gy_strides, void* dV,
                    const int64_t* dv_strides, const float* lam,
                    const float* init_state, const float* states,
                    const float* g_final, float* dlam, float* d_init,
                    int64_t B, int64_t H, int64_t N, int64_t D,
                    int64_t t_offset, void* workspace, size_t workspace_bytes,
                    void* stream);

/* Bytes of workspace kdecay_scan_bwd needs for this shape. */
size_t kdecay_scan_bwd_workspace_bytes(int64_t B, int64_t H, int64_t N,
                                       int64_t D, int v_dtype);

/*
 * Incremental (decode) step for a whole batch, one launch.
 * Replaces the inline update
 *   new_state = lam.view(1,H,1) * past_state + V_current
 *   z_inc     = (1 - lam**(t_pos+1)) / (1 - lam + 1e-6)
 *   out       = new_state / z_inc
 *   /root/reference/src/kilat/arc/attention.py:344-360 (twin :710-717)
 *
 *   state_in   fp32 [B,H,D] contiguous (the cache's global_state, :68-70)
 *   v_t        [B,H,D] contiguous of v_dtype (V_current, :343)
 *   state_out  fp32 [B,H,D]; may alias state_in (in-place update)
 *   out        [B,H,D] of out_dtype (F32 reproduces the reference's type
 *              promotion; BF16/F16 are rounded once from fp32)
 *   t_pos      nullable int32 [B]: position of each sequence's new token.
 *              NULL uses t_pos_scalar for every sequence, as the reference
 *              does (t_pos = past_latent_kv.shape[1], :357-358).
 * new_state is bit-identical to the reference's: one fp32 multiply and one
 * fp32 add, each rounded (never fused).
 */
int kdecay_step(const float* lam, const float* state_in, const void* v_t,
                int v_dtype, float* state_out, void* out, int out_dtype,
                const int32_t* t_pos, int64_t t_pos_scalar, int64_t B,
                int64_t H, int64_t D, void* stream);

/* Library version string, e.g. "kdecay 0.1.0 gfx950". */
const char* kdecay_version(void);

/* Message for the calling thread's last non-zero return ("" if none). */
const char* kdecay_last_error_string(void);

/*
 * Test hook, no counterpart in the reference: the bounded waits of later
 * launches (chunk look-back, the backward's dlam reduction) give up after
 * `polls` polls instead of about a second's worth, so a test can force the
 * give-up path: the launch still returns, the outputs it could not compute
 * are NaN and the workspace's sticky error word is set.  polls <= 0 restores
 * the default.
 * Process-wide, not thread-safe; returns the previous setting (0: default).
 */
int kdecay_debug_set_spin_limit(int polls);

/*
 * Test hook, no counterpart in the reference: the quotient n / d (want_mod
 * == 0) or remainder n % d as the kernels compute it, by the multiply and
 * shift the library derives for d on the host (valid for 0 <= n < 2^31,
 * 1 <= d < 2^31), so a CPU test can check it against exact division.
 */
uint32_t kdecay_debug_fastdiv(uint32_t n, uint32_t d, int want_mod);

#ifdef __cplusplus
}
#endif

#endif /* KDECAY_H */
