/* pararnn_amd — C ABI of the MI355X (gfx950) fused Newton + scan kernels.
 *
 * Plain pointers and sizes only.  All tensors are dense, row-major ("contiguous"
 * in torch terms) device buffers on the current HIP device; `stream` is a
 * hipStream_t passed as void* (NULL = the default stream).  Nothing here
 * allocates device memory or synchronises the host: scratch space comes from
 * the caller's `workspace` (size from the matching *_workspace_size call,
 * 256-byte aligned), and every entry point only enqueues work on `stream`.
 * Calls that share one workspace must not overlap in time.
 *
 * dtype codes: PRNN_F32 (float32), PRNN_BF16 (bfloat16 storage) and PRNN_F16
 * (float16 storage; kernels/precision.py:20-34 admits the same three).  All
 * arithmetic is fp32; 16-bit tensors are widened on load and rounded (nearest
 * even) on store, at the rounding points of the reference in that dtype.
 *
 * Return codes: PRNN_OK, or an error whose message prnn_last_error() returns
 * (thread-local).  The Python shim maps PRNN_ERR_VALUE -> ValueError,
 * PRNN_ERR_TYPE -> TypeError, PRNN_ERR_RUNTIME -> RuntimeError, as the
 * reference's ops raise them (kernels/newton_slstm.py:2725-2728,
 * kernels/precision.py:40-68, kernels/newton_gru_head.py:108-117).
 *
 * Reference interfaces replaced (paths relative to the reference's src/pararnn):
 *   prnn_slstm_init       -> solvers/slstm_picard.py:143-181
 *                            slstm_zero_hidden_init / slstm_picard_init, as
 *                            called by kernels/fused_newton.py:367-372
 *   prnn_slstm_newton     -> kernels/custom_ops.py:486-516
 *                            torch.library op pararnn::newton_slstm_fused
 *   prnn_gru_head_newton  -> kernels/custom_ops.py:311-358
 *                            torch.library op pararnn::newton_gru_head_fused
 *   prnn_slstm_backward   -> solvers/newton/__init__.py:765-866 (_eq26_vjp, diag
 *                            sLSTM path): reverse_scan_block4 (solvers/scan.py:
 *                            166-178) + slstm_recurrence_vjp (kernels/
 *                            vjp_slstm.py:209-240) + _t0_state_vjp
 *                            (solvers/newton/dispatch.py:406-410)
 *   prnn_gru_head_backward -> solvers/newton/__init__.py:798-817 (_eq26_vjp, head
 *                            GRU path): reverse_factor_scan_gru_head (kernels/
 *                            newton_gru_head.py:198-258) + gru_head_t0_vjp +
 *                            gru_head_recurrence_vjp (kernels/vjp_gru.py:656)
 *   prnn_slstm_decode     -> kernels/decode.py:420-467, 553-597 (_slstm_decode_kernel,
 *                            decode_step for ParaSLSTM mix='diag')
 *   prnn_gru_decode       -> kernels/decode.py:260-334, 472-501 (_gru_decode_kernel,
 *                            decode_step for ParaGRU mix='diag'); mix='head' replaces
 *                            the eager cell.step the reference runs for that mix
 *                            (cells/para_gru.py:443-467)
 */
#ifndef PARARNN_AMD_H
#define PARARNN_AMD_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PRNN_API __attribute__((visibility("default")))

enum { PRNN_F32 = 0, PRNN_BF16 = 1, PRNN_F16 = 2 };
enum { PRNN_OK = 0, PRNN_ERR_VALUE = 1, PRNN_ERR_TYPE = 2, PRNN_ERR_RUNTIME = 3 };

/* Library ABI version (bumped on any signature change or added entry point). */
PRNN_API int prnn_abi_version(void);
/* Message of the last failing call on this thread ("" if none). */
PRNN_API const char* prnn_last_error(void);

/* Deterministic mode, process-wide (off by default).  When on, every sLSTM
 * look-back scan (warm start, Newton, backward) produces bit-identical
 * results from run to run: a tile's carry is always the serial chain of
 * published tile aggregates, however the tiles were scheduled.  Off, carries
 * can differ in the last bits between runs (the walk may compose a different
 * set of predecessors).  The head GRU path is deterministic either way.
 * Replaces the reference's reliance on torch.use_deterministic_algorithms
 * (pararnn/determinism.py:41-45, checked at determinism.py:77-113): the
 * Python layer sets this from torch.are_deterministic_algorithms_enabled()
 * before each launch. */
PRNN_API void prnn_set_deterministic(int on);
PRNN_API int prnn_deterministic(void);

/* Bounded waits (no counterpart in the reference).  The sLSTM scans wait on
 * words their predecessor tiles publish; publication order guarantees that
 * they arrive, so a wait that polls more than `rounds` times (process-wide;
 * <= 0 restores the default, 4194304, seconds of polling) means a broken
 * invariant such as a foreign or stale workspace.  The waiting wave then
 * gives up: it takes NaN for the missing value (so the output shows it),
 * sets the call's status word and runs on, so every kernel still ends.
 * prnn_slstm_lookback_status copies that word (1 = a wait gave up, 0 = none)
 * from an sLSTM call's workspace to *status, synchronising `stream`. */
PRNN_API void prnn_set_spin_limit(int rounds);
PRNN_API int prnn_slstm_lookback_status(const void* workspace, int* status, void* stream);

/* Kernel timing, process-wide (off by default; no counterpart in the
 * reference, for benchmarks).  When on, the sLSTM entry points record a HIP
 * event pair on their stream around their main kernel(s) -- after the status
 * word clear: the warm start launch(es), the Newton launch(es), the reverse
 * scan -- and prnn_last_kernel_ms waits for the last pair and returns its
 * elapsed milliseconds (-1 if none).  Not for use under graph capture. */
PRNN_API void prnn_set_kernel_timing(int on);
PRNN_API float prnn_last_kernel_ms(void);

/* ---- ParaSLSTM mix='diag' ------------------------------------------------
 * Layouts: wx (B, T, 4d) gate blocks (i, f, z, o);  r (4, d) recurrent mix,
 * already clamped by the caller;  h0 (B, 4, d) slots (c, n, m, h) or NULL
 * (zeros);  states / out (B, T, 4, d) slots (c, n, m, h).
 * wx, r, h0, states and out all have the dtype `dtype`.
 */

/* Newton initial guess: the zero-hidden frozen-gate scan followed by
 * `picard_iters` frozen-gate passes that freeze the gates at
 * wx + r * h_prev of the previous pass; `states` receives the last pass. */
PRNN_API size_t prnn_slstm_init_workspace_size(int B, int T, int d, int picard_iters, int dtype);
PRNN_API int prnn_slstm_init(const void* wx, const void* r, const void* h0, void* states, int B,
                             int T, int d, int picard_iters, float eps, int dtype,
                             void* workspace, size_t workspace_bytes, void* stream);

/* `max_iters` Newton iterations from the guess `states` (read only);
 * `out` receives the result.  `out` must not alias `states`.  Iterations
 * between the first and the last keep the trajectory in fp32 inside the
 * workspace. */
PRNN_API size_t prnn_slstm_newton_workspace_size(int B, int T, int d, int max_iters, int dtype);
PRNN_API int prnn_slstm_newton(const void* wx, const void* r, const void* h0, const void* states,
                               void* out, int B, int T, int d, int max_iters, float omega,
                               float eps, int dtype, void* workspace, size_t workspace_bytes,
                               void* stream);

/* One Newton iteration with an fp32 result, for the host-checked early exit
 * (replaces the per-iteration body of kernels/newton_slstm.py:2780-2922 that
 * NewtonConfig.fused_early_exit runs, solvers/newton/__init__.py:696-762):
 * `in` is the current iterate, fp32 when in_f32 != 0 (the fp32 work iterate
 * of earlier steps) or else in `dtype` (the guess); `out` receives
 * in + omega * delta in fp32, exactly what the K-iteration call keeps
 * between its iterations.  Workspace: prnn_slstm_newton_workspace_size with
 * max_iters = 1; tag_base as for prnn_slstm_newton_ex. */
PRNN_API int prnn_slstm_newton_step(const void* wx, const void* r, const void* h0,
                                    const void* in, int in_f32, float* out, int B, int T, int d,
                                    float omega, float eps, int dtype, void* workspace,
                                    size_t workspace_bytes, int tag_base, void* stream);

/* ---- ParaGRU mix='head' --------------------------------------------------
 * Layouts: wx (B, T, 3d) gate blocks (z, r, n);  a_z, a_r, a_n
 * (n_heads, d_head, d_head) laid out (in, out) so y = h @ A per head;
 * h0 (B, d) or NULL;  out (B, T, d);  d = n_heads * d_head.
 * d_head must be 64.  The initial guess is f(h_prev0, x_t) with h_prev0 zero
 * except h0 at t = 0; then `max_iters` Newton iterations.
 */
PRNN_API size_t prnn_gru_head_newton_workspace_size(int B, int T, int n_heads, int d_head,
                                                    int max_iters, int dtype);
PRNN_API int prnn_gru_head_newton(const void* wx, const void* a_z, const void* a_r,
                                  const void* a_n, const void* h0, void* out, int B, int T,
                                  int n_heads, int d_head, int max_iters, float omega, int dtype,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* Packed sequences (replace the reference's cu_seqlens handling for the
 * diag sLSTM: the ragged frozen-gate scan solvers/slstm_picard.py:87-103 and
 * the J = 0 segment heads of solvers/scan.py:206-216 with layout.py:115-138,
 * and the paged h0 of kernels/_fused_common.py:106-139).  wx / states / out
 * hold one stream (B = 1) of T steps: sequence s occupies steps
 * [cu_seqlens[s], cu_seqlens[s+1]) (int32 device array of n_seq + 1 entries,
 * 0 = first < ... < last = T).  At the first step of each sequence the
 * previous state is the sequence's initial state -- h0 row block_table[s]
 * when block_table (n_seq int32 device entries) is given, else row s; zeros
 * when h0 is NULL -- and no carry crosses it.  The kernels read cu_seqlens
 * and block_table themselves: no padding, no gather, one launch set for the
 * whole stream.  Workspace from the *_packed_workspace_size calls; tag_base
 * as for the _ex calls.  The caller checks cu_seqlens (the kernels trust it):
 * it must rise strictly, since an empty sequence would make the kernels
 * assign every later step to the wrong sequence (wrong h0 and g_h0 rows).
 * The library itself rejects n_seq outside [1, T] with PRNN_ERR_VALUE. */
PRNN_API size_t prnn_slstm_init_packed_workspace_size(int T, int d, int picard_iters, int dtype);
PRNN_API int prnn_slstm_init_packed(const void* wx, const void* r, const void* h0, void* states,
                                    int T, int d, int picard_iters, float eps, int dtype,
                                    const int* cu_seqlens, int n_seq, const int* block_table,
                                    void* workspace, size_t workspace_bytes, int tag_base,
                                    void* stream);
PRNN_API size_t prnn_slstm_newton_packed_workspace_size(int T, int d, int max_iters, int dtype);
PRNN_API int prnn_slstm_newton_packed(const void* wx, const void* r, const void* h0,
                                      const void* states, void* out, int T, int d, int max_iters,
                                      float omega, float eps, int dtype, const int* cu_seqlens,
                                      int n_seq, const int* block_table, void* workspace,
                                      size_t workspace_bytes, int tag_base, void* stream);
PRNN_API int prnn_slstm_newton_step_packed(const void* wx, const void* r, const void* h0,
                                           const void* in, int in_f32, float* out, int T, int d,
                                           float omega, float eps, int dtype,
                                           const int* cu_seqlens, int n_seq,
                                           const int* block_table, void* workspace,
                                           size_t workspace_bytes, int tag_base, void* stream);

/* One Newton iteration with the reference's eager rounding (replaces the
 * loop body of solvers/newton/__init__.py:516-543 for scan_backend='eager':
 * step_and_jacobian in the tensor dtype, cells/para_slstm.py:241-281 and
 * :378-446, the fp32 block-4 scan of solvers/scan.py:82-100 and 229-246, and
 * the rounded update).  `in` is the current iterate and `out` receives the
 * next one, both (B, T, 4, d) in `dtype`: every cell and Jacobian op rounds to
 * `dtype` as the eager tensor op does, the residual is rounded, the scan runs
 * in fp32, delta is rounded, then in + omega * delta is rounded.  `out` must
 * not alias `in`.  Workspace: prnn_slstm_newton_workspace_size (packed:
 * prnn_slstm_newton_packed_workspace_size) with max_iters = 1; tag_base as
 * for the _ex calls; cu_seqlens / n_seq / block_table as for the packed
 * calls above. */
PRNN_API int prnn_slstm_newton_eager(const void* wx, const void* r, const void* h0,
                                     const void* in, void* out, int B, int T, int d, float omega,
                                     float eps, int dtype, void* workspace,
                                     size_t workspace_bytes, int tag_base, void* stream);
PRNN_API int prnn_slstm_newton_eager_packed(const void* wx, const void* r, const void* h0,
                                            const void* in, void* out, int T, int d, float omega,
                                            float eps, int dtype, const int* cu_seqlens,
                                            int n_seq, const int* block_table, void* workspace,
                                            size_t workspace_bytes, int tag_base, void* stream);

/* Eq. 2.6 backward at the solved trajectory `states` = H* (B, T, 4, d) with
 * upstream gradient `grad` = dL/dH (B, T, 4, d):
 *   mu_{T-1} = grad_{T-1},  mu_t = grad_t + J_{t+1}^T mu_{t+1}  (fp32),
 * then the VJP of every step f(H*_{t-1}, wx_t) with mu_t:
 *   g_wx (B, T, 4d), dtype `dtype`:  dL/dwx (the W_x GEMMs stay with the caller);
 *   g_r  (4, d) fp32:                sum over (b, t) of dL/dz_g * h_{t-1}, before
 *                                    the caller's clamp mask on R;
 *   g_h0 (B, 4, d) fp32 or NULL:     J_0^T mu_0 (gradient of h0).
 * h0 as in the forward (NULL = zeros).  g_r is deterministic (fixed-order sums).
 */
PRNN_API size_t prnn_slstm_backward_workspace_size(int B, int T, int d, int dtype);
PRNN_API int prnn_slstm_backward(const void* wx, const void* r, const void* h0,
                                 const void* states, const void* grad, void* g_wx, float* g_r,
                                 float* g_h0, int B, int T, int d, float eps, int dtype,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* Tagged-workspace variants of the three sLSTM calls (no counterpart in the
 * reference; for callers that keep one workspace across calls).  The sLSTM
 * look-back exchanges {value, tag} words through the workspace; a word is
 * valid when its tag is one of the call's.  With tag_base = 0 (what the plain
 * calls do) every such word is cleared first -- a write of the whole
 * look-back area (~0.6 GB at B=1, T=131072, d=1024, K=2: ~80 us).  With
 * tag_base > 0 only the 64 ticket counters are cleared and the call's tags
 * are tag_base + 1 .. tag_base + PRNN_TAG_SPAN.  The caller then guarantees
 * that every word of the workspace is either zero or was written by an
 * earlier call with a smaller tag_base (the workspace was zero-filled once
 * and only these calls have written it since; advance tag_base by at least
 * PRNN_TAG_SPAN per call; re-zero it before tag_base would pass
 * PRNN_TAG_BASE_MAX).  Not for HIP graph capture: a replay would repeat the
 * captured tags. */
#define PRNN_TAG_SPAN 64
#define PRNN_TAG_BASE_MAX (1 << 30)
PRNN_API int prnn_slstm_init_ex(const void* wx, const void* r, const void* h0, void* states,
                                int B, int T, int d, int picard_iters, float eps, int dtype,
                                void* workspace, size_t workspace_bytes, int tag_base,
                                void* stream);
PRNN_API int prnn_slstm_newton_ex(const void* wx, const void* r, const void* h0,
                                  const void* states, void* out, int B, int T, int d,
                                  int max_iters, float omega, float eps, int dtype,
                                  void* workspace, size_t workspace_bytes, int tag_base,
                                  void* stream);
/* prnn_slstm_backward_ex also returns, when g_b is not NULL, the W_x bias
 * gradient g_b (4, d) fp32: the sum over (b, t) of dL/dwx (of the fp32 values
 * that g_wx rounds), reduced in a fixed order with g_r -- one pass less than
 * summing g_wx afterwards. */
PRNN_API int prnn_slstm_backward_ex(const void* wx, const void* r, const void* h0,
                                    const void* states, const void* grad, void* g_wx,
                                    float* g_r, float* g_h0, float* g_b, int B, int T, int d,
                                    float eps, int dtype, void* workspace,
                                    size_t workspace_bytes, int tag_base, void* stream);

/* Allocation-free variant of prnn_slstm_newton.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * workspace is a library-owned device array of
 * prnn_slstm_newton_noalloc_max_bytes() bytes (64 MiB) per GPU, held until the
 * process ends; shapes whose prnn_slstm_newton_workspace_size exceeds it are
 * rejected with PRNN_ERR_VALUE.  The call allocates nothing and clears what
 * it reads of the array first (a fill kernel on `stream`).  All calls on one
 * GPU share that GPU's array: calls that overlap in time on one GPU (two
 * streams, two host threads) race and give wrong results. */
PRNN_API size_t prnn_slstm_newton_noalloc_max_bytes(void);
PRNN_API int prnn_slstm_newton_noalloc(const void* wx, const void* r, const void* h0,
                                       const void* states, void* out, int B, int T, int d,
                                       int max_iters, float omega, float eps, int dtype,
                                       void* stream);

/* Eq. 2.6 backward of a packed stream (cu_seqlens as for the packed forward;
 * replaces the reference's ragged reverse scan with J = 0 at heads,
 * solvers/scan.py:206-216 reversed, solvers/newton/__init__.py:765-866):
 * nothing flows from a sequence's first step to the step before it, and
 * g_h0 (n_seq, 4, d) fp32 (or NULL) receives J_head^T mu_head per sequence,
 * the gradient of that sequence's h0 row.  Workspace as
 * prnn_slstm_backward_workspace_size(1, T, d, dtype). */
PRNN_API int prnn_slstm_backward_packed(const void* wx, const void* r, const void* h0,
                                        const void* states, const void* grad, void* g_wx,
                                        float* g_r, float* g_h0, float* g_b, int T, int d,
                                        float eps, int dtype, const int* cu_seqlens, int n_seq,
                                        void* workspace, size_t workspace_bytes, int tag_base,
                                        void* stream);

/* Eq. 2.6 backward of the head GRU at `states` = H* (B, T, d) with upstream
 * gradient `grad` = dL/dH (B, T, d) (both in `dtype`):
 *   mu_{T-1} = grad_{T-1},  mu_t = grad_t + J_{t+1}^T mu_{t+1}  (fp32),
 * then the VJP of every step f(H*_{t-1}, wx_t) with mu_t:
 *   g_wx (B, T, 3d), dtype `dtype`:  dL/dwx (the W_x GEMMs stay with the caller);
 *   g_a  (3, n_heads, 64, 64) fp32:  dL/dA_z, dL/dA_r, dL/dA_n ((in, out) layout),
 *                                    before the caller's clamp masks;
 *   g_h0 (B, d) fp32 or NULL:        J_0^T mu_0, written only when h0 is non-NULL.
 * a_* are the (clamped) matrices the forward used.  g_a is deterministic
 * (fixed-order sums).
 */
PRNN_API size_t prnn_gru_head_backward_workspace_size(int B, int T, int n_heads, int d_head,
                                                      int dtype);
PRNN_API int prnn_gru_head_backward(const void* wx, const void* a_z, const void* a_r,
                                    const void* a_n, const void* h0, const void* states,
                                    const void* grad, void* g_wx, float* g_a, float* g_h0, int B,
                                    int T, int n_heads, int d_head, int dtype, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* Wide heads, 64 < d_head <= 128 (replaces the reference's streamed head
 * tier, kernels/newton_gru_head.py:121-150 and its _newton_head_stream_a_kernel
 * at :765-960, one program per (b, head) walking T).  The gates of every
 * step at the current iterate -- z, r, n (B, T, d) fp32 from hp, the previous
 * state of every step (h0's row at a sequence start) -- come first, for all
 * rows at once (prnn_gru_wide_gates below); these walk time, one workgroup
 * per (sequence, head), A_* (n_heads, d_head, d_head) in `dtype`, fp32 work.
 *
 * prnn_gru_wide_walk: one Newton iteration's linear solve and update,
 *   delta_t = J_t delta_{t-1} + lerp(hp_t, n_t, z_t) - hin_t,
 *   out_t = hin_t + omega delta_t
 * (out fp32 when out_f32, which may alias hin; else `dtype`).
 * prnn_gru_wide_reverse: the eq. 2.6 adjoint at H* (hp from H*), grad =
 * dL/dH (fp32 when grad_f32, else `dtype`): g_wx (B, T, 3d) fp32 receives the
 * pre-activation gradients (z, r, n blocks), g_h0 (rows, d) fp32 (or NULL)
 * J^T mu at each sequence's first step.
 * cu_seqlens / n_seq: a packed stream (B = 1) walked per sequence, or NULL. */
PRNN_API int prnn_gru_wide_walk(const float* z, const float* r, const float* n, const float* hp,
                                const float* hin, const void* a_z, const void* a_r,
                                const void* a_n, void* out, int out_f32, int B, int T,
                                int n_heads, int d_head, float omega, int dtype,
                                const int* cu_seqlens, int n_seq, void* stream);
PRNN_API int prnn_gru_wide_reverse(const float* z, const float* r, const float* n,
                                   const float* hp, const void* grad, int grad_f32,
                                   const void* a_z, const void* a_r, const void* a_n,
                                   float* g_wx, float* g_h0, int B, int T, int n_heads,
                                   int d_head, int dtype, const int* cu_seqlens, int n_seq,
                                   void* stream);

/* The gates of every row (b, t) of the wide tier at its previous state:
 * z = sigmoid(wx_z + hp A_z), r = sigmoid(wx_r + hp A_r),
 * n = tanh(wx_n + (hp r) A_n) per head (the cell of cells/para_gru.py:443-467
 * that the reference's streamed kernel evaluates inside its walk).  wx
 * (rows, 3d) and A_* in `dtype`, hp (rows, d) fp32 (h0's row, or zeros, at a
 * sequence's first step), z, r, n (rows, d) fp32. */
PRNN_API int prnn_gru_wide_gates(const void* wx, const float* hp, const void* a_z,
                                 const void* a_r, const void* a_n, float* z, float* r, float* n,
                                 int rows, int n_heads, int d_head, int dtype, void* stream);

/* All max_iters Newton iterations of the wide tier in one launch, without the
 * host's gate GEMMs: per iteration k and (sequence, head), gate workgroups
 * evaluate the gates at the previous iterate and a walk consumes them, a few
 * blocks of steps behind iteration k - 1; the iterate and the gates pass
 * through the workspace as tagged words (same replaced reference tier as
 * above; its program per (b, head) runs the iterations one after another).
 * wx (B, T, 3d) and A_* in `dtype`; h0 (rows, d) fp32 or NULL; guess
 * (B, T, d) fp32, the initial iterate; out (B, T, d) in `dtype` receives the
 * last iterate and must not alias guess.  Workspace:
 * prnn_gru_wide_newton_workspace_size, 8 bytes per element of (B, T, d) for
 * each of max_iters - 1 iterates and six gate planes (three for max_iters
 * 1); tag_base as for the sLSTM _ex calls (0: the call clears the whole
 * workspace), and the status word of a wait that gave up reads with
 * prnn_slstm_lookback_status.
 * max_iters in [1, PRNN_TAG_SPAN]. */
PRNN_API size_t prnn_gru_wide_newton_workspace_size(int B, int T, int n_heads, int d_head,
                                                    int max_iters);
PRNN_API int prnn_gru_wide_newton(const void* wx, const void* a_z, const void* a_r,
                                  const void* a_n, const float* h0, const float* guess,
                                  void* out, int B, int T, int n_heads, int d_head,
                                  int max_iters, float omega, int dtype, const int* cu_seqlens,
                                  int n_seq, void* workspace, size_t workspace_bytes,
                                  int tag_base, void* stream);

/* Head GRU on a packed stream: wx (1, T, 3d) holds n_seq sequences, sequence
 * q on steps [cu_seqlens[q], cu_seqlens[q+1]) (int32 device array, n_seq + 1
 * entries, 0 = cu_seqlens[0] < ... < cu_seqlens[n_seq] = T).  At a sequence's
 * first step the carry is cut (the reference's packed semantics:
 * solvers/scan.py:206-216, layout.py:93-138; its fused head op,
 * kernels/custom_ops.py:311-358, takes rectangular batches only) and the
 * previous state is h0 row block_table[q] (row q when block_table is NULL;
 * zeros when h0 is NULL).  out: (1, T, d).  The library builds the stream's
 * head table in the workspace. */
PRNN_API size_t prnn_gru_head_newton_packed_workspace_size(int T, int n_heads, int d_head,
                                                           int max_iters, int dtype);
PRNN_API int prnn_gru_head_newton_packed(const void* wx, const void* a_z, const void* a_r,
                                         const void* a_n, const void* h0, void* out, int T,
                                         int n_heads, int d_head, int max_iters, float omega,
                                         int dtype, const int* cu_seqlens, int n_seq,
                                         const int* block_table, void* workspace,
                                         size_t workspace_bytes, void* stream);

/* Eq. 2.6 backward of a packed head-GRU stream (cu_seqlens as above):
 * nothing flows from a sequence's first step to the step before it, and
 * g_h0 (n_seq, d) fp32 (or NULL; written only when h0 is non-NULL) receives
 * J_head^T mu_head per sequence. */
PRNN_API size_t prnn_gru_head_backward_packed_workspace_size(int T, int n_heads, int d_head,
                                                             int dtype);
PRNN_API int prnn_gru_head_backward_packed(const void* wx, const void* a_z, const void* a_r,
                                           const void* a_n, const void* h0, const void* states,
                                           const void* grad, void* g_wx, float* g_a,
                                           float* g_h0, int T, int n_heads, int d_head,
                                           int dtype, const int* cu_seqlens, int n_seq,
                                           void* workspace, size_t workspace_bytes,
                                           void* stream);

/* ---- T = 1 decode (serving loop) -----------------------------------------
 * One recurrent step.  state / out: (rows, 4, d) sLSTM or (rows, d) GRU;
 * wx: (B, 4d) / (B, 3d) for this step.  block_table: NULL (row b of state is
 * batch b, out has state's shape) or B int32 slot ids into pool-shaped
 * state / out (in place when out == state).  The recurrent parameters (r
 * (4, d); GRU a_* (d) for n_heads = 0, or (n_heads, 64, 64) (in, out)) are
 * clamped to +-cap in the kernel when has_cap.  No workspace.
 */
PRNN_API int prnn_slstm_decode(const void* state, const void* wx, const void* r, void* out,
                               const int* block_table, int B, int d, float eps, float cap,
                               int has_cap, int dtype, void* stream);
PRNN_API int prnn_gru_decode(const void* h, const void* wx, const void* a_z, const void* a_r,
                             const void* a_n, void* out, const int* block_table, int B, int d,
                             int n_heads, float cap, int has_cap, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PARARNN_AMD_H */
