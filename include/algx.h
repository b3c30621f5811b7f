/*
 * algx -- MI355X (gfx950) kernels for the algebraic-extra hot path, C ABI.
 *
 * Every entry point takes caller-owned device pointers, plain sizes and a
 * hipStream_t (passed as void*), enqueues HIP kernels on that stream and
 * returns 0, or a nonzero status with a message from algx_last_error().
 * No entry point allocates device memory or synchronises with the host:
 * scratch memory is a caller-provided workspace whose size the matching
 * *_workspace_bytes() query reports. Calls on different streams/devices are
 * independent. Library state: the thread-local error text and one
 * process-wide timing probe (algx_set_probe, a benchmark diagnostic that is
 * off unless armed); no entry point's results depend on either.
 *
 * Layouts are row-major as the reference passes them: attention tensors are
 * (B, H, T, D); the head takes hidden states (N, d) and the tied embedding
 * (V, d); QK-norm takes rows of D=64 values, rms_norm rows of d_model values.
 */
#ifndef ALGX_H
#define ALGX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ALGX_BF16 = 0, ALGX_F32 = 1 };
enum { ALGX_SOFTMAX = 0, ALGX_ASINH = 1 };
enum { ALGX_HEAD_CE = 0, ALGX_HEAD_ALG_CE = 1 };
/* State of the backward workspace handed to algx_attn_bwd: RAW = contents
 * unspecified; CLEARED = the same buffer was passed as bwd_workspace to the
 * algx_attn_forward call whose outputs the backward receives, with no other
 * use in between (its dQ accumulator is then already zero). */
enum { ALGX_ATTN_WS_RAW = 0, ALGX_ATTN_WS_CLEARED = 1 };

/* Numeric variant of the attention kernels; mirrors the numeric fields of the
 * reference's Variant (src/algebraic/kernels/flash.py:59-73). Schedule flags
 * of the reference (resident_bwd, diagonal_*, head_resident, compact_stat)
 * select TPU schedules only and have no counterpart here. */
typedef struct {
  int32_t kind;            /* ALGX_SOFTMAX or ALGX_ASINH                       */
  int32_t n;               /* asinh power, a power of two >= 2                 */
  int32_t shift;           /* running-maximum accumulation                     */
  int32_t fast_rho;        /* x + sqrt(1+x^2) without the negative-x reciprocal */
  int32_t inv_stat;        /* unshifted statistic 1/Z instead of Z^(-1/n)      */
  int32_t bounded_scores;  /* guard passed: no clamp of scores                 */
  int32_t precise_output;  /* also write the float32 output (o_precise)        */
  float clamp;             /* score clamp when !shift && !bounded_scores       */
  int32_t poly_rho;        /* bounded radical (radical.py:26-38): polynomial   *
                            * on |x| <= 1; asinh, shift=False, n = 16 and     *
                            * bounded_scores=0 only (the reference refuses    *
                            * range_guard with it, flash.py:835-836)          */
} algx_attn_variant;

/* Text of the last error on this thread ("" when none). */
const char* algx_last_error(void);
/* Library ABI version (increments on incompatible changes). */
int32_t algx_version(void);
/* Diagnostic without a reference counterpart: one 32x32x16 bf16 MFMA with the
 * lane layout every MFMA kernel of the library assumes. a: 32x16 bf16 (row
 * major), bt: B^T as 32x16 bf16 (row major), d: 32x32 float32 = a @ b. */
int32_t algx_selftest_mfma32(const void* a, const void* bt, float* d, void* stream);

/* Diagnostic without a reference counterpart, for benchmarks: while set, the
 * named kernel is launched with hipExtLaunchKernel and the caller's HIP events
 * `start` and `stop` recorded as part of its dispatch, on the stream it runs
 * on (which = ALGX_PROBE_NONE clears). No extra packets enter the stream, so a
 * probed kernel runs as it does unprobed. The setting is process-wide
 * (backward passes often run on another thread). */
enum {
  ALGX_PROBE_NONE = 0,
  ALGX_PROBE_ATTN_FWD = 1,   /* main attention forward kernel                  */
  ALGX_PROBE_ATTN_BWD = 2,   /* main attention backward kernel                 */
  ALGX_PROBE_HEAD_FWD = 3,   /* fused-head forward statistics kernel           */
  ALGX_PROBE_HEAD_DZ = 4,    /* fused-head backward logit-gradient kernel      */
  ALGX_PROBE_HEAD_DH = 5,    /* unused: dh runs in the ALGX_PROBE_HEAD_DE launch */
  ALGX_PROBE_HEAD_DE = 6,    /* fused-head dh + dE GEMM launch                 */
  ALGX_PROBE_QKNORM_FWD = 7,
  ALGX_PROBE_QKNORM_BWD = 8,
  ALGX_PROBE_RMSNORM_FWD = 9,
  ALGX_PROBE_RMSNORM_BWD = 10, /* the row kernel; the dgain finish is not timed  */
  ALGX_PROBE_ALU_FWD = 11,     /* alu and alu_glu forward                        */
  ALGX_PROBE_ALU_BWD = 12      /* alu and alu_glu backward                       */
};
int32_t algx_set_probe(int32_t which, void* start_event, void* stop_event);

/* ---------------------------------------------------------------- QK norm
 * Replaces qk_rms_norm (src/algebraic/kernels/qk_norm.py:62-76) with its
 * custom VJP (:29-59) and the rms_norm math (src/algebraic/algebraic.py:76-83):
 *   y = cast(x * rsqrt(mean(x^2) + eps) * gain)
 * x, y, dy, dx: rows x D (D = 64), dtype ALGX_BF16 or ALGX_F32; gain, dgain: D
 * float32. */
int32_t algx_qknorm_fwd(const void* x, const float* gain, void* y, int64_t rows, int32_t D,
                        int32_t dtype, float eps, void* stream);
int64_t algx_qknorm_bwd_workspace_bytes(int64_t rows, int32_t D, int32_t dtype);
int32_t algx_qknorm_bwd(const void* x, const float* gain, const void* dy, void* dx, float* dgain,
                        void* workspace, int64_t rows, int32_t D, int32_t dtype, float eps,
                        void* stream);
/* The same for the attention's q and k in one launch each way (the reference
 * calls qk_rms_norm once per tensor, qk_norm.py:62-76): q and k have `rows`
 * rows each and their own gains; the results equal two single-tensor calls
 * bit for bit. */
int32_t algx_qknorm_pair_fwd(const void* xq, const void* xk, const float* gain_q,
                             const float* gain_k, void* yq, void* yk, int64_t rows, int32_t D,
                             int32_t dtype, float eps, void* stream);
int64_t algx_qknorm_pair_bwd_workspace_bytes(int64_t rows, int32_t D, int32_t dtype);
int32_t algx_qknorm_pair_bwd(const void* xq, const void* xk, const float* gain_q,
                             const float* gain_k, const void* dyq, const void* dyk, void* dxq,
                             void* dxk, float* dgain_q, float* dgain_k, void* workspace,
                             int64_t rows, int32_t D, int32_t dtype, float eps, void* stream);

/* -------------------------------------------------------------- attention
 * Replaces flash_attention's device work (src/algebraic/kernels/flash.py:763-857):
 * the range-guard reductions (:834-849), the forward kernels (_forward :292-326,
 * head_resident.forward head_resident.py:138-155) and the custom VJP
 * (_flash_bwd :718-726, _backward :630-687, head_resident.backward :158-176).
 *
 * q, q_s, k, v, o, dout, dq, dk, dv: (B, H, T, D) in `dtype`, contiguous and
 * 16-byte aligned, as are o_precise and the backward workspace (the kernels
 * move rows with 16-byte vector accesses; a misaligned pointer is rejected
 * with an error before any launch). sink: (H,)
 * float32 in kernel units (sink_logit / c), or NULL. stat: (B, H, T) float32.
 *
 * algx_attn_prepare forms the pre-scaled query q_s = cast(q * q_scale)
 * (flash.py:833) that the forward and backward consume. Given a guard buffer
 * (algx_attn_guard_words() int32 words) it also reduces max|q_s|^2, max|k|^2,
 * max|v| and |sink| (flash.py:841-849) in the same pass and sets guard[0] = 1
 * when in range. Passing that buffer to the forward/backward selects `low`
 * when guard[0] == 1 and `high` otherwise, on the device, without a host
 * round trip (flash.py:853-856). guard = NULL runs `low`. */
int32_t algx_attn_guard_words(void);
int32_t algx_attn_prepare(const void* q, const void* k, const void* v, const float* sink,
                          void* q_s, int32_t* guard, int32_t B, int32_t H, int32_t T, int32_t D,
                          int32_t dtype, float q_scale, float bound, float vmax, void* stream);

/* o_precise: float32 (B,H,T,D), written only by a variant with
 * precise_output (may be NULL when no such variant can run). */
int32_t algx_attn_fwd(const void* q_s, const void* k, const void* v, const float* sink,
                      void* o, float* o_precise, float* stat, int32_t B, int32_t H, int32_t T,
                      int32_t D, int32_t dtype, const algx_attn_variant* low,
                      const algx_attn_variant* high, const int32_t* guard, void* stream);

/* algx_attn_forward = algx_attn_prepare + algx_attn_fwd in one call
 * (flash.py:823-856 as one unit): the pre-scale, the guard and the forward.
 * For bf16, D = 64, T % 128 == 0 the forward kernel reads the raw q itself,
 * writes q_s (for the backward) and, with a guard buffer, one triple of
 * partial guard maxima per workgroup into `workspace`
 * (algx_attn_forward_workspace_bytes; may be NULL when guard is NULL). A
 * second launch reduces them to the guard word and, only when out of range,
 * recomputes the forward with `high`, completing lax.cond. Other shapes run
 * the two calls. bwd_workspace: NULL, or the algx_attn_bwd_workspace_bytes
 * buffer the backward of this call will receive; the forward prepares it in
 * passing so that algx_attn_bwd can take it as ALGX_ATTN_WS_CLEARED (the
 * reference's forward has no such output: it spares the backward a pass). */
int64_t algx_attn_forward_workspace_bytes(int32_t B, int32_t H, int32_t T, int32_t D);
int32_t algx_attn_forward(const void* q, const void* k, const void* v, const float* sink,
                          void* q_s, void* o, float* o_precise, float* stat, int32_t* guard,
                          void* workspace, void* bwd_workspace, int32_t B, int32_t H, int32_t T,
                          int32_t D, int32_t dtype, float q_scale, float bound, float vmax,
                          const algx_attn_variant* low, const algx_attn_variant* high,
                          void* stream);

/* No counterpart in the reference: algx_attn_forward for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). Same arguments and results, no workspace: the guard's partial
 * maxima live in a static per-device scratch array of the library (768 KiB,
 * held by each GPU the library runs on until the process ends), so
 * B * H * T / 128 may not exceed 65536 whenever a guard word is given (a
 * larger call returns an error before any other check or launch). Every call on one GPU shares that array: calls that
 * overlap on one GPU (concurrent streams) race. */
int32_t algx_attn_forward_noalloc(const void* q, const void* k, const void* v, const float* sink,
                                  void* q_s, void* o, float* o_precise, float* stat,
                                  int32_t* guard, void* bwd_workspace, int32_t B, int32_t H,
                                  int32_t T, int32_t D,
                                  int32_t dtype, float q_scale, float bound, float vmax,
                                  const algx_attn_variant* low, const algx_attn_variant* high,
                                  void* stream);

int64_t algx_attn_bwd_workspace_bytes(int32_t B, int32_t H, int32_t T, int32_t D);
/* dq is w.r.t. the unscaled q: dq = cast(cast(dq_s) * q_scale) as autodiff of
 * flash.py:833 gives; dsink (H,) float32 is w.r.t. the kernel-unit sink
 * (flash.py:721-723) and may be NULL when sink is NULL. workspace_state:
 * ALGX_ATTN_WS_RAW, or ALGX_ATTN_WS_CLEARED for a workspace the forward
 * prepared (see algx_attn_forward), whose dQ accumulator the backward then
 * does not clear again. */
int32_t algx_attn_bwd(const void* q_s, const void* k, const void* v, const float* sink,
                      const void* o, const float* o_precise, const float* stat, const void* dout,
                      void* dq, void* dk, void* dv, float* dsink, void* workspace,
                      int32_t workspace_state, int32_t B, int32_t H, int32_t T, int32_t D,
                      int32_t dtype, float q_scale, const algx_attn_variant* low,
                      const algx_attn_variant* high, const int32_t* guard, void* stream);

/* ------------------------------------------------------------ fused head
 * Replaces fused_head (src/algebraic/kernels/fused_head.py:260-275): forward
 * statistics (_forward :174-191: stat = logsumexp or Z^(-1/n), zt = target
 * logit) and the backward (_backward :194-216), without materialising the
 * (N, V) logits. h: (N, d) and E: (V, d) in `dtype` (the reference casts E to
 * h's dtype, :168); targets int32 (N,); stat, zt float32 (N,).
 * scale: device float32 scalar g * (1 or n/c) / N (fused_head.py:251).
 * dh: (N, d) in dtype; dE: (V, d) float32. bf16 hidden states (ALGX_BF16,
 * d % 8 == 0) run the MFMA kernels; float32 ones (ALGX_F32, any d) a float32
 * path with float32 logits and dz, as the reference computes for float32 h.
 * V is arbitrary (ragged tail masked). */
int64_t algx_head_fwd_workspace_bytes(int32_t N, int32_t d, int32_t V, int32_t dtype);
int32_t algx_head_fwd(const void* h, const void* E, const int32_t* targets, float* stat,
                      float* zt, void* workspace, int32_t N, int32_t d, int32_t V, int32_t kind,
                      int32_t n, float inv_c, float clamp, int32_t dtype, void* stream);
int64_t algx_head_bwd_workspace_bytes(int32_t N, int32_t d, int32_t V, int32_t dtype);
int32_t algx_head_bwd(const void* h, const void* E, const int32_t* targets, const float* stat,
                      const float* scale, void* dh, float* dE, void* workspace, int32_t N,
                      int32_t d, int32_t V, int32_t kind, int32_t n, float inv_c, float clamp,
                      int32_t dtype, void* stream);

/* ------------------------------------------------------ elementwise ops
 * rms_norm (src/algebraic/algebraic.py:76-83) over rows of D values:
 *   y = cast((x * rsqrt(mean(x^2) + eps)) * gain)
 * gain: D float32, or NULL for the parameter-free AVN (model.py:142).
 * x, y, dy, dx: rows x D in dtype, D a multiple of 8 (bf16) or 4 (f32), at most
 * 2048. The backward is the autodiff VJP of that expression; dgain (D float32)
 * is written exactly when gain is given, and then needs the workspace. */
int32_t algx_rms_norm_fwd(const void* x, const float* gain, void* y, int64_t rows, int32_t D,
                          int32_t dtype, float eps, void* stream);
int64_t algx_rms_norm_bwd_workspace_bytes(int64_t rows, int32_t D, int32_t dtype);
/* The block's residual add fused in front of the norm (model.py:177-178,
 * :191 then the next block's :166): xsum = cast(x + r), y = rms_norm(xsum).
 * Backward: dx = cast(cast(rms_norm VJP of dy) + dres), where dres is the
 * gradient reaching xsum along the residual stream; dx is the gradient of
 * both x and r. Same sizes, workspace and dgain rules as rms_norm. */
int32_t algx_add_rms_norm_fwd(const void* x, const void* r, const float* gain, void* xsum, void* y,
                              int64_t rows, int32_t D, int32_t dtype, float eps, void* stream);
int32_t algx_add_rms_norm_bwd(const void* xsum, const float* gain, const void* dy, const void* dres,
                              void* dx, float* dgain, void* workspace, int64_t rows, int32_t D,
                              int32_t dtype, float eps, void* stream);
int32_t algx_rms_norm_bwd(const void* x, const float* gain, const void* dy, void* dx,
                          float* dgain, void* workspace, int64_t rows, int32_t D, int32_t dtype,
                          float eps, void* stream);

/* alu (src/algebraic/algebraic.py:86-117), x/2 (1 + bx / sqrt(1 + b^2 x^2))
 * computed in float32 and rounded to dtype, with the reference's custom VJP
 * dx = cast(dy * ((1 + u)/2 + u r^2 / 2)), u = bx r, r = rsqrt(1 + (bx)^2).
 * n elements, a multiple of 8 (bf16) or 4 (f32). */
int32_t algx_alu_fwd(const void* x, void* y, int64_t n, int32_t dtype, float beta, void* stream);
int32_t algx_alu_bwd(const void* x, const void* dy, void* dx, int64_t n, int32_t dtype, float beta,
                     void* stream);
/* The alu_glu feed-forward product gate * alu(up) (src/algebraic/model.py:186-191)
 * in one pass, rounding as the unfused ops do: out = cast(gate * cast(alu(up))).
 * Backward: dgate = cast(dout * cast(alu(up))), dup = alu VJP of cast(dout * gate). */
int32_t algx_alu_glu_fwd(const void* gate, const void* up, void* out, int64_t n, int32_t dtype,
                         float beta, void* stream);
int32_t algx_alu_glu_bwd(const void* gate, const void* up, const void* dout, void* dgate,
                         void* dup, int64_t n, int32_t dtype, float beta, void* stream);

/* The feed-forward product on the packed projection gu = [gate | up]
 * (rows x 2 cols, the output of one GEMM against [w_g | w_u], model.py:184-191):
 * y (rows x cols) = cast(gate * act(up)) with act = ALGX_GLU_ALU (alu, beta, as
 * algx_alu_glu_fwd) or ALGX_GLU_SILU (x * cast(sigmoid(x)), standard.py:12-13).
 * The backward writes dgu = [dgate | dup] (rows x 2 cols). cols a multiple of 8
 * (bf16) or 4 (f32). */
enum { ALGX_GLU_ALU = 0, ALGX_GLU_SILU = 1 };
int32_t algx_glu_packed_fwd(const void* gu, void* y, int64_t rows, int32_t cols, int32_t act,
                            int32_t dtype, float beta, void* stream);
int32_t algx_glu_packed_bwd(const void* gu, const void* dy, void* dgu, int64_t rows, int32_t cols,
                            int32_t act, int32_t dtype, float beta, void* stream);

/* ------------------------------------------------------ attention prologue
 * The model block's step from projections to attention inputs
 * (src/algebraic/model.py:166-174) in one pass: q, k, v are rows of the
 * (B, T, *) projection output with row stride ld elements (they may point
 * into one fused (B, T, 3 H D) buffer); writes, in (B, H, T, D),
 *   q_out = rotate(cast(rms_norm(q, q_gain))), k_out likewise, v_out = v
 * where rms_norm is algebraic.py:76-83 and rotate the rotate-half product of
 * algebraic.py:172-179 with cos, sin: (T, D/2) float32 tables, rounded to
 * dtype after every product and sum as the reference's ops are. D = 64.
 * q_gain = k_gain = NULL skips the norm (qk_norm off); cos = sin = NULL skips
 * the rotation. The backward writes dq, dk, dv into projection-gradient rows
 * (stride ld) and, with gains, dq_gain and dk_gain (64 float32 each; needs
 * the workspace). */
int32_t algx_qk_prologue_fwd(const void* q, const void* k, const void* v, int64_t ld,
                             const float* q_gain, const float* k_gain, const float* cos_t,
                             const float* sin_t, void* q_out, void* k_out, void* v_out, int32_t B,
                             int32_t T, int32_t H, int32_t D, int32_t dtype, float eps,
                             void* stream);
int64_t algx_qk_prologue_bwd_workspace_bytes(int32_t B, int32_t T, int32_t H, int32_t D,
                                             int32_t dtype);
int32_t algx_qk_prologue_bwd(const void* q, const void* k, const float* q_gain, const float* k_gain,
                             const float* cos_t, const float* sin_t, const void* dq_out,
                             const void* dk_out, const void* dv_out, void* dq, void* dk, void* dv,
                             int64_t ld, float* dq_gain, float* dk_gain, void* workspace,
                             int32_t B, int32_t T, int32_t H, int32_t D, int32_t dtype, float eps,
                             void* stream);

/* ------------------------------------------------------------ layout moves
 * Byte moves of the model step that the reference leaves to XLA.
 * algx_swap_axes: dst (B, Q, P, row) = src (B, P, Q, row), rows of row_bytes
 * bytes (a positive multiple of 16) moved whole; src and dst 16-byte aligned,
 * not overlapping, fewer than 2^32 16-byte vectors. The attention output's
 * a.transpose(0, 2, 1, 3).reshape(B, T, d) (src/algebraic/model.py:182) and,
 * with P and Q exchanged, its gradient.
 * algx_transpose: dst [K][N][M] = src [K][M][N] for elements of elem_bytes
 * = 2 or 4 bytes, K <= 65535, not overlapping: the swapaxes(X, -2, -1) of the
 * Newton-Schulz iteration (src/algebraic/optimizers.py:41, :49, :58, :62). */
int32_t algx_swap_axes(const void* src, void* dst, int64_t B, int64_t P, int64_t Q,
                       int64_t row_bytes, void* stream);
int32_t algx_transpose(const void* src, void* dst, int64_t K, int64_t M, int64_t N,
                       int32_t elem_bytes, void* stream);
/* algx_concat_cast: joined [rows][sum cols] (bf16 or float32, dtype) from
 * nparts (1 to 4) float32 parts [rows][cols[i]], cols[i] positive multiples of
 * 4, parts 16-byte and joined 8- (bf16) or 16-byte (f32) aligned, none
 * overlapping. algx_split_cast: the inverse (the gradient of the parts). The
 * model's per-step compute-dtype copies of the stacked weights
 * (src/algebraic/model.py:167-169, :184-189 cast each weight per block) joined
 * for the fused [w_q | w_k | w_v] and [w_g | w_u] GEMMs. */
int32_t algx_concat_cast(void* const* parts, const int64_t* cols, int32_t nparts, void* joined,
                         int64_t rows, int32_t dtype, void* stream);
int32_t algx_split_cast(const void* joined, void* const* parts, const int64_t* cols,
                        int32_t nparts, int64_t rows, int32_t dtype, void* stream);

/* ------------------------------------------------------------- Muon steps
 * The elementwise parts of Muon's update (src/algebraic/optimizers.py:200-204)
 * over n float32 elements (pointers 16-byte aligned):
 * algx_muon_momentum: m <- mu m + (1 - mu) g; look = (1 - mu) g + mu m
 *   (:200-201), look being the matrix newton_schulz_5 orthogonalises (:202).
 * algx_muon_apply: p <- p * decay - step * o (:203-204), o the
 *   orthogonalised update in bf16 (8-byte aligned) or float32 (o_dtype),
 *   decay = 1 - lr * wd for decayed leaves (else 1), step = lr times the
 *   aspect factor sqrt(max(1, M / N)) of newton_schulz_5 (:63). */
int32_t algx_muon_momentum(const float* g, float* m, float* look, int64_t n, float mu,
                           void* stream);
int32_t algx_muon_apply(float* p, const void* o, int64_t n, int32_t o_dtype, float decay,
                        float step, void* stream);
/* algx_adamw_step: the Adam-family leaf update (optimizers.py:222-226) over n
 * float32 elements in place: m = b1 m + (1 - b1) g, v = b2 v + (1 - b2) g^2,
 * p = p * decay - lr * (m / c1) / (sqrt(v / c2) + eps), with c1, c2 the bias
 * corrections 1 - b^t and decay = 1 - lr * wd for decayed leaves (else 1). */
int32_t algx_adamw_step(float* p, const float* g, float* m, float* v, int64_t n, float b1,
                        float b2, float c1, float c2, float eps, float decay, float lr,
                        void* stream);
/* algx_ns_normalize: out[k] = cast(x[k] / sqrt(sum(x[k]^2) + eps)) for K float32
 * matrices of MN elements (newton_schulz_5's pre-normalisation,
 * src/algebraic/optimizers.py:44-45), out in bf16 or float32 (out_dtype),
 * K <= 65535; the workspace holds per-block partial sums (size from the query). */
int64_t algx_ns_normalize_workspace_bytes(int64_t K, int64_t MN);
int32_t algx_ns_normalize(const float* x, void* out, int64_t K, int64_t MN, int32_t out_dtype,
                          float eps, void* workspace, void* stream);
/* algx_gemm_bf16_batched: the products of newton_schulz_5's iteration
 * (src/algebraic/optimizers.py:46-60: A = X X^T, B = b A + c A A,
 * X <- a X + B X, and the refinements X <- 1.5 X - 0.5 (X X^T) X), as a
 * batched bf16 GEMM with the linear combination fused:
 *   C[i] = alpha * sum_k opA(m, k) opB(n, k) + beta * D[i]   (float32 sums)
 * over `batch` matrices (operand i at base + i * stride). opA(m, k) is
 * A[m*lda + k] when a_kc (k-contiguous) else A[k*lda + m]; opB(n, k)
 * likewise with ldb and b_kc. C and D (optional: null skips beta) are
 * row-major [M][N] with ldc / ldd; D may be C. bf16 throughout; M, N, K,
 * leading dimensions and strides multiples of 8, pointers 16-byte aligned.
 * symmetric != 0 states that C is symmetric (M == N; the product symmetric,
 * D symmetric when given), as X X^T and A A are: only the tiles on and above
 * the diagonal are formed and mirrored. */
int32_t algx_gemm_bf16_batched(const void* A, const void* B, const void* D, void* C,
                               int32_t batch, int32_t M, int32_t N, int32_t K, int32_t a_kc,
                               int32_t b_kc, int32_t symmetric, int64_t lda, int64_t ldb,
                               int64_t ldd, int64_t ldc, int64_t stride_a, int64_t stride_b,
                               int64_t stride_d,
                               int64_t stride_c, float alpha, float beta, void* stream);
/* algx_gemm_bf16_splitk: the weight gradients of the model's projections
 * (autodiff of `h @ w` at src/algebraic/model.py:166-191: dW = h^T dY, a
 * product whose K is the batch's token count while M x N is one weight):
 *   C[m][n] = cast_bf16(sum_k opA(m, k) opB(n, k))
 * with opA, opB as in algx_gemm_bf16_batched (a_kc / b_kc, lda / ldb), C
 * bf16 row-major with ldc. K is cut into `splits` equal chunks formed by
 * separate workgroups into float32 slices of the workspace
 * (algx_gemm_bf16_splitk_workspace_bytes(M, N, splits)), which a second
 * launch adds in chunk order and casts. M, N and K / splits multiples of 8,
 * leading dimensions multiples of 8, pointers 16-byte aligned,
 * 1 <= splits <= 1024. */
int64_t algx_gemm_bf16_splitk_workspace_bytes(int32_t M, int32_t N, int32_t splits);
int32_t algx_gemm_bf16_splitk(const void* A, const void* B, void* C, void* workspace, int32_t M,
                              int32_t N, int32_t K, int32_t a_kc, int32_t b_kc, int64_t lda,
                              int64_t ldb, int64_t ldc, int32_t splits, void* stream);
/* algx_gemm_bf16_grouped: up to 4 batches of algx_gemm_bf16_batched products
 * in one launch (the operands, sizes and strides of each group its own; the
 * operand layouts, symmetry and alpha/beta shared). Muon orthogonalises
 * matrices of several shapes at each step (newton_schulz_5,
 * src/algebraic/optimizers.py:27-65, called per Muon weight at :202): one
 * launch per product over all of them fills the
 * tail of each group's last round of workgroups with the others' tiles.
 * Results equal one algx_gemm_bf16_batched call per group, bit for bit
 * (groups whose K is not a multiple of 32 run in a second launch, on the
 * register-staged path their own call takes). */
typedef struct algx_gemm_batch {
  const void* A;
  const void* B;
  const void* D; /* may be null (no beta term) or equal to C */
  void* C;
  int32_t batch, M, N, K;
  int64_t lda, ldb, ldd, ldc;
  int64_t stride_a, stride_b, stride_d, stride_c;
} algx_gemm_batch;
int32_t algx_gemm_bf16_grouped(const algx_gemm_batch* groups, int32_t ngroups, int32_t a_kc,
                               int32_t b_kc, int32_t symmetric, float alpha, float beta,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ALGX_H */
