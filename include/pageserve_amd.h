/*
 * pageserve_amd: C ABI of the MI355X (gfx950) INT8 weight-only linear path.
 *
 * Every entry point takes plain device pointers, element counts and an opaque
 * hipStream_t (passed as void*; NULL means the default stream).  All launches
 * are asynchronous on that stream; no entry point synchronises the host and
 * none allocates device memory.  Buffers are owned by the caller.
 *
 * Workspace (linear entry points): some shapes split the reduction over K
 * across workgroups and combine the partial results through a
 * caller-provided device buffer.  pgs_w8a16_workspace_bytes() gives the size
 * a call needs (0 = none).  The buffer must be 256-byte aligned and
 * zero-filled before its first use; every call leaves it valid for the next
 * one (its leading slots are left zeroed), so one buffer of the largest size
 * needed can serve all calls.  Calls that share a workspace must be ordered
 * (same stream, or synchronised); overlapping calls on one workspace race.
 * Passing NULL disables the split (always correct, slower for short-N shapes).
 * Under HIP graph capture a graph replays with the workspace it was captured
 * with: give each captured graph a workspace that it alone uses and zero it
 * inside the capture (a kernel fill, recorded in the graph), so that every
 * replay starts from empty slots whatever else used that memory meanwhile.
 *
 * Return value: PGS_OK (0) or one of the PGS_ERR_* codes below.  A call that
 * returns an error has launched nothing.  pgs_last_error() gives a
 * human-readable message for the calling thread's most recent failure.
 *
 * Layouts (no leading-dimension argument):
 *   weight w   [n, k]  fp32 or bf16   row-major (out_features, in_features)
 *   q          [n, k]  int8           row-major, per-output-row symmetric
 *                                     quantization (QuantizedWeight.q)
 *   qp         packed  int8           the same values in "MFMA tile" order,
 *                                     pgs_packed_bytes(n, k) bytes: 16-row x
 *                                     64-column blocks of 1 KiB, stored
 *                                     [ceil(n/16)][ceil(k/64)]; inside a block
 *                                     byte 16*l + b (l = 0..63, b = 0..15) is
 *                                     q[16*blk_row + l%16][64*blk_col +
 *                                     16*(l/16) + b]; padding is zero.  The
 *                                     linear entry points read weights only in
 *                                     this layout (one contiguous KiB per
 *                                     wavefront load).
 *   scale      [n]     fp32           (the reference stores it as [n, 1])
 *   x          [m, k]  bf16           row-major activations
 *   bias       [n]     bf16           optional (NULL = none)
 *   y          [m, n]  bf16 or fp32   row-major, y = x . (q * scale)^T + bias
 *
 * Reference interface (Rakshit-gen/pageserve, a Python package with no FFI):
 * each entry point below names the Python function or call site it replaces.
 */
#ifndef PAGESERVE_AMD_H
#define PAGESERVE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element type codes */
#define PGS_DTYPE_F32 0
#define PGS_DTYPE_BF16 1
#define PGS_DTYPE_F16 2

/* return codes */
#define PGS_OK 0
#define PGS_ERR_INVALID_ARGUMENT 1 /* bad size, null pointer, bad dtype code */
#define PGS_ERR_MISALIGNED 2       /* pointer not aligned to its element size */
#define PGS_ERR_LAUNCH 3           /* the HIP runtime rejected a kernel launch */
#define PGS_ERR_NO_DEVICE 4        /* no HIP device, or the stream's device is not a gfx950 */
#define PGS_ERR_TIMEOUT 5          /* a bounded device-side wait gave up (pgs_w8a16_decode_span_status) */

/* ABI version: bumped whenever a signature below changes. */
int pgs_abi_version(void);

/* Static string for a return code. */
const char* pgs_error_string(int code);

/* Detail of the calling thread's most recent failed call ("" if none). */
const char* pgs_last_error(void);

/*
 * Diagnostic, no counterpart in the reference: the kernel instance (with its
 * template arguments), grid size and K split of the calling thread's most
 * recent launch by a linear entry point ("" if none).  Lets tests and
 * profiles name the launch plan a shape takes.
 */
const char* pgs_last_plan(void);

/*
 * Whether `stream` is being captured into a HIP graph: *capturing = 1 and
 * *capture_id = the capture's id while a capture is active (2 if it was
 * invalidated), else 0 and 0.  No counterpart in the reference; hosts use it
 * to give each captured graph its own workspace (see the workspace notes
 * above).
 */
int pgs_stream_capture_state(void* stream, int* capturing, unsigned long long* capture_id);

/*
 * Replaces quantize_per_channel(weight) -- engine/quantization.py:16-23.
 *   absmax[r] = max(max_j |w[r,j]|, 1e-8f)
 *   scale[r]  = absmax[r] / 127.0f                 (IEEE fp32 division)
 *   q[r,j]    = clamp(rint(w[r,j] / scale[r]), -127, 127)   (ties to even)
 * Bit-exact with the reference's CPU arithmetic.  w_dtype: PGS_DTYPE_F32 or
 * PGS_DTYPE_BF16 (a bf16 weight widens exactly, as weight.float() does).
 * Non-finite weights follow the reference's CPU arithmetic: a row holding a
 * NaN gets a NaN scale (torch's amax and clamp keep NaN), a row holding an
 * infinity and no NaN gets an infinite scale, and every quotient that is NaN
 * (NaN / s, inf / inf, w / NaN) becomes q = 0, the value torch's CPU
 * conversion of NaN to int8 gives; finite / inf is 0.
 */
int pgs_quantize_per_channel(const void* w, int w_dtype, int64_t n, int64_t k,
                             int8_t* q, float* scale, void* stream);

/*
 * quantize_per_channel with the int8 result written in the packed layout
 * (same values as pgs_quantize_per_channel; padding zeroed).  This is how
 * QuantizedWeight(weight) stores its weight (engine/quantization.py:36-38).
 */
int pgs_quantize_per_channel_packed(const void* w, int w_dtype, int64_t n,
                                    int64_t k, int8_t* qp, float* scale,
                                    void* stream);

/* Bytes of the packed layout of an [n, k] int8 matrix (-1 for bad sizes). */
int64_t pgs_packed_bytes(int64_t n, int64_t k);

/*
 * Row-major q -> packed qp (padding written as zero), and back.  No
 * counterpart in the reference, which only has the row-major form
 * (QuantizedWeight.q, engine/quantization.py:38): unpack is how that form
 * is produced from the packed storage.
 */
int pgs_pack_weight(const int8_t* q, int64_t n, int64_t k, int8_t* qp,
                    void* stream);
int pgs_unpack_weight(const int8_t* qp, int64_t n, int64_t k, int8_t* q,
                      void* stream);

/*
 * Replaces dequantize(q, scale, dtype) -- engine/quantization.py:26-27.
 *   out[r,j] = dtype(float(q[r,j]) * scale[r])  (fp32 product, then one
 *   round-to-nearest-even conversion to out_dtype).  Bit-exact.
 * out_dtype: PGS_DTYPE_F32, PGS_DTYPE_BF16 or PGS_DTYPE_F16.
 */
int pgs_dequantize(const int8_t* q, const float* scale, int64_t n, int64_t k,
                   void* out, int out_dtype, void* stream);

/* dequantize from the packed layout; row-major [n, k] output, bit-exact. */
int pgs_dequantize_packed(const int8_t* qp, const float* scale, int64_t n,
                          int64_t k, void* out, int out_dtype, void* stream);

/*
 * Replaces F.linear(x, _resolve(W), b) for a QuantizedWeight W --
 * engine/model.py:25-26 (_resolve -> QuantizedWeight.get -> dequantize) feeding
 * the projections at engine/model.py:168-170 (q/k/v, with bias), :184 (o),
 * :188-190 (gate, up, down) and, with y_dtype = PGS_DTYPE_F32, the lm_head
 * at engine/model.py:193.
 *   y[i,r] = sum_j x[i,j] * q[r,j] * scale[r] (+ bias[r]),  fp32 accumulate,
 * with the weight given packed (qp).  The dense weight is never materialised.  y_dtype: PGS_DTYPE_BF16 or
 * PGS_DTYPE_F32.  Dispatches on m: the skinny kernel for m <= 32, the
 * MFMA tile kernel above.
 */
int pgs_w8a16_linear(const void* x, const int8_t* qp, const float* scale,
                     const void* bias, void* y, int y_dtype, int64_t m,
                     int64_t n, int64_t k, void* workspace,
                     size_t workspace_bytes, void* stream);

/*
 * pgs_w8a16_linear for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, launch plan
 * and results as pgs_w8a16_linear with a workspace, but the K-split scratch
 * (pair slots, partial tiles) is a fixed 64 MiB device array inside the
 * library, one per GPU, held until the process ends; the call allocates
 * nothing and frees nothing.  A shape whose plan needs more scratch than that
 * returns PGS_ERR_INVALID_ARGUMENT (every projection of a 2048-hidden /
 * 11008-intermediate model up to 2048 tokens needs at most 60.5 MiB).  Every
 * call on one GPU shares the array: calls that overlap on one GPU (other
 * streams, concurrently replayed graphs) race; stream-ordered calls do not.
 * The first call on a device must have that device current.
 */
int pgs_w8a16_linear_noalloc(const void* x, const int8_t* qp, const float* scale,
                             const void* bias, void* y, int y_dtype, int64_t m,
                             int64_t n, int64_t k, void* stream);

/*
 * Replaces x = residual + F.linear(h, _resolve(W)) -- engine/model.py:184
 * (o_proj) and :190 (down_proj) -- with one launch: the residual add runs in
 * the linear's epilogue, with the reference's roundings,
 *   y = bf16( residual + bf16( x . (q * scale)^T + bias ) )
 * (fp32 output: y = residual + x . (q * scale)^T + bias).  residual: bf16
 * [m, n]; y may be the residual buffer itself (in place).  Otherwise as
 * pgs_w8a16_linear.
 */
int pgs_w8a16_linear_residual(const void* x, const int8_t* qp, const float* scale,
                              const void* bias, const void* residual, void* y,
                              int y_dtype, int64_t m, int64_t n, int64_t k,
                              void* workspace, size_t workspace_bytes,
                              void* stream);

/*
 * Replaces rms_norm(x, weight, eps) -- engine/model.py:29-34, applied before
 * the q|k|v (engine/model.py:166) and gate|up (:187) projections -- with one
 * kernel:
 *   r = 1 / sqrt(mean_j x[i,j]^2 + eps)   (fp32)
 *   h[i,j] = bf16( weight[j] * bf16( x[i,j] * r ) )
 * x, weight, h: bf16 ([m, k], [k], [m, k]); h may not alias x.
 */
int pgs_rmsnorm(const void* x, const void* weight, float eps, void* h,
                int64_t m, int64_t k, void* stream);

/*
 * Replaces q = apply_rope(q, cos, sin); k = apply_rope(k, cos, sin) --
 * engine/model.py:53-56 (apply_rope, rotate_half at :37-39), applied at
 * :172-173 -- with one kernel for both tensors.  With h = head_dim / 2, per
 * (token, head) and i < h, the reference's bf16 op chain
 * x * cos + rotate_half(x) * sin with its roundings:
 *   out[i]     = bf16( bf16(x[i]     * cos[i])     + bf16(-x[i + h] * sin[i]) )
 *   out[i + h] = bf16( bf16(x[i + h] * cos[i + h]) + bf16( x[i]     * sin[i + h]) )
 * q, q_out: bf16 [m, q_heads, head_dim]; k, k_out: bf16 [m, k_heads, head_dim]
 * (k_heads = 0: q only); cos, sin: bf16 [m, head_dim], the rows of the
 * reference's cos_cache / sin_cache for the m tokens.  Outputs may alias
 * their inputs (in place).  head_dim even.
 */
int pgs_rope(const void* q, void* q_out, int64_t q_heads, const void* k, void* k_out,
             int64_t k_heads, const void* cos, const void* sin, int64_t m,
             int64_t head_dim, void* stream);

/*
 * One output of a grouped linear: several quantized weights that read the
 * same activations (the q/k/v triple of engine/model.py:168-170).
 */
typedef struct pgs_linear_out {
  const int8_t* qp;    /* [n, k] int8, packed layout */
  const float* scale;  /* [n] fp32 */
  const void* bias;    /* [n] bf16 or NULL */
  void* y;             /* [m, n] of y_dtype */
  int64_t n;           /* rows of this weight */
} pgs_linear_out;

#define PGS_MAX_GROUP 4

/*
 * Replaces the three F.linear calls of engine/model.py:168-170 (q, k, v
 * projections of the same normalised hidden state) with one launch.  Each
 * output is what pgs_w8a16_linear computes for it, up to the order of the
 * fp32 summation over K (the K split is planned for the whole group, so a
 * member may be split differently than on its own).
 * 1 <= n_outs <= PGS_MAX_GROUP.
 */
int pgs_w8a16_linear_group(const void* x, const pgs_linear_out* outs,
                           int n_outs, int y_dtype, int64_t m, int64_t k,
                           void* workspace, size_t workspace_bytes,
                           void* stream);

/*
 * Replaces gate = F.linear(h, Wg); up = F.linear(h, Wu); F.silu(gate) * up
 * -- engine/model.py:188-190 -- with one fused launch:
 *   act[i,r] = silu(g) * u,  g = sum_j x[i,j] q_gate[r,j] * s_gate[r],
 *                            u = sum_j x[i,j] q_up[r,j] * s_up[r]
 * (both weights packed)
 * computed in fp32 and rounded once to bf16.  act: bf16 [m, n].
 * The down projection is a separate pgs_w8a16_linear call on act.
 */
int pgs_w8a16_swiglu(const void* x, const int8_t* qp_gate, const float* s_gate,
                     const int8_t* qp_up, const float* s_up, void* act,
                     int64_t m, int64_t n, int64_t k, void* workspace,
                     size_t workspace_bytes, void* stream);

/*
 * Replaces h = rms_norm(x, weight, eps) followed by the q/k/v projections of
 * h -- engine/model.py:166 (rms_norm at :29-34) and :168-170 -- with one
 * launch where the plan allows (m <= 4 tokens, K % 64 == 0, no K split, bf16
 * outputs, 16-byte aligned norm weight): the kernel normalises the
 * activations it stages, with the reference's roundings
 * (h = bf16(weight * bf16(x * r)), r = 1/sqrt(mean(x^2) + eps) in fp32);
 * otherwise pgs_rmsnorm into the workspace, then pgs_w8a16_linear_group.
 * The fp32 sum of squares is formed in a fixed order (deterministic) that
 * differs from pgs_rmsnorm's, so h may differ from it in the last bf16 bit.
 * workspace: pgs_w8a16_rmsnorm_workspace_bytes() bytes.
 */
int pgs_w8a16_rmsnorm_linear_group(const void* x, const void* norm_weight, float eps,
                                   const pgs_linear_out* outs, int n_outs, int y_dtype,
                                   int64_t m, int64_t k, void* workspace,
                                   size_t workspace_bytes, void* stream);

/*
 * Replaces h = rms_norm(x, weight, eps); silu(F.linear(h, Wg)) * F.linear(h,
 * Wu) -- engine/model.py:187-189 -- with one launch where the plan allows
 * (same conditions and roundings as pgs_w8a16_rmsnorm_linear_group),
 * otherwise pgs_rmsnorm into the workspace, then pgs_w8a16_swiglu.
 */
int pgs_w8a16_rmsnorm_swiglu(const void* x, const void* norm_weight, float eps,
                             const int8_t* qp_gate, const float* s_gate,
                             const int8_t* qp_up, const float* s_up, void* act,
                             int64_t m, int64_t n, int64_t k, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * Workspace bytes a linear call needs (0 = none): n[0..n_outs-1] are the
 * out_features of its members (one member for pgs_w8a16_linear; for
 * pgs_w8a16_swiglu pass swiglu = 1 and n[0] = intermediate size).  The value
 * is exact for the same (m, n, k) and never larger than the plan needs.
 * No counterpart in the reference, whose dense F.linear needs no workspace.
 */
size_t pgs_w8a16_workspace_bytes(int64_t m, const int64_t* n, int n_outs,
                                 int64_t k, int swiglu);

/*
 * Workspace bytes of pgs_w8a16_rmsnorm_linear_group / pgs_w8a16_rmsnorm_swiglu
 * (same arguments as pgs_w8a16_workspace_bytes): always room for the
 * normalised activations ([m, k] bf16, used when the norm cannot run inside
 * the linear kernel) after the linear's own workspace and after the pair
 * slots at its start (kept empty for later calls sharing the workspace).  No
 * counterpart in the reference.
 */
size_t pgs_w8a16_rmsnorm_workspace_bytes(int64_t m, const int64_t* n, int n_outs,
                                         int64_t k, int swiglu);

/*
 * Replaces the greedy next token of server.py:51 (int(logits[-1].argmax()),
 * also app.py:87-93 and engine/runner.py:79) after the lm_head projection of
 * engine/model.py:193, without writing the logits: for each of the m rows of
 * x, idx[t] = argmax over r of y[t, r] = x[t] . (q[r] * scale[r]) (+ bias[r])
 * in fp32 -- torch.argmax's choice: the first index of the maximum, a NaN
 * counting as the maximum, -0.0 equal to +0.0 -- and, if vmax is not NULL,
 * vmax[t] = y[t, idx[t]] (bit-equal to pgs_w8a16_linear's fp32 output; a
 * canonical quiet NaN for a NaN maximum).  1 <= m <= 32 (pass only the rows
 * whose argmax is needed, e.g. the last prompt row).  idx: int64 [m];
 * vmax: fp32 [m].  workspace: pgs_w8a16_argmax_workspace_bytes(m, n, k)
 * bytes (per-workgroup partial maxima, fully rewritten by every call; no
 * zero-fill needed), 8-byte aligned.  Two launches (the projection with a
 * per-workgroup maximum in its epilogue, then one workgroup per row).
 */
int pgs_w8a16_linear_argmax(const void* x, const int8_t* qp, const float* scale,
                            const void* bias, int64_t* idx, float* vmax, int64_t m,
                            int64_t n, int64_t k, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Workspace bytes of pgs_w8a16_linear_argmax (0 for unsupported sizes). */
size_t pgs_w8a16_argmax_workspace_bytes(int64_t m, int64_t n, int64_t k);

/* One decoder layer's weights after its attention (engine/model.py:184-190). */
typedef struct pgs_span_weights {
  const int8_t* qp_o;    const float* s_o;     /* o_proj [hidden, hidden], packed */
  const void* ln_post;                         /* post_attention_layernorm weight, bf16 [hidden] */
  const int8_t* qp_gate; const float* s_gate;  /* gate_proj [inter, hidden] */
  const int8_t* qp_up;   const float* s_up;    /* up_proj [inter, hidden] */
  const int8_t* qp_down; const float* s_down;  /* down_proj [hidden, inter] */
} pgs_span_weights;

/* The next layer's part before its attention (engine/model.py:165-173). */
typedef struct pgs_span_next {
  const void* ln_in;                 /* input_layernorm weight, bf16 [hidden] */
  pgs_linear_out q, k, v;            /* q/k/v projections: weight, scale, bias (or NULL), output [m, n] bf16 */
  const void* cos; const void* sin;  /* bf16 [m, head_dim] rows of the RoPE tables (applied to q and k), or NULL */
  int64_t head_dim;
} pgs_span_next;

/*
 * Replaces everything one decode step runs between two attention calls --
 * engine/model.py:184-190 of layer l, then :165-173 of layer l + 1 -- with
 * one launch:
 *   x1 = residual + o_proj(attn)          (pgs_w8a16_linear_residual)
 *   h  = rms_norm(x1, ln_post, eps)       (pgs_rmsnorm)
 *   a  = silu(gate(h)) * up(h)            (pgs_w8a16_swiglu)
 *   x_out = x1 + down(a)                  (pgs_w8a16_linear_residual)
 *   h' = rms_norm(x_out, next->ln_in, eps)
 *   q, k, v = projections of h' (+ bias); RoPE of q and k with cos/sin
 * each with the rounding of the entry point named beside it (results equal
 * those of the chain of those entry points up to the order of the fp32 sums).
 * next = NULL: the last layer (no q/k/v).  The weights stream from HBM once,
 * in one persistent launch of one workgroup per CU whose stages meet through
 * tagged exchanges in the workspace, so the device must not run other work
 * meanwhile.  Compiled configurations: pgs_w8a16_decode_span_supported().
 * attn, residual, x_out: bf16 [m, hidden]; x_out may not alias residual.
 * workspace: pgs_w8a16_decode_span_workspace_bytes() bytes, 256-byte
 * aligned, zero-filled before its first use; calls sharing it must be
 * stream-ordered.  The waits inside the launch are bounded: a launch that
 * gives up (a workgroup that never ran, another kernel occupying CUs) leaves
 * an error word in the workspace and returns; later launches on that
 * workspace then do nothing until pgs_w8a16_decode_span_status() clears it.
 * No counterpart in the reference (its forward_step runs these as separate
 * torch calls).
 */
int pgs_w8a16_decode_span(const void* attn, const void* residual, void* x_out,
                          const pgs_span_weights* w, const pgs_span_next* next,
                          float eps, int64_t m, int64_t hidden, int64_t inter,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of pgs_w8a16_decode_span (0 for unsupported sizes). */
size_t pgs_w8a16_decode_span_workspace_bytes(int64_t m, int64_t hidden, int64_t inter);

/* 1 if pgs_w8a16_decode_span has a compiled configuration for these sizes. */
int pgs_w8a16_decode_span_supported(int64_t m, int64_t hidden, int64_t inter,
                                    int64_t nq, int64_t nkv, int64_t head_dim);

/*
 * Synchronises `stream` and reads the workspace's error word: PGS_OK, or
 * PGS_ERR_TIMEOUT if a launch gave up since the workspace was cleared; with
 * reset != 0 the workspace header and exchange buffers are then zero-filled
 * (a kernel on `stream`) so the next launch can run.
 */
int pgs_w8a16_decode_span_status(void* workspace, int reset, void* stream);

/*
 * Test hook, no counterpart in the reference: the number of polls after
 * which a decode span launch gives up (0 = the default), and force_giveup
 * != 0 makes every launch wait for a tag that no workgroup writes, so that
 * the give-up path runs.  Process-wide; affects later launches.
 */
int pgs_w8a16_decode_span_test_hooks(int spin_limit, int force_giveup);

/*
 * Tracing aid, no counterpart in the reference: with a device buffer set,
 * every later decode span launch writes per-workgroup stage timestamps
 * (s_memrealtime, a constant 100 MHz clock) into it, laid out
 * [slots][256 workgroups][16] uint64 with slots = bytes / 32768 (at most
 * 65535) and slot = launch tag % slots (the tag advances by one per launch
 * on a workspace).  Entries 0..12: launch start, end of the prologue, end of
 * o_proj's stream, o_proj's result published, x1 gathered (RMSNorm done),
 * end of gate|up's stream, activations published, activations gathered,
 * end of down_proj's stream, x2 published, x2 gathered (next RMSNorm done),
 * end of q|k|v's stream, end of the launch; 13..15: polls of the three
 * gathers (wave 0's).  NULL turns it off.  Process-wide; the buffer must outlive the
 * launches that write it, including every replay of a graph captured while
 * it was set (the launch holds its address).
 */
int pgs_w8a16_decode_span_trace(void* buffer, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* PAGESERVE_AMD_H */
