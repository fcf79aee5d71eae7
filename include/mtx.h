/*
 * mtx.h -- C ABI of libmtx_hip.so, the MI355X (gfx950) kernel library behind
 * minitorch_amd.
 *
 * The reference (samitmohan/minitorch) is pure Python/NumPy and has no foreign
 * function interface; every entry point below replaces a NumPy-level operation
 * on the causal-attention hot path.  Each declaration cites the reference code
 * it stands in for (paths relative to the reference repository root).  The
 * reference-side binding a maintainer would add is a ctypes stub;
 * minitorch_amd/_lib.py is that stub.
 *
 * Conventions
 *  - Every function returns an int status (MTX_OK = 0).  On failure
 *    mtx_last_error() returns a thread-local description.  Arguments are
 *    validated on the host before any HIP call, so invalid input never reaches
 *    a kernel.
 *  - Pointers are device pointers; strides are in elements.  Tensors of shape
 *    (B,H,T,D) take 4 strides {b,h,t,d}; the d stride must be 1.
 *  - `stream` is a hipStream_t (NULL = the null stream).  Calls are
 *    asynchronous with respect to the host.
 *  - Compute entry points allocate nothing: workspaces are sized by a
 *    *_workspace_bytes query and passed in by the caller.  Device memory may
 *    come from any allocator; the library's own caching allocator
 *    (mtx_malloc, with copies, streams, events and graphs, at the end of this
 *    header) lets a caller use the library with no other GPU framework.
 *  - dtype codes: MTX_F32 (fp32 in / fp32 compute) and MTX_BF16 (bf16 storage,
 *    fp32 accumulation).
 */
#ifndef MTX_H_
#define MTX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum mtx_status {
  MTX_OK = 0,
  MTX_ERR_ARG = 1,    /* null pointer, bad stride, bad flag */
  MTX_ERR_SHAPE = 2,  /* unsupported or inconsistent shape */
  MTX_ERR_DTYPE = 3,  /* unsupported dtype */
  MTX_ERR_HIP = 4     /* error reported by the HIP runtime */
};

enum mtx_dtype { MTX_F32 = 0, MTX_BF16 = 1 };

/* Thread-local description of the last failure on this thread. */
const char* mtx_last_error(void);

/* Library version string, and the gfx target the kernels were built for. */
const char* mtx_version(void);

/* ------------------------------------------------------------------------ */
/* Causal multi-head attention                                              */
/* ------------------------------------------------------------------------ */
/*
 * Fused attention forward.  Replaces transformer.py:36-44 of the reference:
 *   scores = (q @ k.transpose(-2,-1)) * scale      (tensor.py:207-208, 148-150)
 *   scores = scores + triu(ones(T,T),1) * -1e9      (tensor.py:111-113)
 *   attn   = F.softmax(scores, axis=-1)             (functional.py:62-66)
 *   out    = attn @ v                               (tensor.py:207-208)
 * computed flash-style with an online softmax; the (B,H,T,T) matrix never
 * exists.  Writes o (same dtype as q) and lse[b,h,i] = log sum_j exp(scale *
 * q_i.k_j) over visible keys, fp32, contiguous (B,H,Tq).
 * Causal rule: key j is visible to query i iff j <= i + (Tk - Tq); for Tq==Tk
 * this is exactly the reference's triu(k=1) mask (the -1e9 entries give exact
 * zeros in the reference, so skipping them is equivalent).
 * D must be one of 16, 32, 64, 128.  Tq, Tk >= 1, Tq <= Tk when causal.
 * The t (row) stride of every tensor must be < 2^24 elements.
 */
int mtx_attn_fwd(int dtype, int B, int H, int Tq, int Tk, int D,
                 const void* q, const int64_t* q_strides,
                 const void* k, const int64_t* k_strides,
                 const void* v, const int64_t* v_strides,
                 void* o, const int64_t* o_strides,
                 float* lse, float scale, int causal, void* stream);

/*
 * How fp32 attention (dtype MTX_F32, D = 64) computes its products,
 * process-wide, read at launch or graph recording: MTX_GEMM_BF16X3 (the
 * default) on the bf16 matrix cores with every fp32 operand value, P and dS
 * split into three bf16 pieces and the six piece products of weight >= 2^-16
 * accumulated in fp32 (as the GEMMs' mode of the same name); MTX_GEMM_FP32 on
 * fp32 MFMA.  Other head sizes and bf16 attention are not affected.  No reference
 * counterpart (the reference computes in NumPy float64 after the scale).
 */
int mtx_attn_set_mode(int mode);
int mtx_attn_get_mode(void);

/*
 * How mtx_attn_bwd (and the dropout-free mtx_attn_bwd_noalloc) computes the
 * gradient of bf16 attention with D <= 64: MTX_ATTN_BWD_TWOPASS (default;
 * deterministic: bit-identical on every run) or MTX_ATTN_BWD_ONEPASS (one
 * key-outer kernel with fp32 atomics for dQ; slower on MI355X).  Other
 * dtypes and head sizes always run two passes.  Returns MTX_OK or
 * MTX_ERR_ARG for an unknown mode.  Process-wide.  No reference counterpart (the reference runs the backward
 * as NumPy closures, tensor.py:210-218, functional.py:69-73).
 */
enum mtx_attn_bwd_modes { MTX_ATTN_BWD_TWOPASS = 0, MTX_ATTN_BWD_ONEPASS = 8 };
int mtx_attn_set_bwd_mode(int mode);
int mtx_attn_get_bwd_mode(void);

/* Bytes of workspace mtx_attn_bwd needs (the per-row delta = rowsum(dO*O)). */
size_t mtx_attn_bwd_workspace_bytes(int B, int H, int Tq);

/*
 * Fused attention backward.  Replaces the backward closures the reference runs
 * for the same sub-graph: matmul (tensor.py:210-218) twice, mul-by-scale
 * (tensor.py:152-156), the mask add (tensor.py:115-119) and softmax
 * (functional.py:69-73).  With P = exp(scale*QK^T - lse):
 *   dV = P^T dO;  dP = dO V^T;  dS = P*(dP - rowsum(dO*O));
 *   dQ = scale dS K;  dK = scale dS^T Q.
 * The reference's rowsum(P*dP) equals rowsum(dO*O) exactly in real arithmetic.
 * Gradients are fp32 for both dtypes.  accumulate != 0 adds into dq/dk/dv
 * (the reference's _accum_grad, tensor.py:29-33); 0 overwrites them.
 * Structure (mtx_attn_set_bwd_mode): by default two deterministic passes
 * (dQ query-outer, dK/dV key-outer, no atomics).  bf16 inputs with D <= 64
 * can instead run a one-pass backward (MTX_ATTN_BWD_ONEPASS: a delta kernel
 * that also zeroes dq, then one key-outer kernel that writes dK/dV and adds
 * dQ into dq with fp32 atomics; dQ's summation order over key blocks then
 * varies from run to run in the last bits).
 */
int mtx_attn_bwd(int dtype, int B, int H, int Tq, int Tk, int D,
                 const void* q, const int64_t* q_strides,
                 const void* k, const int64_t* k_strides,
                 const void* v, const int64_t* v_strides,
                 const void* o, const int64_t* o_strides,
                 const void* dout, const int64_t* do_strides,
                 const float* lse,
                 float* dq, const int64_t* dq_strides,
                 float* dk, const int64_t* dk_strides,
                 float* dv, const int64_t* dv_strides,
                 void* workspace, size_t workspace_bytes,
                 float scale, int causal, int accumulate, void* stream);

/*
 * mtx_attn_bwd without allocation: the same kernels and results (bit for bit
 * in two-pass mode; the one-pass mode's dQ differs from run to run in the
 * last bits, for both entry points alike), with the per-row delta held in a fixed device array the library owns
 * (MTX_ATTN_SCRATCH_BYTES per GPU, kept until the process ends) instead of a
 * caller workspace.  The caller passes inputs and outputs only; the call
 * allocates nothing (no hipMalloc, no library allocation).  B*H*Tq must be at
 * most MTX_ATTN_SCRATCH_BYTES / 4 rows (else MTX_ERR_SHAPE).  Calls that
 * overlap on one GPU (two streams, two threads) share the array and race.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, serving loops that forbid allocation).
 */
#define MTX_ATTN_SCRATCH_BYTES (8u << 20)
int mtx_attn_bwd_noalloc(int dtype, int B, int H, int Tq, int Tk, int D,
                         const void* q, const int64_t* q_strides,
                         const void* k, const int64_t* k_strides,
                         const void* v, const int64_t* v_strides,
                         const void* o, const int64_t* o_strides,
                         const void* dout, const int64_t* do_strides,
                         const float* lse,
                         float* dq, const int64_t* dq_strides,
                         float* dk, const int64_t* dk_strides,
                         float* dv, const int64_t* dv_strides,
                         float scale, int causal, int accumulate, void* stream);

/*
 * The passes of mtx_attn_bwd, selectable by a bit mask, so a caller can time
 * them separately.  Same arguments as mtx_attn_bwd.  DELTA writes
 * delta = rowsum(dO*O) to the workspace; DKDV and DQ read it.  When DELTA and
 * DQ are both selected they run as one kernel (the dQ pass computes delta for
 * its rows and stores it); selected passes run in the order DELTA, DQ, DKDV,
 * and DELTA|DQ|DKDV (= ALL) is mtx_attn_bwd, whose structure follows
 * mtx_attn_set_bwd_mode.  Adding the bit MTX_ATTN_BWD_ONEPASS (8) selects the
 * one-pass kernels explicitly (bf16, D <= 64, else MTX_ERR_SHAPE): DELTA then
 * computes delta and zeroes dq (unless accumulate), DQ|DKDV (together) writes
 * dK/dV and adds dQ into dq.  (No reference counterpart: the reference runs
 * this backward as the per-node closures listed at mtx_attn_bwd.)
 */
enum mtx_attn_bwd_phases {
  MTX_ATTN_BWD_DELTA = 1,
  MTX_ATTN_BWD_DKDV = 2,
  MTX_ATTN_BWD_DQ = 4,
  MTX_ATTN_BWD_ALL = 7
};
int mtx_attn_bwd_phase(int phases, int dtype, int B, int H, int Tq, int Tk, int D,
                       const void* q, const int64_t* q_strides,
                       const void* k, const int64_t* k_strides,
                       const void* v, const int64_t* v_strides,
                       const void* o, const int64_t* o_strides,
                       const void* dout, const int64_t* do_strides,
                       const float* lse,
                       float* dq, const int64_t* dq_strides,
                       float* dk, const int64_t* dk_strides,
                       float* dv, const int64_t* dv_strides,
                       void* workspace, size_t workspace_bytes,
                       float scale, int causal, int accumulate, void* stream);

/*
 * Attention with dropout on the softmax output: the reference's
 * MultiHeadAttention applies attn_drop (Dropout, layers.py:115-122) to
 * softmax(scores) before attn @ v (transformer.py:42-44), i.e.
 *   out = (P * keep * keep_scale) @ v,  keep_scale = 1/(1-p).
 * keep is a uint8 mask (nonzero = kept) laid out as (B, H, Tq, keep_ld):
 * element (b, h, i, j) at keep[((b*H + h)*Tq + i)*keep_ld + j]; keep_ld >= Tk,
 * keep_ld % 4 == 0, keep 4-byte aligned.  lse stays the log-sum-exp of the
 * undropped scores.  Other arguments as mtx_attn_fwd.
 */
int mtx_attn_fwd_dropout(int dtype, int B, int H, int Tq, int Tk, int D,
                         const void* q, const int64_t* q_strides,
                         const void* k, const int64_t* k_strides,
                         const void* v, const int64_t* v_strides,
                         void* o, const int64_t* o_strides,
                         float* lse, float scale, int causal,
                         const uint8_t* keep, int64_t keep_ld, float keep_scale,
                         void* stream);

/*
 * Backward of mtx_attn_fwd_dropout, with the same keep mask: the reference's
 * dropout closure (layers.py:124-126, grad * mask * scale) composed with the
 * closures listed at mtx_attn_bwd.  With Z = keep * keep_scale and
 * dP' = dO V^T:  dV = (P*Z)^T dO;  dS = P*(Z*dP' - rowsum(dO*O));  dQ, dK as
 * in mtx_attn_bwd (rowsum(P*Z*dP') = rowsum(dO*O) still holds).  Other
 * arguments as mtx_attn_bwd.
 */
int mtx_attn_bwd_dropout(int dtype, int B, int H, int Tq, int Tk, int D,
                         const void* q, const int64_t* q_strides,
                         const void* k, const int64_t* k_strides,
                         const void* v, const int64_t* v_strides,
                         const void* o, const int64_t* o_strides,
                         const void* dout, const int64_t* do_strides,
                         const float* lse,
                         float* dq, const int64_t* dq_strides,
                         float* dk, const int64_t* dk_strides,
                         float* dv, const int64_t* dv_strides,
                         void* workspace, size_t workspace_bytes,
                         float scale, int causal, int accumulate,
                         const uint8_t* keep, int64_t keep_ld, float keep_scale,
                         void* stream);

/*
 * Dropout keep-mask drawn on the device, replacing the host draw
 * np.random.rand(*shape) > p of Dropout.forward (layers.py:120) where the
 * mask feeds a fused kernel.  Philox4x32-10 keyed by seed; the 32-bit output
 * word (e % 4) of counter offset + e/4 gives element e (row-major index over
 * rows x cols) the uniform u = (word >> 8) * 2^-24, and keep = (u > p).
 * Element (i, j) is written to keep[i*ld + j]; bytes j >= cols of a row are
 * left untouched.  A later call with offset += ceil(rows*cols/4) draws fresh
 * numbers.  0 <= p < 1.
 */
int mtx_dropout_keep_philox(uint8_t* keep, int64_t rows, int cols, int64_t ld, float p,
                            uint64_t seed, uint64_t offset, void* stream);

/*
 * Packed q/k/v projection support.  MultiHeadAttention's q_proj, k_proj and
 * v_proj (transformer.py:32-34, three Linear(C, C) on the same input) run as
 * one GEMM over the concatenated (C_in, 3C) weight; the reference has no
 * packed layout (it runs three matmuls, tensor.py:207-223).
 * mtx_pack3_f32:   dst (rows, 3*cols) = [s0 | s1 | s2], each (rows, cols).
 * mtx_unpack3_f32: d_b (rows, cols) = src[:, b*cols:(b+1)*cols], added to d_b
 *                  when bit b of accumulate_mask is set (the reference's
 *                  _accum_grad, tensor.py:29-33).
 * All operands contiguous fp32.
 */
int mtx_pack3_f32(const float* s0, const float* s1, const float* s2, int64_t rows, int64_t cols,
                  float* dst, void* stream);
int mtx_unpack3_f32(const float* src, int64_t rows, int64_t cols, float* d0, float* d1, float* d2,
                    int accumulate_mask, void* stream);

/*
 * Decode-step attention: one query per (b, h) against its L cached keys,
 * o = softmax(scale * q k^T) v, lse = log sum_j exp(scale * q.k_j).  This is
 * the reference's attention sub-graph (transformer.py:36-44) at the last
 * position, which GPT.generate recomputes per token (transformer.py:93-104);
 * with a KV cache it is the whole attention work of a step.  q and o are
 * (B, H, 1, D), k and v (B, H, L, D) views (4 element strides each, the t
 * stride of q/o unused, unit d stride, so (B, T, C) caches pass as head views).
 * lengths: optional device int32[B]; sequence b then uses its first
 * min(lengths[b], L) keys (ragged batches; a length of 0 gives o = 0,
 * lse = -inf), so one call shape serves every step of a decode loop.
 * lse may be NULL.  0 <= L <= 8192; D in {16, 32, 64, 128}; fp32 or bf16.
 */
int mtx_attn_decode(int dtype, int B, int H, int L, int D,
                    const void* q, const int64_t* q_strides,
                    const void* k, const int64_t* k_strides,
                    const void* v, const int64_t* v_strides,
                    void* o, const int64_t* o_strides,
                    float* lse, const int* lengths, float scale, void* stream);

/*
 * A decode step's q/k/v projection and its attention in one launch (fp32):
 * for each sequence b and head h, [q | k | v] = x[b] @ W + bias restricted to
 * head h's D columns of each third (W the packed (C, 3C) projection, row
 * stride ldw; C = H*D; the C-long sums cut into 16 ranges, each k ascending
 * with fused multiply-adds, added in range order, then the bias), k and v
 * written to row lengths[b] - 1 of the caches kc / vc ((B, Tmax, C), row
 * stride cst, sequence stride csb; skipped unless 1 <= lengths[b] <= Tmax),
 * and o[b][hD .. hD+D) = softmax(scale q k^T) v over the first
 * min(lengths[b], Tmax) cache rows, the new row taken from the projection.
 * Replaces, in GPT.generate's per-token forward (transformer.py:93-104), the
 * q/k/v projections of MultiHeadAttention.forward (transformer.py:32-34,
 * layers.py:31-37) and its attention sub-graph (transformer.py:36-44) at the
 * last position: the pair mtx_gemm_step_f32 + mtx_attn_decode.  D in
 * {64, 128}, C <= 1024, 1 <= Tmax <= 2048; cache rows 16-byte aligned.
 * Input rows: with ln_gamma NULL, x holds the normalised rows (pws, x_out
 * NULL).  With ln_gamma set, x holds raw residual rows and the projection
 * reads LayerNorm(r) (gamma, ln_beta, eps: the block's ln1, layers.py:82-86)
 * where r = x[b] or, with pws, r = (sum_s pws[s][b] + pbias) + x[b]: the
 * pending second residual add of the previous block (x + mlp(ln2(x)),
 * transformer.py:65), pks partial products [pks][B][C] of
 * mtx_gemm_partials_f32 summed in s order, the arithmetic of
 * mtx_gemm_ln_f32's reduce; r is then written to x_out[b] (row stride ldxo,
 * not overlapping x) when x_out is set.
 */
int mtx_decode_qkv_attn_f32(int B, int H, int D, const float* x, int64_t ldx, const float* pws, int pks,
                            const float* pbias, float* x_out, int64_t ldxo, const float* ln_gamma,
                            const float* ln_beta, float eps, const float* W, int64_t ldw, const float* bias,
                            float* kc, float* vc, int64_t csb, int64_t cst, int Tmax, const int* lengths,
                            float scale, float* o, int64_t ldo, void* stream);

/*
 * Greedy pick over rows of x (rows, cols; row stride ld): idx[r * idx_stride]
 * = first index of the row maximum (np.argmax, the build's greedy harness over
 * the logits of transformer.py:97-98) and, if margin != NULL,
 * margin[r * margin_stride] = largest - second largest value (0 on ties).
 */
int mtx_argmax_f32(int rows, int cols, const float* x, int64_t ld, int64_t* idx, int64_t idx_stride,
                   float* margin, int64_t margin_stride, void* stream);

/*
 * KV-cache append for a decode step: cache[b, lengths[b] - 1, :] = x[b, :] for
 * b < B (C floats; rows with lengths[b] - 1 outside [0, T) are skipped), the
 * position read on the device.  Replaces, for cached decoding, the k/v
 * projections' recomputation over the whole context that GPT.generate does per
 * token (transformer.py:93-104 through transformer.py:33-35).
 */
int mtx_kv_append_f32(int B, int C, int T, const float* x, int64_t x_stride_b, float* cache,
                      int64_t cache_stride_b, int64_t cache_stride_t, const int* lengths, void* stream);

/*
 * End of a decode step: lengths[b] += 1 for b < B and, if pos != NULL,
 * pos[0] += 1 (the position index of the next token).  With mtx_kv_append_f32
 * and the lengths argument of mtx_attn_decode it lets a recorded step replay
 * unchanged for every token.  (No reference counterpart: the reference's loop
 * grows idx on the host, transformer.py:95-103.)
 */
int mtx_decode_advance(int B, int* lengths, int64_t* pos, void* stream);

/*
 * The greedy step's pick and bookkeeping in one launch.  Replaces, per
 * generated token, the harness's np.argmax of the last logits and the
 * np.concatenate of idx_next onto idx (transformer.py:97-103, argmax in place
 * of the sampling), plus mtx_decode_advance: for each row b of x (rows x
 * cols, row stride ld) the first-maximum index goes to cur[b] and to
 * ids[lengths[b] * rows + b] (a time-major (Tmax, rows) int64 buffer; rows
 * with lengths[b] outside [0, Tmax) skip it), the top-2 margin to
 * margins[(lengths[b] - t_base) * rows + b] when margins != NULL and that
 * row is in [0, n_margins); then lengths[b] += 1 and, if pos != NULL,
 * pos[0] += 1.  lengths holds `rows` entries.
 */
int mtx_greedy_pick_f32(int rows, int cols, const float* x, int64_t ld, int64_t* cur, int64_t* ids, int Tmax,
                        float* margins, int t_base, int n_margins, int* lengths, int64_t* pos, void* stream);

/*
 * out[i, :] = wa[ia[i], :] + wb[ib[i * ib_stride], :] for i < n: the token
 * and position embeddings and their sum, transformer.py:84-87 (Embedding
 * lookups, layers.py:102-104 / tensor.py:374-387, then Tensor.__add__,
 * tensor.py:111-113), in one pass.  ib_stride 0 broadcasts one position id
 * (a decode step).  Ids outside a table are clamped (the caller validates).
 */
int mtx_embedding2_fwd_f32(const float* wa, int64_t lda, int64_t Va, const int64_t* ia, const float* wb,
                           int64_t ldb, int64_t Vb, const int64_t* ib, int64_t ib_stride, float* out, int64_t ldo,
                           int64_t n, int C, void* stream);

/*
 * mtx_embedding2_fwd_f32 and then the first block's LayerNorm of its rows in
 * one launch: out[i] = wa[ia[i]] + wb[ib[i * ib_stride]] and
 * y[i] = (out[i] - mean) / sqrt(var + eps) * gamma + beta (biased variance
 * over the C values; the arithmetic of mtx_embedding2_fwd_f32 followed by
 * mtx_layernorm_fwd_f32).  Replaces, in GPT.generate's per-token forward,
 * transformer.py:84-87 (token + position embeddings) and the first block's
 * ln1 (transformer.py:63, layers.py:82-86).  C <= 2048.
 */
int mtx_embedding2_ln_fwd_f32(const float* wa, int64_t lda, int64_t Va, const int64_t* ia, const float* wb,
                              int64_t ldb, int64_t Vb, const int64_t* ib, int64_t ib_stride, float* out,
                              int64_t ldo, int64_t n, int C, const float* gamma, const float* beta, float eps,
                              float* y, int64_t ldy, void* stream);

/*
 * The output projection (lm_head) and mtx_greedy_pick_f32 of a decode step
 * in one launch: per row r of x (rows, K), logits[c] = sum_k x[r][k] *
 * W[k][c] + bias[c] (W (K, V) row stride ldw; K cut into 16 equal ranges,
 * each summed k ascending with fused multiply-adds, the range sums added in
 * range order, then the bias), then the first-maximum pick and its bookkeeping
 * exactly as mtx_greedy_pick_f32 (cur, ids, margins, lengths, pos).
 * Replaces, in the greedy harness over transformer.py:93-104, the head
 * Linear of transformer.py:91 (layers.py:31-37) and np.argmax of the last
 * position's logits.  V <= 256, K <= 8192.
 * With ln_gamma set, x holds raw rows: the row used is LayerNorm(r) (gamma,
 * ln_beta, eps; K <= 1024), r = x[row] or, with pws, the pending update of
 * mtx_decode_qkv_attn_f32, r = (sum_s pws[s][row] + pbias) + x[row] -- the
 * last block's second residual add and ln_f (transformer.py:65, 90).
 */
int mtx_head_pick_f32(int rows, int K, int V, const float* x, int64_t ldx, const float* pws, int pks,
                      const float* pbias, const float* ln_gamma, const float* ln_beta, float eps, const float* W,
                      int64_t ldw, const float* bias, int64_t* cur, int64_t* ids, int Tmax, float* margins,
                      int t_base, int n_margins, int* lengths, int64_t* pos, void* stream);

/*
 * `steps` consecutive greedy decode steps of a GPT in ONE launch (persistent,
 * cooperative; each step's pick feeds the next step inside the launch, past
 * one more grid-wide barrier): the token + position embeddings, every block (ln1, fused
 * q/k/v projection with the cache writes, decode attention, out_proj,
 * residual, ln2, fc1 + GELU, fc2, residual) and ln_f + lm_head + the pick
 * with its bookkeeping (as mtx_head_pick_f32: cur, ids, margins, lengths,
 * pos).  Replaces one iteration of GPT.generate's loop (transformer.py:93-104:
 * the forward of transformer.py:80-91 at the last position, then np.argmax)
 * for the KV-cache decode; the multi-launch chain of mtx_decode_qkv_attn_f32,
 * mtx_gemm_ln_f32, mtx_gemm_step_f32, mtx_gemm_partials_f32 and
 * mtx_head_pick_f32 computes the same step in 2 + 5 per block launches.
 *
 * Model (plain pointers, fp32, row-major and contiguous): C = n_head * 64
 * (head size 64) in {128, 256, 384, 512}, MLP width F = 4C (the block's
 * Linear(C, 4C), transformer.py:57-59), V <= 256, 1 <= n_layer <= 16, Tmax
 * <= 1024 cache rows, B >= 1; k_cache, v_cache and w_out 16-byte aligned.
 * Weights are (in, out): w_qkv (C, 3C) with columns q | k | v, b_qkv (3C);
 * w_out (C, C); w_fc1 (C, F); w_fc2 (F, C); w_head (C, V).  k_cache/v_cache
 * are (B, Tmax, C).  Row b's new token sits at row lengths[b] - 1 of its
 * caches and attends to rows [0, lengths[b]); the embedding reads token
 * cur[b] (clamped to n_tok) and position pos[0] (clamped to n_pos).
 *
 * Grid-wide ordering: the launch is cooperative (every workgroup resident,
 * or the launch fails), and the blocks' stages are separated by grid-wide
 * barriers (two per block) in device memory held in the workspace.  Every
 * barrier wait is bounded: a wait longer than wait_limit_us microseconds
 * (0: the default, 2 s; negative: every wait fails at once, for tests of the
 * failure path) sets an error word, every workgroup leaves the kernel, and
 * every later step on that workspace returns at its start.  Read it with
 * mtx_decode_step_status (which synchronises the stream);
 * mtx_decode_step_reset clears it.
 *
 * Workspace: mtx_decode_step_workspace_bytes(B, C, n_head, F) bytes of
 * device memory, 256-byte aligned, zeroed once before the first step (or by
 * mtx_decode_step_reset); it holds the barrier words, the residual rows and
 * the partial products between stages.  Steps that share a workspace must
 * not overlap (one stream); they may differ in model and batch size (each
 * launch counts its barriers from the base the launch before it left).
 * Deterministic: fixed summation orders.
 */
typedef struct mtx_decode_layer {
  const float* ln1_gamma;
  const float* ln1_beta;
  const float* w_qkv;
  const float* b_qkv;
  const float* w_out;
  const float* b_out;
  const float* ln2_gamma;
  const float* ln2_beta;
  const float* w_fc1;
  const float* b_fc1;
  const float* w_fc2;
  const float* b_fc2;
  float* k_cache;
  float* v_cache;
  float ln1_eps;
  float ln2_eps;
} mtx_decode_layer;

typedef struct mtx_decode_model {
  int n_layer, B, C, n_head, F, V, Tmax;
  const float* tok_emb;
  int64_t n_tok;
  const float* pos_emb;
  int64_t n_pos;
  const mtx_decode_layer* layers; /* host array of n_layer entries */
  const float* lnf_gamma;
  const float* lnf_beta;
  float lnf_eps;
  const float* w_head;
  const float* b_head;
} mtx_decode_model;

size_t mtx_decode_step_workspace_bytes(int B, int C, int n_head, int F);
int mtx_decode_step_f32(const mtx_decode_model* m, int steps, int64_t* cur, int64_t* ids, float* margins,
                        int t_base, int n_margins, int* lengths, int64_t* pos, void* workspace,
                        size_t workspace_bytes, int64_t wait_limit_us, void* stream);
/* MTX_OK, or MTX_ERR_HIP with a message when a step's barrier wait ran out. */
int mtx_decode_step_status(const void* workspace, void* stream);
int mtx_decode_step_reset(void* workspace, void* stream);

/* ------------------------------------------------------------------------ */
/* GEMM                                                                     */
/* ------------------------------------------------------------------------ */
/*
 * Strided-batched fp32 GEMM on MFMA: for b < batch,
 *   C[b] = alpha * A[b] @ B[b] + beta * C[b] + bias (bias[n], may be NULL).
 * A is M x K with element (m,k) at a + b*sa_b + m*sa_m + k*sa_k (sa_m or sa_k
 * must be 1); B is K x N likewise (sb_k or sb_n must be 1); C is M x N.  A
 * batch stride of 0 broadcasts that operand.  Replaces Tensor.__matmul__
 * (tensor.py:207-208) and its backward products (tensor.py:210-218, transposes
 * as stride swaps) and Linear.forward (layers.py:31-37, bias fused).  With a
 * workspace of mtx_gemm_workspace_bytes() bytes, long-K products are split
 * over K and reduced deterministically; without one they run unsplit.
 *
 * Products with M >= 128, N >= 128 and M*N*K*batch >= 2^27 run, by default
 * (MTX_GEMM_BF16X3), on the bf16 matrix cores -- unless they have fewer than
 * 256 tiles of 128 x 128 and K < 1024; those, like smaller products, take the
 * fp32 kernel -- with every fp32 operand value split into three bf16
 * pieces (x = x0 + x1 + x2 to 2^-24 |x|) and the six piece products of
 * weight >= 2^-16 accumulated in fp32: a dot product's error is the fp32
 * accumulation error plus at most ~2^-22 sum|a_k b_k|.  Non-finite inputs,
 * and finite ones of magnitude above bf16's largest value (~3.39e38, whose
 * high piece rounds to Inf), give NaN where fp32 arithmetic could give a
 * finite value or +-Inf.  MTX_GEMM_FP32 selects the fp32 MFMA kernel for
 * them instead.
 * The mode is process-wide and read when a product is launched (or
 * recorded into a graph); every entry point of this section follows it.
 */
enum mtx_gemm_mode { MTX_GEMM_FP32 = 0, MTX_GEMM_BF16X3 = 1 };
int mtx_gemm_set_mode(int mode);
int mtx_gemm_get_mode(void);
size_t mtx_gemm_workspace_bytes(int M, int N, int K, int batch);
int mtx_gemm_f32(int M, int N, int K, int batch,
                 float alpha, const float* a, int64_t sa_m, int64_t sa_k, int64_t sa_b,
                 const float* b, int64_t sb_k, int64_t sb_n, int64_t sb_b,
                 float beta, float* c, int64_t sc_m, int64_t sc_n, int64_t sc_b,
                 const float* bias, void* workspace, size_t workspace_bytes, void* stream);

/*
 * mtx_gemm_f32 with an activation epilogue, for Linear followed by GELU
 * (the MLP of TransformerBlock, transformer.py:56-58; F.gelu
 * functional.py:54-59) and its backward:
 *   act 0: as mtx_gemm_f32 (aux unused);
 *   act 1: C = gelu(V) with V = alpha*A@B + beta*C + bias; when aux is not
 *          NULL, V (the pre-activation the backward needs) is stored to aux;
 *   act 2: C = V * gelu'(aux), aux the pre-activation (the GELU closure's
 *          grad * gelu'(x) applied to the product that yields grad);
 *   act 4: C = V + aux, aux a residual stream other than C (the block's
 *          x + attn(...) and x + mlp(...), transformer.py:64-65, as the
 *          output projection's epilogue).
 * aux is M x N per batch with strides (sx_m, sx_n, sx_b).  gelu is the tanh
 * form with the reference's float32 constants.
 */
int mtx_gemm_act_f32(int M, int N, int K, int batch,
                     float alpha, const float* a, int64_t sa_m, int64_t sa_k, int64_t sa_b,
                     const float* b, int64_t sb_k, int64_t sb_n, int64_t sb_b,
                     float beta, float* c, int64_t sc_m, int64_t sc_n, int64_t sc_b,
                     const float* bias, int act, float* aux, int64_t sx_m, int64_t sx_n,
                     int64_t sx_b, void* workspace, size_t workspace_bytes, void* stream);

/*
 * A decode-step projection with its residual add, followed by the
 * LayerNorm that reads the updated rows next, in two launches:
 *   C = alpha * A @ B + bias + beta * C       (batch 1, C row stride sc_m,
 *                                              unit column stride)
 *   y[m] = (C[m] - mean) / sqrt(var + eps) * ln_gamma + ln_beta
 * (biased variance over the N values of row m; y row stride ldy; y must
 * not overlap C).  Replaces, in GPT.generate's per-token forward
 * (transformer.py:93-104), a block's residual adds x + attn(ln1(x)) and
 * x + mlp(ln2(x)) (transformer.py:64-65; the output projection and the
 * second MLP Linear, layers.py:31-37) together with the LayerNorm applied
 * to their result next (ln2, the following block's ln1, or ln_f:
 * transformer.py:63-65, 89; layers.py:82-86).  M <= 64, K <= 4096,
 * N <= 2048.  K is split into 2 to 8 ranges (one for K <= 16; enough workgroups for a
 * narrow N); their partial products go to the workspace
 * (mtx_gemm_ln_workspace_bytes) and one kernel sums them in range order,
 * applies bias and residual, and normalises the rows with the arithmetic
 * of mtx_layernorm_fwd_f32.  Deterministic; the product's rounding differs
 * from mtx_gemm_f32's only by the grouping of the K sums.
 */
size_t mtx_gemm_ln_workspace_bytes(int M, int N, int K);
int mtx_gemm_ln_f32(int M, int N, int K, float alpha, const float* a, int64_t sa_m, int64_t sa_k,
                    const float* b, int64_t sb_k, int64_t sb_n, float beta, float* c, int64_t sc_m,
                    const float* bias, const float* ln_gamma, const float* ln_beta, float eps, float* y,
                    int64_t ldy, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The first half of mtx_gemm_ln_f32 alone: the K ranges' partial products
 * P_s = A[:, range s] @ B[range s, :] (M x N each, row-major, P_s at
 * workspace + s*M*N floats; the ranges and their count *nsplit, set on the
 * host, are mtx_gemm_ln_f32's).  Sum_s P_s in s order equals the product that
 * mtx_gemm_ln_f32 reduces; a later launch that reads the rows anyway adds
 * them (mtx_decode_qkv_attn_f32, mtx_head_pick_f32), so a decode step's
 * second MLP product (layers.py:31-37 inside TransformerBlock.forward's
 * x + mlp(ln2(x)), transformer.py:64-65) needs no reduce launch of its own.
 * Same limits and workspace size as mtx_gemm_ln_f32.
 */
int mtx_gemm_partials_f32(int M, int N, int K, const float* a, int64_t sa_m, int64_t sa_k, const float* b,
                          int64_t sb_k, int64_t sb_n, void* workspace, size_t workspace_bytes, int* nsplit,
                          void* stream);

/*
 * Weight and bias gradients of a Linear layer in one pass over dY:
 *   C = A @ B + beta * C            (dW = X^T dY: tensor.py:216-218 through
 *                                    Linear.forward's x @ W, layers.py:31-37)
 *   dbias[n] = sum_k B[k][n]        (+ dbias[n] when dbias_accumulate; the
 *                                    add's _sum_to_shape of b, tensor.py:20-30,
 *                                    111-119)
 * batch 1; strides as mtx_gemm_f32.  The column sums come from the B values
 * the MFMA tiles already load; with split K they are reduced with the C
 * partials (workspace: mtx_gemm_workspace_bytes(M, N, K, 1)).
 */
int mtx_gemm_wgrad_f32(int M, int N, int K, const float* a, int64_t sa_m, int64_t sa_k,
                       const float* b, int64_t sb_k, int64_t sb_n, float beta, float* c, int64_t sc_m,
                       int64_t sc_n, float* dbias, int dbias_accumulate, void* workspace,
                       size_t workspace_bytes, void* stream);

/* One decode-step projection in a single launch (no workspace):
 *   P = A @ B + bias, A (M, K) row stride lda (unit k stride), B (K, N) row
 *   stride ldb (unit n stride), M <= 64 rows, K <= 512;
 *   columns [0, ncols_c) of P:  C = act(P + beta * C), act 0 = none,
 *                               1 = GELU (tanh form, functional.py:54-59);
 *   columns [ncols_c, N):       the first half to kcache, the second to
 *                               vcache, at row lengths[m] - 1 of sequence m
 *                               (rows outside [0, T) are skipped).
 * Replaces, in GPT.generate's per-token forward (transformer.py:93-104), the
 * fused q/k/v projection (transformer.py:32-34, layers.py:31-37) plus the
 * two cache writes, and Linear + GELU of the MLP (transformer.py:56-58).
 * MTX_ERR_SHAPE outside the size limits (callers then use mtx_gemm_f32,
 * mtx_kv_append_f32 and mtx_gelu_fwd_f32). */
int mtx_gemm_step_f32(int M, int N, int K, const float* a, int64_t lda, const float* b, int64_t ldb,
                      float beta, float* c, int64_t ldc, const float* bias, int act, int ncols_c,
                      float* kcache, float* vcache, int64_t cache_stride_b, int64_t cache_stride_t,
                      int T, const int* lengths, void* stream);

/* ------------------------------------------------------------------------ */
/* Elementwise and reductions                                               */
/* ------------------------------------------------------------------------ */
enum mtx_ew_op {
  MTX_EW_COPY = 0,         /* a                         (strided copy)        */
  MTX_EW_ADD = 1,          /* a + b                     tensor.py:113         */
  MTX_EW_SUB = 2,          /* a - b                     tensor.py:131         */
  MTX_EW_MUL = 3,          /* a * b                     tensor.py:150         */
  MTX_EW_DIV = 4,          /* a / b                     tensor.py:168         */
  MTX_EW_POW = 5,          /* a ** b                    tensor.py:188         */
  MTX_EW_AXPBY = 6,        /* alpha*a + beta*b                                */
  MTX_EW_SCALE_SHIFT = 7,  /* alpha*a + beta                                  */
  MTX_EW_EXP = 8,          /* exp(a)                    tensor.py:393         */
  MTX_EW_LOG = 9,          /* log(max(a, 1e-12))        tensor.py:405         */
  MTX_EW_TANH = 10,        /* tanh(a)                   functional.py:41      */
  MTX_EW_NEG = 11,         /* -a                                              */
  MTX_EW_RECIP_CLAMP = 12, /* 1/max(a, 1e-12)           tensor.py:410         */
  MTX_EW_TANH_GRAD = 13,   /* (1 - a*a) * b             functional.py:46      */
  MTX_EW_SQUARE = 14,      /* a*a                                             */
  MTX_EW_SQRT = 15,        /* sqrt(a)                                         */
  MTX_EW_FILL = 16,        /* alpha (a unused)                                */
  MTX_EW_MAXIMUM = 17,     /* max(a, b)                                       */
  MTX_EW_EQ = 18,          /* a == b ? 1 : 0            tensor.py:284         */
  MTX_EW_GT = 19,          /* a > b ? 1 : 0                                   */
  MTX_EW_ABS = 20,         /* |a|                       tensor.py:440         */
  MTX_EW_SIGN = 21,        /* sign(a)                   tensor.py:444         */
  MTX_EW_NUM_OPS = 22
};
/*
 * out = op(a, b) (+ out if accumulate) over an ndim <= 8 index space `shape`;
 * each operand has its own element strides (0 = broadcast).  Unary ops ignore
 * b.  The accumulate form is the reference's _accum_grad (tensor.py:29-33).
 */
int mtx_ewise_f32(int op, int ndim, const int64_t* shape,
                  const float* a, const int64_t* a_strides,
                  const float* b, const int64_t* b_strides,
                  float* out, const int64_t* out_strides,
                  float alpha, float beta, int accumulate, void* stream);

enum mtx_red_op { MTX_RED_SUM = 0, MTX_RED_MAX = 1 };
/*
 * out = alpha * reduce(a over the axes with reduce_mask[d] != 0) (+ out).
 * out is contiguous over the kept axes in order.  Replaces Tensor.sum / mean
 * (alpha = 1/count) / max (tensor.py:227-294) and _sum_to_shape
 * (tensor.py:20-26).  Deterministic; long reductions use the workspace.
 */
size_t mtx_reduce_workspace_bytes(int ndim, const int64_t* shape, const int* reduce_mask);
int mtx_reduce_f32(int op, int ndim, const int64_t* shape, const float* a, const int64_t* a_strides,
                   const int* reduce_mask, float* out, float alpha, int accumulate,
                   void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Row kernels (last axis contiguous; rows with a leading stride)           */
/* ------------------------------------------------------------------------ */
/*
 * Softmax (log_mode = 0, functional.py:62-66) or log_softmax (log_mode = 1,
 * functional.py:81-86) over rows of length L.  causal_tq > 0 treats the rows
 * as stacked (causal_tq, L) score matrices and hides column j of row i when
 * j > i + (L - causal_tq): the reference's triu(-1e9) mask (transformer.py:39-40)
 * with its exact-zero result.
 */
int mtx_softmax_fwd_f32(const float* x, int64_t ldx, float* y, int64_t ldy, int64_t rows, int L,
                        int causal_tq, int log_mode, void* stream);
/* Backward: softmax functional.py:69-73, log_softmax functional.py:88-92. */
int mtx_softmax_bwd_f32(const float* y, int64_t ldy, const float* dy, int64_t lddy, float* dx, int64_t lddx,
                        int64_t rows, int L, int log_mode, int accumulate, void* stream);

/* LayerNorm, layers.py:82-86 as one pass; saves per-row mean and std. C <= 2048. */
int mtx_layernorm_fwd_f32(const float* x, int64_t ldx, const float* gamma, const float* beta,
                          float* y, int64_t ldy, float* mean, float* std_, int64_t rows, int C,
                          float eps, void* stream);
size_t mtx_layernorm_bwd_workspace_bytes(int64_t rows, int C);
/* LayerNorm backward: dx (if non-NULL) and dgamma/dbeta (if non-NULL), in one
 * pass over x and dy when both are asked for.  accumulate: bit 0 adds into dx,
 * bit 1 adds into dgamma and dbeta.  addend (may be NULL; needs dx and bit 0
 * clear; row stride ldadd): dx = the LayerNorm gradient + addend, the other
 * contribution to x's gradient (the reference's _accum_grad, tensor.py:29-33,
 * for the residual stream that feeds both a LayerNorm and the block's residual
 * add, transformer.py:64-65) without first copying it into dx.  workspace: at
 * least mtx_layernorm_bwd_workspace_bytes(rows, C) when dgamma is given. */
int mtx_layernorm_bwd_f32(const float* x, int64_t ldx, const float* gamma, const float* mean,
                          const float* std_, const float* dy, int64_t lddy, float* dx, int64_t lddx,
                          const float* addend, int64_t ldadd, float* dgamma, float* dbeta, int64_t rows, int C,
                          int accumulate, void* workspace, size_t workspace_bytes, void* stream);

/* GELU (tanh form, functional.py:54-59), contiguous n elements. */
int mtx_gelu_fwd_f32(const float* x, float* y, int64_t n, void* stream);
int mtx_gelu_bwd_f32(const float* x, const float* dy, float* dx, int64_t n, int accumulate, void* stream);

/*
 * Softmax cross-entropy with integer labels (loss.py:17-27): per-row
 * row_loss = lse - logits[label] and lse.  Backward: dlogits = g * scale *
 * (softmax - onehot), g read from device memory (the upstream scalar grad).
 */
int mtx_xent_fwd_f32(const float* logits, int64_t ld, const int64_t* labels, float* row_loss,
                     float* lse, int64_t rows, int V, void* stream);
int mtx_xent_bwd_f32(const float* logits, int64_t ld, const int64_t* labels, const float* lse,
                     const float* gscalar, float scale, float* dlogits, int64_t ldd, int64_t rows, int V,
                     int accumulate, void* stream);

/* ------------------------------------------------------------------------ */
/* Embedding and optimizer                                                  */
/* ------------------------------------------------------------------------ */
/* out[i, :] = weight[idx[i], :]   (layers.py:102-104 -> tensor.py:374-375) */
int mtx_embedding_fwd_f32(const float* weight, int64_t ldw, int64_t V, const int64_t* idx, int64_t n,
                          float* out, int64_t ldo, int C, void* stream);
/* dweight[v, :] (+)= sum_{i: idx[i]==v} grad[i, :]  (np.add.at, tensor.py:382); deterministic */
int mtx_embedding_bwd_f32(const int64_t* idx, int64_t n, const float* grad, int64_t ldg, float* dweight,
                          int64_t lddw, int64_t V, int C, int accumulate, void* stream);

/*
 * One-hot rows: out[i, v] = (idx[i] == v) as float32, (n, V) row-major.  With
 * a GEMM, dweight = onehot^T @ grad is the embedding backward for small
 * vocabularies (np.add.at, tensor.py:382) on MFMA, deterministic.
 */
int mtx_onehot_f32(const int64_t* idx, int64_t n, int64_t V, float* out, void* stream);

/*
 * Adam over many tensors in one launch (optim.py:37-59).  `table` is a device
 * array of ntensors entries {float* p; const float* g; float* m; float* v;
 * int64_t n; int64_t block0}, block0 and total_blocks from mtx_adam_blocks
 * (host helper: each launch block covers 2048 elements of one tensor).
 * Tensors whose four pointers are 16-byte aligned are accessed as float4.
 */
int mtx_adam_blocks(const int64_t* sizes, int ntensors, int64_t* block0_out, int64_t* total_blocks);
int mtx_adam_f32(const void* table, int ntensors, int64_t total_blocks, double lr, double beta1,
                 double beta2, double eps, double weight_decay, int step, void* stream);

/*
 * The same update with the step count t in device memory (*step, int32: the
 * launch increments it, then updates with the new t), so a training step
 * recorded as a HIP graph replays unchanged.  The bias corrections are read
 * from bias_table (2 * table_len floats: entry (t - 1) % table_len holds
 * 1 - beta1^t, 1 - beta2^t, the float32 values mtx_adam_f32 computes),
 * filled on the host by mtx_adam_bias_table for the steps about to run.
 * (No counterpart in the reference, whose Adam keeps t on the host,
 * optim.py:43-59; for callers that replay recorded steps.)
 */
int mtx_adam_bias_table(double beta1, double beta2, int first_step, int len, float* out);
int mtx_adam_dev_f32(const void* table, int ntensors, int64_t total_blocks, double lr, double beta1,
                     double beta2, double eps, double weight_decay, int* step, const float* bias_table,
                     int table_len, void* stream);

/*
 * Zero the gradient of every tensor in an Adam table (the g field of each
 * entry, n floats) in one launch.  Replaces Optimizer.zero_grad
 * (optim.py:11-13) for callers that keep persistent gradient buffers so a
 * recorded step replays unchanged: the reference drops the gradients (sets
 * them to None); accumulating into zeros gives the same values.
 */
int mtx_zero_grads_f32(const void* table, int ntensors, int64_t total_blocks, void* stream);

/* ------------------------------------------------------------------------ */
/* Runtime: devices, memory, copies, streams, events, graphs                 */
/* ------------------------------------------------------------------------ */
/*
 * What the reference gets from NumPy (tensor.py:50-61: a Tensor owns its data
 * array; .data is read on the host) a caller of this library gets here, with
 * no other GPU framework: device memory it owns, copies to and from the host,
 * a stream to order work on, events to time it and HIP graphs to replay it.
 * The compute entry points above still take any device pointers.
 */
/* Number of visible GPUs (0, and MTX_OK, on a machine without one). */
int mtx_device_count(int* n);
/* Make `device` current for this thread and set up its per-device state. */
int mtx_device_init(int device);
/* Wait for all work on the current device. */
int mtx_device_sync(void);

/*
 * Caching allocator.  mtx_malloc returns device memory of at least `bytes`
 * (256-byte aligned); mtx_free gives it back to the library's cache, from
 * which later requests of about the same size are served without hipMalloc.
 * Reuse follows stream order: memory freed after the last work that uses it
 * was issued may be handed to the next request, so callers that use more than
 * one stream synchronise before freeing memory another stream still uses.
 * During a graph capture (mtx_graph_begin .. mtx_graph_end) freed blocks go
 * to that graph's private pool and are not handed out outside the graph while
 * it exists.  mtx_empty_cache synchronises the device and releases the
 * general pool's cached blocks; mtx_memory_stats reports bytes in use and
 * cached (either pointer may be NULL).
 */
int mtx_malloc(void** out, size_t bytes);
int mtx_free(void* p);
int mtx_empty_cache(void);
int mtx_memory_stats(size_t* in_use, size_t* cached);

/*
 * Copies.  h2d and d2h return when the copy is complete (they wait for the
 * stream, so earlier work on it is finished too); d2d is asynchronous.
 */
int mtx_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int mtx_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int mtx_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/*
 * Set `count` elements of `width` bytes (1, 2, 4 or 8; dst aligned to width)
 * to the low `width` bytes of `pattern`.  A kernel (not hipMemsetAsync), so it
 * may be recorded into a graph and replayed.
 */
int mtx_fill(void* dst, size_t count, uint64_t pattern, int width, void* stream);

/* Streams (default priority) and events. */
int mtx_stream_create(void** out);
int mtx_stream_destroy(void* stream);
int mtx_stream_sync(void* stream);
int mtx_event_create(void** out);
int mtx_event_destroy(void* event);
int mtx_event_record(void* event, void* stream);
/* Milliseconds between two recorded events (waits for `end`). */
int mtx_event_elapsed_ms(void* start, void* end, float* ms);
int mtx_stream_wait_event(void* stream, void* event);

/*
 * HIP graphs.  mtx_graph_begin starts recording the work issued on `stream`
 * (a created stream, not NULL); mtx_graph_end stops and instantiates it into
 * *graph.  mtx_graph_launch replays it on any stream; mtx_graph_destroy
 * releases it (after synchronising the device) and returns its memory pool
 * to the cache.  One capture at a time per process.
 */
int mtx_graph_begin(void* stream);
int mtx_graph_end(void* stream, void** graph);
int mtx_graph_launch(void* graph, void* stream);
int mtx_graph_destroy(void* graph);

#ifdef __cplusplus
}
#endif

#endif /* MTX_H_ */
