/*
 * mtx.h -- C ABI of libmtx_hip.so, the MI355X (gfx950) kernel library behind
 * minitorch_amd.
 *
 * The reference (samitmohan/minitorch) is pure Python/NumPy and has no foreign
 * function interface; every entry point below replaces a NumPy-level operation
 * on the causal-attention hot path.  Each declaration cites the reference code
 * it stands in for (paths relative to the reference repository root).  The
 * reference-side binding a maintainer would add is a ctypes stub, shown in
 * INTEGRATION.md; minitorch_amd/_lib.py is that stub.
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
 *  - The library allocates nothing on its own: workspaces are sized by a
 *    *_workspace_bytes query and passed in by the caller.
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
 */
int mtx_attn_fwd(int dtype, int B, int H, int Tq, int Tk, int D,
                 const void* q, const int64_t* q_strides,
                 const void* k, const int64_t* k_strides,
                 const void* v, const int64_t* v_strides,
                 void* o, const int64_t* o_strides,
                 float* lse, float scale, int causal, void* stream);

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
 * Deterministic: no atomics (dK/dV and dQ come from two separate passes).
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
 * The three passes of mtx_attn_bwd, selectable by a bit mask, so a caller can
 * time them separately or run the dK/dV and dQ passes on two streams once the
 * delta pass has finished.  Same arguments as mtx_attn_bwd.  DELTA writes the
 * workspace; DKDV and DQ read it.  (No reference counterpart: the reference
 * runs this backward as the per-node closures listed at mtx_attn_bwd.)
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

#ifdef __cplusplus
}
#endif

#endif /* MTX_H_ */
