// Deterministic reductions (fp32).
//
// Replaces the NumPy reductions behind Tensor.sum / Tensor.mean / Tensor.max
// (tensor.py:227-294) and the broadcast-gradient reduction _sum_to_shape
// (tensor.py:20-26) used by every broadcasting backward closure (bias and
// LayerNorm-parameter gradients, the positional-embedding gradient).
//
// The host splits the input's dimensions into kept ("outer", the output) and
// reduced ones.  Each output element is reduced by one thread walking the
// reduced index space in a fixed order; when there are few outputs and many
// reduced elements the reduced range is split into S chunks whose partial
// results go to the caller's workspace and are combined in chunk order by a
// second kernel.  No atomics: results are bit-reproducible.
#include "mtx_common.h"

#include <algorithm>

namespace mtx {
namespace {

constexpr int kMaxD = 8;

struct RedArgs {
  int64_t kshape[kMaxD], kstr[kMaxD];  // kept dims of the input (row-major order)
  int64_t rshape[kMaxD], rstr[kMaxD];  // reduced dims
  int nk, nr;
  int64_t nout, nred, chunk;           // outputs, reduced count, reduced elements per split
  int nsplit;
  const float* a;
  float* out;     // contiguous over kept dims
  float* ws;      // [nsplit][nout] partials
  float alpha;
  int op;         // MTX_RED_SUM / MTX_RED_MAX
  int accumulate;
};

__device__ __forceinline__ int64_t kept_offset(const RedArgs& g, int64_t o) {
  int64_t off = 0;
#pragma unroll
  for (int d = kMaxD - 1; d >= 0; --d) {
    if (d >= g.nk) continue;
    off += (o % g.kshape[d]) * g.kstr[d];
    o /= g.kshape[d];
  }
  return off;
}

__device__ __forceinline__ int64_t red_offset(const RedArgs& g, int64_t r) {
  int64_t off = 0;
#pragma unroll
  for (int d = kMaxD - 1; d >= 0; --d) {
    if (d >= g.nr) continue;
    off += (r % g.rshape[d]) * g.rstr[d];
    r /= g.rshape[d];
  }
  return off;
}

// Block = 64 outputs (threadIdx.x) x 4 reduction lanes (threadIdx.y).  When
// the kept axes are innermost, the 64 outputs of a block are consecutive in
// memory, so every reduction step is a coalesced 256-byte read.
__global__ __launch_bounds__(256) void reduce_kernel(const RedArgs g) {
  __shared__ float part[4][64];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t o = (int64_t)blockIdx.x * 64 + tx;
  const int s = blockIdx.y;
  const bool is_max = g.op == MTX_RED_MAX;
  float acc = is_max ? -INFINITY : 0.f;
  if (o < g.nout) {
    const float* base = g.a + kept_offset(g, o);
    const int64_t r0 = (int64_t)s * g.chunk;
    const int64_t r1 = min(g.nred, r0 + g.chunk);
    if (g.nr == 1) {
      const int64_t st = g.rstr[0];
#pragma unroll 8
      for (int64_t r = r0 + ty; r < r1; r += 4) {
        const float v = base[r * st];
        acc = is_max ? fmaxf(acc, v) : acc + v;
      }
    } else {
      for (int64_t r = r0 + ty; r < r1; r += 4) {
        const float v = base[red_offset(g, r)];
        acc = is_max ? fmaxf(acc, v) : acc + v;
      }
    }
  }
  part[ty][tx] = acc;
  __syncthreads();
  if (ty != 0 || o >= g.nout) return;
  float t = part[0][tx];
#pragma unroll
  for (int j = 1; j < 4; ++j) t = is_max ? fmaxf(t, part[j][tx]) : t + part[j][tx];
  if (g.nsplit > 1) {
    g.ws[(int64_t)s * g.nout + o] = t;
  } else {
    float v = g.alpha * t;
    if (g.accumulate) v += g.out[o];
    g.out[o] = v;
  }
}

__global__ __launch_bounds__(256) void reduce_combine_kernel(const RedArgs g) {
  __shared__ float part[4][64];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t o = (int64_t)blockIdx.x * 64 + tx;
  const bool is_max = g.op == MTX_RED_MAX;
  float acc = is_max ? -INFINITY : 0.f;
  if (o < g.nout) {
#pragma unroll 8
    for (int s = ty; s < g.nsplit; s += 4) {
      const float v = g.ws[(int64_t)s * g.nout + o];
      acc = is_max ? fmaxf(acc, v) : acc + v;
    }
  }
  part[ty][tx] = acc;
  __syncthreads();
  if (ty != 0 || o >= g.nout) return;
  float t = part[0][tx];
#pragma unroll
  for (int j = 1; j < 4; ++j) t = is_max ? fmaxf(t, part[j][tx]) : t + part[j][tx];
  float v = g.alpha * t;
  if (g.accumulate) v += g.out[o];
  g.out[o] = v;
}

void merge_dims(int64_t* shp, int64_t* str, int& n) {
  int m = 0;
  for (int d = 0; d < n; ++d) {
    if (shp[d] == 1 && n > 1) continue;  // extent 1: contributes no offset
    if (m > 0 && str[m - 1] == str[d] * shp[d]) {
      shp[m - 1] *= shp[d];
      str[m - 1] = str[d];
    } else {
      shp[m] = shp[d];
      str[m] = str[d];
      ++m;
    }
  }
  if (m == 0) { shp[0] = 1; str[0] = 0; m = 1; }
  n = m;
}

int plan_splits(int64_t nout, int64_t nred) {
  // enough blocks (64 outputs each) to fill the GPU, >= 64 reduced elements per split
  const int64_t bx = (nout + 63) / 64;
  int64_t s = 1;
  while (bx * s < 1024 && nred / (s * 2) >= 64 && s < 512) s *= 2;
  return (int)s;
}

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" size_t mtx_reduce_workspace_bytes(int ndim, const int64_t* shape, const int* reduce_mask) {
  if (ndim < 0 || ndim > kMaxD || (ndim && (!shape || !reduce_mask))) return 0;
  int64_t nout = 1, nred = 1;
  for (int d = 0; d < ndim; ++d) (reduce_mask[d] ? nred : nout) *= shape[d];
  const int s = plan_splits(nout, nred);
  return s > 1 ? (size_t)s * nout * sizeof(float) : 0;
}

extern "C" int mtx_reduce_f32(int op, int ndim, const int64_t* shape, const float* a,
                              const int64_t* a_strides, const int* reduce_mask, float* out,
                              float alpha, int accumulate, void* workspace, size_t workspace_bytes,
                              void* stream) {
  MTX_CHECK_ARG(op == MTX_RED_SUM || op == MTX_RED_MAX, "reduce: unknown op %d", op);
  MTX_CHECK_SHAPE(ndim >= 0 && ndim <= kMaxD, "reduce: ndim %d not in [0, %d]", ndim, kMaxD);
  MTX_CHECK_ARG(a && out && (ndim == 0 || (shape && a_strides && reduce_mask)), "reduce: null argument");
  RedArgs g{};
  g.a = a; g.out = out; g.alpha = alpha; g.op = op; g.accumulate = accumulate ? 1 : 0;
  int64_t nout = 1, nred = 1;
  for (int d = 0; d < ndim; ++d) {
    MTX_CHECK_SHAPE(shape[d] >= 1, "reduce: extents must be >= 1");
    if (reduce_mask[d]) {
      g.rshape[g.nr] = shape[d]; g.rstr[g.nr] = a_strides[d]; ++g.nr; nred *= shape[d];
    } else {
      g.kshape[g.nk] = shape[d]; g.kstr[g.nk] = a_strides[d]; ++g.nk; nout *= shape[d];
    }
  }
  if (g.nr == 0) { g.rshape[0] = 1; g.rstr[0] = 0; g.nr = 1; }
  // merge neighbouring dims whose strides chain (stride[i] == stride[i+1] *
  // extent[i+1]): the row-major index order, and so the summation order, is
  // unchanged, and a contiguous (B, T, C) -> (C) reduction takes the
  // single-dim path without per-element index division
  merge_dims(g.rshape, g.rstr, g.nr);
  merge_dims(g.kshape, g.kstr, g.nk);
  g.nout = nout;
  g.nred = nred;
  int s = plan_splits(nout, nred);
  if (s > 1 && (!workspace || workspace_bytes < (size_t)s * nout * sizeof(float))) s = 1;
  g.nsplit = s;
  g.chunk = (nred + s - 1) / s;
  g.ws = static_cast<float*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int bx = (int)((nout + 63) / 64);
  MTX_CHECK_SHAPE((nout + 63) / 64 < (1 << 30), "reduce: too many outputs");
  hipLaunchKernelGGL(reduce_kernel, dim3(bx, s), dim3(256), 0, st, g);
  MTX_LAUNCHED();
  if (s > 1) {
    hipLaunchKernelGGL(reduce_combine_kernel, dim3(bx), dim3(256), 0, st, g);
    MTX_LAUNCHED();
  }
  return MTX_OK;
}
