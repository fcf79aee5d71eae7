// Broadcasting elementwise kernels (fp32).
//
// Replaces the NumPy ufunc calls behind the reference's Tensor arithmetic
// (tensor.py:111-202: + - * / ** with broadcasting; tensor.py:391-415 exp and
// the clamped log) and the elementwise pieces of their backward closures.
// Operands are N-d strided views (stride 0 = broadcast); the output may be
// strided too, and `accumulate` adds into it (the reference's _accum_grad,
// tensor.py:29-33).  The host collapses dimensions first, so the common cases
// (contiguous, or a contiguous tensor against a broadcast row) run as 1-D or
// 2-D index arithmetic.
#include "mtx_common.h"

namespace mtx {
namespace {

constexpr int kMaxDim = 8;

struct EwArgs {
  int64_t shape[kMaxDim];
  int64_t sa[kMaxDim], sb[kMaxDim], so[kMaxDim];
  const float* a;
  const float* b;
  float* o;
  int64_t n;
  float alpha, beta;
  int ndim;
  int op;
  int accumulate;
};

__device__ __forceinline__ float apply(int op, float x, float y, float alpha, float beta) {
  switch (op) {
    case MTX_EW_COPY: return x;
    case MTX_EW_ADD: return x + y;
    case MTX_EW_SUB: return x - y;
    case MTX_EW_MUL: return x * y;
    case MTX_EW_DIV: return x / y;
    case MTX_EW_POW: return powf(x, y);
    case MTX_EW_AXPBY: return alpha * x + beta * y;
    case MTX_EW_SCALE_SHIFT: return alpha * x + beta;
    case MTX_EW_EXP: return expf(x);
    case MTX_EW_LOG: return logf(fmaxf(x, 1e-12f));
    case MTX_EW_TANH: return tanhf(x);
    case MTX_EW_NEG: return -x;
    case MTX_EW_RECIP_CLAMP: return 1.0f / fmaxf(x, 1e-12f);
    case MTX_EW_TANH_GRAD: return (1.0f - x * x) * y;
    case MTX_EW_SQUARE: return x * x;
    case MTX_EW_SQRT: return sqrtf(x);
    case MTX_EW_FILL: return alpha;
    case MTX_EW_MAXIMUM: return fmaxf(x, y);
    case MTX_EW_EQ: return x == y ? 1.0f : 0.0f;
    case MTX_EW_GT: return x > y ? 1.0f : 0.0f;
    case MTX_EW_ABS: return fabsf(x);
    case MTX_EW_SIGN: return (x > 0.f) ? 1.f : ((x < 0.f) ? -1.f : 0.f);
    default: return 0.f;
  }
}

__device__ __forceinline__ bool needs_b(int op) {
  return op == MTX_EW_ADD || op == MTX_EW_SUB || op == MTX_EW_MUL || op == MTX_EW_DIV ||
         op == MTX_EW_POW || op == MTX_EW_AXPBY || op == MTX_EW_TANH_GRAD || op == MTX_EW_MAXIMUM ||
         op == MTX_EW_EQ || op == MTX_EW_GT;
}

// general N-d path
__global__ __launch_bounds__(256) void ew_nd_kernel(const EwArgs g) {
  const bool hb = needs_b(g.op);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < g.n;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t rem = i, oa = 0, ob = 0, oo = 0;
#pragma unroll
    for (int d = kMaxDim - 1; d >= 0; --d) {
      if (d >= g.ndim) continue;
      const int64_t idx = rem % g.shape[d];
      rem /= g.shape[d];
      oa += idx * g.sa[d];
      ob += idx * g.sb[d];
      oo += idx * g.so[d];
    }
    const float x = g.op == MTX_EW_FILL ? 0.f : g.a[oa];
    const float y = hb ? g.b[ob] : 0.f;
    float r = apply(g.op, x, y, g.alpha, g.beta);
    if (g.accumulate) r += g.o[oo];
    g.o[oo] = r;
  }
}

// contiguous fast path: a, b (if used), o all contiguous with the same shape,
// or b a scalar (sb = 0)
__global__ __launch_bounds__(256) void ew_flat_kernel(const EwArgs g, int b_scalar) {
  const bool hb = needs_b(g.op);
  const int64_t n4 = g.n / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    f32x4 x = g.op == MTX_EW_FILL ? f32x4{0.f, 0.f, 0.f, 0.f} : reinterpret_cast<const f32x4*>(g.a)[i];
    f32x4 y = {0.f, 0.f, 0.f, 0.f};
    if (hb) {
      if (b_scalar) { const float s = g.b[0]; y = f32x4{s, s, s, s}; }
      else y = reinterpret_cast<const f32x4*>(g.b)[i];
    }
    f32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = apply(g.op, x[j], y[j], g.alpha, g.beta);
    if (g.accumulate) r += reinterpret_cast<const f32x4*>(g.o)[i];
    reinterpret_cast<f32x4*>(g.o)[i] = r;
  }
  for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < g.n; i += stride) {
    const float x = g.op == MTX_EW_FILL ? 0.f : g.a[i];
    const float y = hb ? (b_scalar ? g.b[0] : g.b[i]) : 0.f;
    float r = apply(g.op, x, y, g.alpha, g.beta);
    if (g.accumulate) r += g.o[i];
    g.o[i] = r;
  }
}

bool op_is_binary(int op) {
  return op == MTX_EW_ADD || op == MTX_EW_SUB || op == MTX_EW_MUL || op == MTX_EW_DIV ||
         op == MTX_EW_POW || op == MTX_EW_AXPBY || op == MTX_EW_TANH_GRAD || op == MTX_EW_MAXIMUM ||
         op == MTX_EW_EQ || op == MTX_EW_GT;
}

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" int mtx_ewise_f32(int op, int ndim, const int64_t* shape,
                             const float* a, const int64_t* a_strides,
                             const float* b, const int64_t* b_strides,
                             float* out, const int64_t* out_strides,
                             float alpha, float beta, int accumulate, void* stream) {
  MTX_CHECK_ARG(op >= 0 && op < MTX_EW_NUM_OPS, "ewise: unknown op %d", op);
  MTX_CHECK_SHAPE(ndim >= 0 && ndim <= kMaxDim, "ewise: ndim %d not in [0, %d]", ndim, kMaxDim);
  MTX_CHECK_ARG(out != nullptr && (ndim == 0 || (shape && out_strides)), "ewise: null output/shape");
  const bool bin = op_is_binary(op);
  MTX_CHECK_ARG(op == MTX_EW_FILL || (a != nullptr && (ndim == 0 || a_strides)), "ewise: null a");
  MTX_CHECK_ARG(!bin || (b != nullptr && (ndim == 0 || b_strides)), "ewise: op %d needs b", op);
  EwArgs g{};
  g.a = a; g.b = b; g.o = out; g.alpha = alpha; g.beta = beta; g.op = op;
  g.accumulate = accumulate ? 1 : 0;
  g.ndim = ndim;
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) {
    MTX_CHECK_SHAPE(shape[d] >= 0, "ewise: negative extent");
    g.shape[d] = shape[d];
    g.sa[d] = a_strides ? a_strides[d] : 0;
    g.sb[d] = (bin && b_strides) ? b_strides[d] : 0;
    g.so[d] = out_strides[d];
    n *= shape[d];
  }
  g.n = n;
  if (n == 0) return MTX_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // contiguous test
  bool oc = true, ac = true, bc = true, bs = bin;
  int64_t expect = 1;
  for (int d = ndim - 1; d >= 0; --d) {
    if (shape[d] != 1) {
      if (g.so[d] != expect) oc = false;
      if (g.sa[d] != expect) ac = false;
      if (bin && g.sb[d] != expect) bc = false;
      if (bin && g.sb[d] != 0) bs = false;
    }
    expect *= shape[d];
  }
  if (op == MTX_EW_FILL) ac = true;
  const bool aligned = (((uintptr_t)out | (uintptr_t)(op == MTX_EW_FILL ? nullptr : a) |
                         (uintptr_t)((bin && !bs) ? b : nullptr)) & 15u) == 0;
  const int blocks = (int)std::min<int64_t>((n + 1023) / 1024 + 1, 8192);
  if (oc && ac && (!bin || bc || bs) && aligned) {
    hipLaunchKernelGGL(ew_flat_kernel, dim3(blocks), dim3(256), 0, st, g, bs ? 1 : 0);
  } else {
    hipLaunchKernelGGL(ew_nd_kernel, dim3((int)std::min<int64_t>((n + 255) / 256, 16384)), dim3(256), 0,
                       st, g);
  }
  MTX_LAUNCHED();
  return MTX_OK;
}
