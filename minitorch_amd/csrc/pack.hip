// Column-block packing of three same-shape matrices.
//
// The q, k and v projections of MultiHeadAttention (transformer.py:32-34)
// are three Linear(C, C) layers applied to the same input.  They run here as
// one GEMM over the concatenated (C_in, 3C) weight, which needs the three
// weights (and biases) side by side, and the (C_in, 3C) weight gradient of
// that GEMM split back into the three layers' gradients.
#include "mtx_common.h"

namespace mtx {
namespace {

// dst (rows, 3*cols) <- [s0 | s1 | s2], each (rows, cols) contiguous
template <int V>
__global__ __launch_bounds__(256) void pack3_kernel(const float* __restrict__ s0, const float* __restrict__ s1,
                                                    const float* __restrict__ s2, int64_t rows, int64_t cols,
                                                    float* __restrict__ dst) {
  const int64_t per = cols / V;  // vectors per source row
  const int64_t n = rows * per * 3;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / (3 * per), rem = i - r * 3 * per;
    const int b = (int)(rem / per);
    const int64_t c = (rem - b * per) * V;
    const float* s = b == 0 ? s0 : (b == 1 ? s1 : s2);
    if constexpr (V == 4) {
      *reinterpret_cast<f32x4*>(dst + r * 3 * cols + b * cols + c) = *reinterpret_cast<const f32x4*>(s + r * cols + c);
    } else {
      dst[r * 3 * cols + b * cols + c] = s[r * cols + c];
    }
  }
}

// d_b (rows, cols) <- (acc_b ? d_b : 0) + src[:, b*cols : (b+1)*cols]
template <int V>
__global__ __launch_bounds__(256) void unpack3_kernel(const float* __restrict__ src, int64_t rows, int64_t cols,
                                                      float* __restrict__ d0, float* __restrict__ d1,
                                                      float* __restrict__ d2, int acc) {
  const int64_t per = cols / V;
  const int64_t n = rows * per * 3;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / (3 * per), rem = i - r * 3 * per;
    const int b = (int)(rem / per);
    const int64_t c = (rem - b * per) * V;
    float* d = b == 0 ? d0 : (b == 1 ? d1 : d2);
    const bool a = (acc >> b) & 1;
    if constexpr (V == 4) {
      f32x4 v = *reinterpret_cast<const f32x4*>(src + r * 3 * cols + b * cols + c);
      if (a) v += *reinterpret_cast<const f32x4*>(d + r * cols + c);
      *reinterpret_cast<f32x4*>(d + r * cols + c) = v;
    } else {
      float v = src[r * 3 * cols + b * cols + c];
      if (a) v += d[r * cols + c];
      d[r * cols + c] = v;
    }
  }
}

unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 4096); }

bool vec4_ok(int64_t cols, std::initializer_list<const void*> ps) {
  if (cols % 4) return false;
  for (const void* p : ps)
    if ((uintptr_t)p & 15u) return false;
  return true;
}

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" int mtx_pack3_f32(const float* s0, const float* s1, const float* s2, int64_t rows, int64_t cols,
                             float* dst, void* stream) {
  MTX_CHECK_ARG(rows >= 0 && cols >= 1, "rows=%lld, cols=%lld", (long long)rows, (long long)cols);
  if (rows == 0) return MTX_OK;
  MTX_CHECK_ARG(s0 && s1 && s2 && dst, "null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (vec4_ok(cols, {s0, s1, s2, dst}))
    hipLaunchKernelGGL(pack3_kernel<4>, dim3(grid_for(rows * cols * 3 / 4)), dim3(256), 0, st, s0, s1, s2, rows, cols, dst);
  else
    hipLaunchKernelGGL(pack3_kernel<1>, dim3(grid_for(rows * cols * 3)), dim3(256), 0, st, s0, s1, s2, rows, cols, dst);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_unpack3_f32(const float* src, int64_t rows, int64_t cols, float* d0, float* d1, float* d2,
                               int accumulate_mask, void* stream) {
  MTX_CHECK_ARG(rows >= 0 && cols >= 1, "rows=%lld, cols=%lld", (long long)rows, (long long)cols);
  MTX_CHECK_ARG((accumulate_mask & ~7) == 0, "accumulate_mask=%d must use bits 0..2", accumulate_mask);
  if (rows == 0) return MTX_OK;
  MTX_CHECK_ARG(src && d0 && d1 && d2, "null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (vec4_ok(cols, {src, d0, d1, d2}))
    hipLaunchKernelGGL(unpack3_kernel<4>, dim3(grid_for(rows * cols * 3 / 4)), dim3(256), 0, st, src, rows, cols, d0,
                       d1, d2, accumulate_mask);
  else
    hipLaunchKernelGGL(unpack3_kernel<1>, dim3(grid_for(rows * cols * 3)), dim3(256), 0, st, src, rows, cols, d0, d1,
                       d2, accumulate_mask);
  MTX_LAUNCHED();
  return MTX_OK;
}
