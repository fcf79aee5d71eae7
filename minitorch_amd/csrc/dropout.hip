// Dropout keep-masks drawn on the device from a counter-based generator.
//
// The reference draws its dropout masks on the host, `np.random.rand(*shape)
// > p` (layers.py:120).  A fused attention kernel cannot replay NumPy's
// stream, so the attention dropout here consumes an explicit uint8 keep-mask
// (mtx_attn_fwd_dropout / mtx_attn_bwd_dropout), which the caller either
// draws on the host exactly as the reference does or generates with this
// kernel: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC'11), keyed by a 64-bit seed, counter =
// offset + element/4, each 32-bit output w giving the uniform
// u = (w >> 8) * 2^-24 in [0, 1) of one element; the element is kept iff
// u > p, the reference's comparison.
#include "mtx_common.h"

namespace mtx {
namespace {

struct U4 {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ U4 philox4x32_10(U4 c, uint32_t k0, uint32_t k1) {
  constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;  // round multipliers
  constexpr uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;  // key increments (Weyl sequence)
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += kW0;
      k1 += kW1;
    }
    const uint32_t hi0 = __umulhi(kM0, c.x), lo0 = kM0 * c.x;
    const uint32_t hi1 = __umulhi(kM1, c.z), lo1 = kM1 * c.z;
    c = U4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
  }
  return c;
}

// one Philox call per 4 consecutive elements of the logical rows x cols
// array; element (i, j) is stored at keep[i * ld + j]
__global__ __launch_bounds__(256) void keep_philox_kernel(uint8_t* __restrict__ keep, int64_t rows, int cols,
                                                          int64_t ld, float p, uint32_t k0, uint32_t k1,
                                                          uint64_t offset) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n = rows * (int64_t)cols;
  const int64_t e0 = 4 * t;
  if (e0 >= n) return;
  const uint64_t ctr = offset + (uint64_t)t;
  const U4 r = philox4x32_10(U4{(uint32_t)ctr, (uint32_t)(ctr >> 32), 0u, 0u}, k0, k1);
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
  int64_t row = e0 / cols;
  int col = (int)(e0 - row * cols);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (e0 + i < n) {
      const float u = (float)(w[i] >> 8) * 0x1p-24f;
      keep[row * ld + col] = u > p ? 1 : 0;
      if (++col == cols) {
        col = 0;
        ++row;
      }
    }
  }
}

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" int mtx_dropout_keep_philox(uint8_t* keep, int64_t rows, int cols, int64_t ld, float p,
                                       uint64_t seed, uint64_t offset, void* stream) {
  MTX_CHECK_ARG(rows >= 0 && cols >= 1, "rows=%lld, cols=%d: need rows >= 0, cols >= 1", (long long)rows, cols);
  MTX_CHECK_ARG(ld >= cols, "ld=%lld must be >= cols=%d", (long long)ld, cols);
  MTX_CHECK_ARG(p >= 0.f && p < 1.f, "p=%g must be in [0, 1)", (double)p);
  if (rows == 0) return MTX_OK;
  MTX_CHECK_ARG(keep != nullptr, "keep: null pointer");
  const int64_t calls = (rows * (int64_t)cols + 3) / 4;
  MTX_CHECK_SHAPE(calls <= (int64_t)0x7fffffff * 256, "mask too large");
  const unsigned blocks = (unsigned)((calls + 255) / 256);
  hipLaunchKernelGGL(keep_philox_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), keep, rows,
                     cols, ld, p, (uint32_t)seed, (uint32_t)(seed >> 32), offset);
  MTX_LAUNCHED();
  return MTX_OK;
}
