// Shared device/host helpers for the minitorch_amd HIP library (gfx950 only).
//
// Everything here is internal to libmtx_hip.so; the public C ABI is declared in
// include/mtx.h.  Status codes, the thread-local error string and the MFMA
// fragment helpers used by the attention, GEMM and row kernels live here.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

#include "../../include/mtx.h"

namespace mtx {

// ---------------------------------------------------------------------------
// error plumbing (host)
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define MTX_CHECK_ARG(cond, ...)                                  \
  do {                                                            \
    if (!(cond)) return ::mtx::fail(MTX_ERR_ARG, __VA_ARGS__);    \
  } while (0)
#define MTX_CHECK_SHAPE(cond, ...)                                \
  do {                                                            \
    if (!(cond)) return ::mtx::fail(MTX_ERR_SHAPE, __VA_ARGS__);  \
  } while (0)
// A failing runtime call also leaves its error as the thread's last error;
// it is reported here and cleared, so that the next launch check
// (MTX_LAUNCHED) does not take it for that launch's
#define MTX_HIP(expr)                                                           \
  do {                                                                          \
    hipError_t _e = (expr);                                                     \
    if (_e != hipSuccess) {                                                     \
      (void)hipGetLastError();                                                  \
      return ::mtx::fail(MTX_ERR_HIP, "%s: %s", #expr, hipGetErrorString(_e));  \
    }                                                                           \
  } while (0)
// check the launch that was just issued
#define MTX_LAUNCHED()                                                          \
  do {                                                                          \
    hipError_t _e = hipGetLastError();                                          \
    if (_e != hipSuccess)                                                       \
      return ::mtx::fail(MTX_ERR_HIP, "launch: %s", hipGetErrorString(_e));     \
  } while (0)

// ---------------------------------------------------------------------------
// GELU, tanh form with the reference's float32 constants
// (functional.py:54-59: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))));
// shared by the elementwise kernel and the GEMM epilogue so both compute the
// same expression
// ---------------------------------------------------------------------------
__device__ __forceinline__ float gelu_c0() { return 0.7978845834732056f; }  // float32(sqrt(2/pi))
__device__ __forceinline__ float gelu_c1() { return 0.044714998453855515f; }  // float32(0.044715)
__device__ __forceinline__ float gelu_tanh(float v) {
  const float inner = (v + v * v * v * gelu_c1()) * gelu_c0();
  return v * 0.5f * (tanhf(inner) + 1.0f);
}
// The same two functions with tanh(u) = 1 - 2 / (exp(2u) + 1) (one exp and
// one reciprocal instead of tanhf's range reduction: absolute error of tanh
// about 2e-7), for GEMM epilogues where tanhf's cost would stall the tile's
// stores.  exp overflowing to +inf gives tanh = 1, underflowing to 0 gives -1.
__device__ __forceinline__ float tanh_fast(float u) {
  return 1.0f - 2.0f * __frcp_rn(__expf(2.0f * u) + 1.0f);
}
__device__ __forceinline__ float gelu_tanh_fast(float v) {
  const float inner = (v + v * v * v * gelu_c1()) * gelu_c0();
  return v * 0.5f * (tanh_fast(inner) + 1.0f);
}
__device__ __forceinline__ float gelu_grad_fast(float v) {
  const float inner = (v + v * v * v * gelu_c1()) * gelu_c0();
  const float t = tanh_fast(inner);
  return 0.5f * (t + 1.0f) + 0.5f * v * (1.0f - t * t) * gelu_c0() * (1.0f + 3.0f * gelu_c1() * v * v);
}
// d gelu_tanh / dv: the product rule through 0.5 v (1 + tanh(u)),
// u = c0 (v + c1 v^3) (the reference's gelu backward, functional.py:54-59
// composed with tanh's, functional.py:39-51)
__device__ __forceinline__ float gelu_grad(float v) {
  const float inner = (v + v * v * v * gelu_c1()) * gelu_c0();
  const float t = tanhf(inner);
  return 0.5f * (t + 1.0f) + 0.5f * v * (1.0f - t * t) * gelu_c0() * (1.0f + 3.0f * gelu_c1() * v * v);
}

// ---------------------------------------------------------------------------
// wave64 reductions (butterfly over lane xor 32, 16, ..., 1: every lane gets
// the same bits)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// ---------------------------------------------------------------------------
// vector types
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint16_t bf16_t;  // storage type of bf16 in global memory

__device__ __forceinline__ float bf2f(bf16_t x) {
  return __uint_as_float(((uint32_t)x) << 16);
}
// round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ bf16_t f2bf(float x) {
  __bf16 b = (__bf16)x;
  return __builtin_bit_cast(bf16_t, b);
}

// ---------------------------------------------------------------------------
// element type traits: loads of 16-byte chunks, conversions
// ---------------------------------------------------------------------------
template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kVec = 4;  // elements per 16-byte chunk
  __device__ __forceinline__ static float to_f(float x) { return x; }
  __device__ __forceinline__ static float from_f(float x) { return x; }
};
template <> struct Elem<bf16_t> {
  static constexpr int kVec = 8;
  __device__ __forceinline__ static float to_f(bf16_t x) { return bf2f(x); }
  __device__ __forceinline__ static bf16_t from_f(float x) { return f2bf(x); }
};

// ---------------------------------------------------------------------------
// 16x16 MFMA family.  For every instruction used here lane l supplies
// A[row = l%16][k = kmap(l/16, e)] and B[k = kmap(l/16, e)][col = l%16] for its
// e = 0..KPL-1 operand elements, with the same k-map for A and B, and receives
// C[row = 4*(l/16) + r][col = l%16], r = 0..3.  Because the k-map is shared by
// both operands, the kernels only need to feed matching k-sets to A and B; the
// concrete k-map of the hardware never matters.
// ---------------------------------------------------------------------------
template <typename T> struct Mfma;
template <> struct Mfma<float> {
  static constexpr int KI = 4;   // k per instruction
  static constexpr int KPL = 1;  // operand elements per lane
  typedef float frag;
  __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<bf16_t> {
  static constexpr int KI = 32;
  static constexpr int KPL = 8;
  typedef bf16x8 frag;
  __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// XOR shuffles inside a wave64 (ds_bpermute based)
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// 32-bit LDS/global helpers --------------------------------------------------
__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  bf16x2 v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

inline int cdiv(int a, int b) { return (a + b - 1) / b; }

// LayerNorm statistics of one row held by a wave, lane-strided
// (v[i] = x[lane + 64 i], 0 past C): mean, then v[i] <- x - mean (0 past C)
// and sd = sqrt(biased variance + eps) (layers.py:82-86).
template <int VPL>
__device__ __forceinline__ void ln_stats(float (&v)[VPL], int lane, int C, float eps, float& mean, float& sd) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) s += v[i];
  mean = wave_sum(s) / (float)C;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int j = lane + 64 * i;
    const float d = j < C ? v[i] - mean : 0.f;
    v[i] = d;
    q += d * d;
  }
  const float var = wave_sum(q) / (float)C;
  sd = sqrtf(var + eps);
}
// normalised, scaled and shifted value of d = x - mean (layers.py:85-86)
__device__ __forceinline__ float ln_apply(float d, float sd, float gamma, float beta) {
  return (d / sd) * gamma + beta;
}

}  // namespace mtx
